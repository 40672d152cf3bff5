// Decode matvec in the reference's AVX2 f32 order for gfx950: y[r] =
// dot(W[r, :], x) over Q8_0 / Q4_K / Q6_K weights read in place from HBM,
// against a pre-quantized activation (Q8_0 or Q8_K). Restates the row loops
//   kernels.rs:36-70 (matvec_q8), kquant.rs:536-564 (matvec_q4k / matvec_q6k)
// with the per-row dot of dot_q8_avx2 (kernels.rs:263-286), dot_q4k_avx2
// (kquant.rs:260-305) and dot_q6k_avx2 (kquant.rs:454-510) bit for bit. (The
// scalar order's decode kernel is nrq_wstream.hip.)
//
// One workgroup owns `tr` consecutive rows. Those rows are one contiguous
// byte range of W; it is streamed HBM -> VGPR -> LDS with 16-byte loads
// (every lane's load is issued before any is consumed). Lane (row, k) then
// owns the k-th i32/f32 lane of the reference's __m256 accumulators (bytes
// 4k..4k+3 of every 32-byte vector), runs the fmadd chain over blocks, and the
// 8 lanes reduce in hsum256's order ((a0+a4)+(a2+a6))+((a1+a5)+(a3+a7)).
//
// The same staging and integer code also gives the exact per-(row, block)
// integer sums of the scalar kernels (block_sums_kernel, a diagnostic entry).
#include "nrq_device.h"
#include "nrq_launch.h"

namespace nrq {

template <int FMT>
struct Fmt;

template <>
struct Fmt<kQ8_0> {
  static constexpr int BS = kQ8_0Bytes;
  static constexpr int QK = 32;
  static constexpr int XB = kQ8_0Bytes;
  // x in LDS: xq[bpr*8] i32 (aligned qs dwords), xd[bpr] f32
  static __host__ __device__ int x_lds_bytes(int bpr) { return bpr * 8 * 4 + bpr * 4; }
};
template <>
struct Fmt<kQ4K> {
  static constexpr int BS = kQ4KBytes;
  static constexpr int QK = 256;
  static constexpr int XB = kQ8KBytes;
  // xq[bpr*64] i32, xd[bpr] f32, xbs[bpr*8] i32 (bsums[2j] + bsums[2j+1])
  static __host__ __device__ int x_lds_bytes(int bpr) { return bpr * 64 * 4 + bpr * 4 + bpr * 8 * 4; }
};
template <>
struct Fmt<kQ6K> {
  static constexpr int BS = kQ6KBytes;
  static constexpr int QK = 256;
  static constexpr int XB = kQ8KBytes;
  // xq[bpr*64] i32, xd[bpr] f32, xc[bpr*64] i32 (-32 * sum of the dword's 4 bytes)
  static __host__ __device__ int x_lds_bytes(int bpr) { return bpr * 64 * 4 + bpr * 4 + bpr * 64 * 4; }
};

// ---- staging: weights HBM -> VGPR -> LDS, activation L2 -> VGPR -> LDS --------

// Raw activation window in LDS: the aligned dwords around X.
template <int FMT>
__host__ __device__ constexpr int x_raw_bytes(int bpr) {
  return ((FMT == kQ8_0 ? bpr * kQ8_0Bytes : bpr * kQ8KBytes) + 8 + 15) & ~15;
}

// Issues every 16-byte weight load and every activation dword load of this
// lane before the first LDS store, so a lane keeps MAXC + MAXX requests in
// flight; then stores both. Activation dwords beyond NT*MAXX (very wide rows
// only) are copied by a plain loop.
template <int NT, int MAXC, int MAXX>
__device__ __forceinline__ void stage_tile_and_x(const u32x4* __restrict__ wsrc, int n16, u32x4* wdst,
                                                 const uint32_t* __restrict__ xsrc, int nx, uint32_t* xdst) {
  const int tid = threadIdx.x;
  u32x4 v[MAXC];
  uint32_t xv[MAXX];
#pragma unroll
  for (int c = 0; c < MAXC; c++) {
    int i = tid + c * NT;
    if (i < n16) v[c] = __builtin_nontemporal_load(wsrc + i);
  }
#pragma unroll
  for (int c = 0; c < MAXX; c++) {
    int i = tid + c * NT;
    if (i < nx) xv[c] = xsrc[i];
  }
#pragma unroll
  for (int c = 0; c < MAXC; c++) {
    int i = tid + c * NT;
    if (i < n16) wdst[i] = v[c];
  }
#pragma unroll
  for (int c = 0; c < MAXX; c++) {
    int i = tid + c * NT;
    if (i < nx) xdst[i] = xv[c];
  }
  for (int i = tid + MAXX * NT; i < nx; i += NT) xdst[i] = xsrc[i];
}

// Repacks the raw activation (LDS, starting xskew bytes into `raw`) into the
// layout the block code reads: aligned qs dwords, f32 scales, and per-format
// extras (Q4_K: bsums pair sums; Q6_K: -32 * byte sum of each qs dword).
template <int FMT, int NT>
__device__ void repack_x(const uint8_t* raw, uint32_t xskew, int bpr, uint8_t* lds) {
  const int tid = threadIdx.x;
  const uint32_t* raw32 = (const uint32_t*)raw;
  if constexpr (FMT == kQ8_0) {
    uint32_t* xq = (uint32_t*)lds;
    float* xd = (float*)(lds + bpr * 32);
    for (int i = tid; i < bpr * 8; i += NT) {
      int b = i >> 3, t = i & 7;
      uint32_t o = xskew + (uint32_t)b * kQ8_0Bytes;
      xq[i] = lds_u32_even(raw32, o + 2 + 4 * t);
      if (t == 0) xd[b] = f16_bits_to_f32(lds_u16(raw, o));
    }
  } else {
    // Q8_K blocks are 73 dwords: d @0, qs @1..64, bsums @65..72.
    uint32_t* xq = (uint32_t*)lds;
    float* xd = (float*)(lds + bpr * 256);
    int32_t* xe = (int32_t*)(lds + bpr * 260);
    for (int i = tid; i < bpr * 64; i += NT) {
      int b = i >> 6, t = i & 63;
      uint32_t v = raw32[b * 73 + 1 + t];
      xq[i] = v;
      if constexpr (FMT == kQ6K) xe[i] = sdot4(v, 0xe0e0e0e0u, 0);  // -32 * (sum of the 4 bytes)
      if (t == 0) xd[b] = __uint_as_float(raw32[b * 73]);
    }
    if constexpr (FMT == kQ4K) {
      for (int i = tid; i < bpr * 8; i += NT) {
        int b = i >> 3, j = i & 7;
        uint32_t v = raw32[b * 73 + 65 + j];  // bsums[2j] | bsums[2j+1] << 16
        xe[i] = (int32_t)(int16_t)(v & 0xffffu) + (int32_t)(int16_t)(v >> 16);
      }
    }
  }
}

// LDS layout of one workgroup: [repacked x | weight tile | raw activation].
template <int FMT>
struct TileGeom {
  int xrep, wtile, aux;
  __host__ __device__ TileGeom(int bpr, int tr) {
    xrep = (Fmt<FMT>::x_lds_bytes(bpr) + 15) & ~15;
    wtile = (int)(((size_t)tr * bpr * Fmt<FMT>::BS + 15 + 32 + 15) & ~(size_t)15);
    aux = x_raw_bytes<FMT>(bpr);
  }
  __host__ __device__ size_t total() const { return (size_t)xrep + wtile + aux; }
};

// Prologue shared by the kernels: stage rows [row0, row0+nr) of W and the
// activation, repack the activation. Returns the tile's byte skew.
template <int FMT, int NT, int MAXC, int MAXX>
__device__ __forceinline__ uint32_t stage_all(const uint8_t* __restrict__ W, const uint8_t* __restrict__ X, int bpr,
                                              int row0, int nr, const TileGeom<FMT>& G, uint8_t* smem) {
  using F = Fmt<FMT>;
  uint8_t* lds_x = smem;
  uint8_t* lds_w = smem + G.xrep;
  uint8_t* lds_aux = lds_w + G.wtile;
  const size_t rowbytes = (size_t)bpr * F::BS;
  // Rows are contiguous, so the tile is one byte range of W; W is 16-byte aligned.
  const size_t t0 = (size_t)row0 * rowbytes;
  const size_t t1 = t0 + (size_t)nr * rowbytes;
  const size_t a0 = t0 & ~(size_t)15;
  const int n16 = (int)((((t1 + 15) & ~(size_t)15) - a0) >> 4);
  const uintptr_t xa = (uintptr_t)X;
  const uint32_t xskew = (uint32_t)(xa & 3u);
  const int nx = (int)((xskew + (size_t)bpr * F::XB + 3) >> 2);
  stage_tile_and_x<NT, MAXC, MAXX>((const u32x4*)(W + a0), n16, (u32x4*)lds_w,
                                   (const uint32_t*)(xa - xskew), nx, (uint32_t*)lds_aux);
  __syncthreads();
  repack_x<FMT, NT>(lds_aux, xskew, bpr, lds_x);
  __syncthreads();
  return (uint32_t)(t0 - a0);
}

// ---- exact integer sums of one block (the scalar kernels' sub-dots) ---------------

// kernels.rs:75-78: acc = sum over the 32 quants of w*x (i32, exact)
__device__ __forceinline__ int block_q8_0_ints(const uint8_t* lds_w, uint32_t o, const uint32_t* xq, int b) {
  const uint32_t* w32 = (const uint32_t*)lds_w;
  uint32_t q0 = o + 2;
  uint32_t base = q0 >> 2, sh = q0 & 3u;
  uint32_t D[9];
#pragma unroll
  for (int t = 0; t < 9; t++) D[t] = w32[base + t];
  int acc = 0;
#pragma unroll
  for (int t = 0; t < 8; t++) acc = sdot4(__builtin_amdgcn_alignbyte(D[t + 1], D[t], sh), xq[b * 8 + t], acc);
  return acc;
}

// kquant.rs:200-214: sub_j = sum over sub-block j's 32 quants of q4*q8 (i32),
// sum_m = sum_j m_j * (bsums[2j] + bsums[2j+1]) (i32).
struct Q4KInts {
  int sub[8];
  int sc[8];
  int sum_m;
  uint32_t dd;  // d | dmin << 16 (f16 bits)
};

__device__ __forceinline__ void block_q4k_ints(const uint8_t* lds_w, uint32_t o, const uint32_t* xq,
                                               const int32_t* xbs, int b, Q4KInts& r) {
  const uint4 hdr = *(const uint4*)(lds_w + o);
  int mn[8];
  q4k_unpack_scales(hdr.y, hdr.z, hdr.w, r.sc, mn);
  const uint4* qs4 = (const uint4*)(lds_w + o + 16);
  const uint32_t* xb = xq + b * 64;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    uint4 qa = qs4[2 * c], qb = qs4[2 * c + 1];
    uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    int lo = 0, hi = 0;
#pragma unroll
    for (int t = 0; t < 8; t++) {
      lo = sdot4(q[t] & 0x0f0f0f0fu, xb[16 * c + t], lo);
      hi = sdot4((q[t] >> 4) & 0x0f0f0f0fu, xb[16 * c + 8 + t], hi);
    }
    r.sub[2 * c] = lo;
    r.sub[2 * c + 1] = hi;
  }
  int sum_m = 0;
#pragma unroll
  for (int j = 0; j < 8; j++) sum_m += mn[j] * xbs[b * 8 + j];
  r.sum_m = sum_m;
  r.dd = hdr.x;
}

// Reads the 210-byte Q6_K block at even LDS offset o as 53 realigned dwords.
__device__ __forceinline__ void load_q6k_block(const uint8_t* lds_w, uint32_t o, uint32_t v[53]) {
  const uint32_t* w32 = (const uint32_t*)lds_w;
  uint32_t base = o >> 2, sh = o & 3u;
  uint32_t prev = w32[base];
#pragma unroll
  for (int t = 0; t < 53; t++) {
    uint32_t next = w32[base + t + 1];
    v[t] = __builtin_amdgcn_alignbyte(next, prev, sh);
    prev = next;
  }
}

// kquant.rs:232-242: gs[8h + g] = sum over the group's 16 quants of (q-32)*q8
// (i32); the -32 term comes from the activation's own bytes (xc), not from
// its bsums, exactly as the scalar kernel never reads bsums here.
__device__ __forceinline__ void block_q6k_ints(const uint32_t v[53], const uint32_t* xq, const int32_t* xc, int b,
                                               int gs[16]) {
  const uint32_t* xb = xq + b * 64;
  const int32_t* cb = xc + b * 64;
#pragma unroll
  for (int g = 0; g < 16; g++) gs[g] = 0;
#pragma unroll
  for (int h = 0; h < 2; h++) {
#pragma unroll
    for (int t = 0; t < 8; t++) {
      uint32_t q6[4];
      q6k_planes(v[16 * h + t], v[16 * h + 8 + t], v[32 + 8 * h + t], q6);
#pragma unroll
      for (int n = 0; n < 4; n++) {
        int xi = 32 * h + 8 * n + t;
        int g = 8 * h + 2 * n + (t >> 2);
        gs[g] = sdot4(q6[n], xb[xi], gs[g] + cb[xi]);
      }
    }
  }
}

// ---- AVX2 order: lane (row, k) of the __m256 accumulators --------------------------

// kernels.rs:267-278: p32 lane k = sum of bytes 4k..4k+3 of w*x (exact for the
// [-127,127] activations q8::quantize produces); acc_k = fma(dw*dx, f32(p), acc_k)
__device__ __forceinline__ float lane_q8_0_avx2(const uint8_t* lds_w, uint32_t o_row, int bpr, int k,
                                                const uint32_t* xq, const float* xd) {
  const uint32_t* w32 = (const uint32_t*)lds_w;
  float acc = 0.0f;
  for (int b = 0; b < bpr; b++) {
    uint32_t o = o_row + (uint32_t)b * kQ8_0Bytes;
    uint32_t q = lds_u32_even(w32, o + 2 + 4 * k);
    int p = sdot4(q, xq[b * 8 + k], 0);
    float d = f16_bits_to_f32(lds_u16(lds_w, o)) * xd[b];
    acc = fmaf(d, (float)p, acc);
  }
  return acc;
}

// kquant.rs:267-303: sumi lane k = sum_j sc_j * (4-byte dot of sub-block j's
// bytes 4k..4k+3); acc_k = fma(d, f32(sumi), acc_k); acc_min += dmin*f32(min_sum)
__device__ __forceinline__ float lane_q4k_avx2(const uint8_t* lds_w, uint32_t o_row, int bpr, int k,
                                               const uint32_t* xq, const float* xd, const int32_t* xbs,
                                               float* acc_min_out) {
  float acc = 0.0f, acc_min = 0.0f;
  for (int b = 0; b < bpr; b++) {
    uint32_t o = o_row + (uint32_t)b * kQ4KBytes;
    const uint4 hdr = *(const uint4*)(lds_w + o);
    int sc[8], mn[8];
    q4k_unpack_scales(hdr.y, hdr.z, hdr.w, sc, mn);
    int min_sum = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) min_sum += mn[j] * xbs[b * 8 + j];
    const uint32_t* qs = (const uint32_t*)(lds_w + o + 16);
    const uint32_t* xb = xq + b * 64;
    int sumi = 0;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      uint32_t q = qs[8 * c + k];
      int lo = sdot4(q & 0x0f0f0f0fu, xb[16 * c + k], 0);
      int hi = sdot4((q >> 4) & 0x0f0f0f0fu, xb[16 * c + 8 + k], 0);
      sumi += sc[2 * c] * lo + sc[2 * c + 1] * hi;
    }
    float xdb = xd[b];
    float d = f16_bits_to_f32(hdr.x & 0xffffu) * xdb;
    float dmin = f16_bits_to_f32(hdr.x >> 16) * xdb;
    acc_min = acc_min + dmin * (float)min_sum;
    acc = fmaf(d, (float)sumi, acc);
  }
  *acc_min_out = acc_min;
  return acc;
}

// kquant.rs:462-508: sumi lane k = sum over (half, plane n) of
// sc[8h + 2n + k/4] * sum_{4 bytes} (q6-32)*q8; acc_k = fma(d, f32(sumi), acc_k)
__device__ __forceinline__ float lane_q6k_avx2(const uint8_t* lds_w, uint32_t o_row, int bpr, int k,
                                               const uint32_t* xq, const float* xd, const int32_t* xc) {
  const uint32_t* w32 = (const uint32_t*)lds_w;
  float acc = 0.0f;
  for (int b = 0; b < bpr; b++) {
    uint32_t o = o_row + (uint32_t)b * kQ6KBytes;
    const uint32_t* xb = xq + b * 64;
    const int32_t* cb = xc + b * 64;
    uint32_t scw[4];
#pragma unroll
    for (int i = 0; i < 4; i++) scw[i] = lds_u32_even(w32, o + 192 + 4 * i);
    int sumi = 0;
#pragma unroll
    for (int h = 0; h < 2; h++) {
      uint32_t qlA = lds_u32_even(w32, o + 64 * h + 4 * k);
      uint32_t qlB = lds_u32_even(w32, o + 64 * h + 32 + 4 * k);
      uint32_t qh = lds_u32_even(w32, o + 128 + 32 * h + 4 * k);
      uint32_t q6[4];
      q6k_planes(qlA, qlB, qh, q6);
#pragma unroll
      for (int n = 0; n < 4; n++) {
        int xi = 32 * h + 8 * n + k;
        int p = sdot4(q6[n], xb[xi], cb[xi]);
        int g = 8 * h + 2 * n + (k >> 2);
        int s = (int)(int8_t)((scw[g >> 2] >> (8 * (g & 3))) & 0xffu);
        sumi += s * p;
      }
    }
    float d = f16_bits_to_f32(lds_u16(lds_w, o + 208)) * xd[b];
    acc = fmaf(d, (float)sumi, acc);
  }
  return acc;
}

// ---- the kernels -------------------------------------------------------------------

constexpr int kMatvecNT = 256;
constexpr int kMatvecMaxC = 12;  // 16-byte weight loads per lane: a 48 KiB tile per workgroup
constexpr int kMatvecMaxX = 8;   // activation dwords per lane issued with the tile
constexpr size_t kLdsLimit = 65536;

template <int FMT, int NT, int MAXC, int MAXX>
__global__ __launch_bounds__(NT) void matvec_avx2_kernel(const uint8_t* __restrict__ W, const uint8_t* __restrict__ X,
                                                         float* __restrict__ Y, int rows, int bpr, int tr) {
  using F = Fmt<FMT>;
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x;
  const int row0 = blockIdx.x * tr;
  const int nr = min(tr, rows - row0);
  const TileGeom<FMT> G(bpr, tr);
  const uint32_t skew = stage_all<FMT, NT, MAXC, MAXX>(W, X, bpr, row0, nr, G, smem);
  const uint8_t* lds_x = smem;
  const uint8_t* lds_w = smem + G.xrep;
  const uint32_t* xq = (const uint32_t*)lds_x;
  const float* xd = (const float*)(lds_x + (FMT == kQ8_0 ? bpr * 32 : bpr * 256));
  const int32_t* xe = (const int32_t*)(lds_x + bpr * 260);

  const int rowbytes = bpr * F::BS;
  for (int li = tid; li < nr * 8; li += NT) {
    int r = li >> 3, k = li & 7;
    uint32_t o_row = skew + (uint32_t)(r * rowbytes);
    float acc, acc_min = 0.0f;
    if constexpr (FMT == kQ8_0) acc = lane_q8_0_avx2(lds_w, o_row, bpr, k, xq, xd);
    else if constexpr (FMT == kQ4K) acc = lane_q4k_avx2(lds_w, o_row, bpr, k, xq, xd, xe, &acc_min);
    else acc = lane_q6k_avx2(lds_w, o_row, bpr, k, xq, xd, xe);
    // hsum256: ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7))
    float h = acc + __shfl_xor(acc, 4);
    h = h + __shfl_xor(h, 2);
    h = h + __shfl_xor(h, 1);
    if (k == 0) Y[row0 + r] = h - acc_min;
  }
}

// Per-(row, block) exact integer sums through the production staging and
// integer code (block_*_ints); out is [rows][bpr][PER].
template <int FMT, int NT, int MAXC, int MAXX>
__global__ __launch_bounds__(NT) void block_sums_kernel(const uint8_t* __restrict__ W, const uint8_t* __restrict__ X,
                                                        int32_t* __restrict__ out, int rows, int bpr, int tr) {
  using F = Fmt<FMT>;
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x;
  const int row0 = blockIdx.x * tr;
  const int nr = min(tr, rows - row0);
  const TileGeom<FMT> G(bpr, tr);
  const uint32_t skew = stage_all<FMT, NT, MAXC, MAXX>(W, X, bpr, row0, nr, G, smem);
  const uint8_t* lds_w = smem + G.xrep;
  const uint32_t* xq = (const uint32_t*)smem;
  const int32_t* xe = (const int32_t*)(smem + bpr * 260);
  constexpr int PER = FMT == kQ8_0 ? 1 : (FMT == kQ4K ? 9 : 16);
  for (int i = tid; i < nr * bpr; i += NT) {
    int r = i / bpr;
    int b = i - r * bpr;
    uint32_t o = skew + (uint32_t)i * F::BS;
    int32_t* dst = out + ((size_t)(row0 + r) * bpr + b) * PER;
    if constexpr (FMT == kQ8_0) {
      dst[0] = block_q8_0_ints(lds_w, o, xq, b);
    } else if constexpr (FMT == kQ4K) {
      Q4KInts q;
      block_q4k_ints(lds_w, o, xq, xe, b, q);
      for (int j = 0; j < 8; j++) dst[j] = q.sub[j];
      dst[8] = q.sum_m;
    } else {
      uint32_t v[53];
      load_q6k_block(lds_w, o, v);
      int gs[16];
      block_q6k_ints(v, xq, xe, b, gs);
      for (int g = 0; g < 16; g++) dst[g] = gs[g];
    }
  }
}

// ---- host-side launch ------------------------------------------------------------

// Rows per workgroup: as many as fit a 48 KiB weight tile and the 64 KiB LDS
// budget; `lanes8`: at most NT/8, one lane per (row, k) of the AVX2 order.
template <int FMT>
static int pick_tile_rows(int rows, int bpr, bool lanes8, int cap) {
  const size_t rowbytes = (size_t)bpr * Fmt<FMT>::BS;
  const size_t max_tile = (size_t)kMatvecNT * kMatvecMaxC * 16 - 32;
  int tr = (int)(max_tile / rowbytes);
  if (lanes8 && tr > kMatvecNT / 8) tr = kMatvecNT / 8;
  if (cap > 0 && cap < tr) tr = cap;
  if (tr > rows) tr = rows;
  while (tr > 0 && TileGeom<FMT>(bpr, tr).total() > kLdsLimit) tr--;
  return tr;
}

template <int FMT>
static int launch_matvec_avx2(const MatvecLaunch& L) {
  const int tr = pick_tile_rows<FMT>(L.rows, L.bpr, true, L.tile_rows);
  if (tr <= 0) return NRQ_LAUNCH_TOO_WIDE;
  const int grid = (L.rows + tr - 1) / tr;
  const size_t lds = TileGeom<FMT>(L.bpr, tr).total();
  hipLaunchKernelGGL((matvec_avx2_kernel<FMT, kMatvecNT, kMatvecMaxC, kMatvecMaxX>), dim3(grid), dim3(kMatvecNT), lds,
                     (hipStream_t)L.stream, (const uint8_t*)L.w, (const uint8_t*)L.x, L.y, L.rows, L.bpr, tr);
  return hipGetLastError() == hipSuccess ? 0 : NRQ_LAUNCH_FAILED;
}

template <int FMT>
static int launch_block_sums_t(const void* w, const void* x, int32_t* out, int rows, int bpr, void* stream) {
  const int tr = pick_tile_rows<FMT>(rows, bpr, false, 0);
  if (tr <= 0) return NRQ_LAUNCH_TOO_WIDE;
  const int grid = (rows + tr - 1) / tr;
  const size_t lds = TileGeom<FMT>(bpr, tr).total();
  hipLaunchKernelGGL((block_sums_kernel<FMT, kMatvecNT, kMatvecMaxC, kMatvecMaxX>), dim3(grid), dim3(kMatvecNT), lds,
                     (hipStream_t)stream, (const uint8_t*)w, (const uint8_t*)x, out, rows, bpr, tr);
  return hipGetLastError() == hipSuccess ? 0 : NRQ_LAUNCH_FAILED;
}

int launch_block_sums(int dtype, const void* w, const void* x, int32_t* out, int rows, int bpr, void* stream) {
  if (rows <= 0 || bpr <= 0) return 0;
  if (dtype == kQ8_0) return launch_block_sums_t<kQ8_0>(w, x, out, rows, bpr, stream);
  if (dtype == kQ4K) return launch_block_sums_t<kQ4K>(w, x, out, rows, bpr, stream);
  if (dtype == kQ6K) return launch_block_sums_t<kQ6K>(w, x, out, rows, bpr, stream);
  return NRQ_LAUNCH_BAD_ARG;
}

int launch_matvec(int dtype, int order, const MatvecLaunch& L) {
  if (L.rows <= 0 || L.bpr <= 0) return 0;
  if (order == kOrderScalar) return launch_wstream_scalar(dtype, L);
  if (dtype == kQ8_0) return launch_matvec_avx2<kQ8_0>(L);
  if (dtype == kQ4K) return launch_matvec_avx2<kQ4K>(L);
  if (dtype == kQ6K) return launch_matvec_avx2<kQ6K>(L);
  return NRQ_LAUNCH_BAD_ARG;
}

}  // namespace nrq
