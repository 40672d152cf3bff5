// Decode matvec, scalar f32 order, one lane per block, per-wave streaming.
// Bit-identical to the reference's scalar kernels
//   dot_q8_scalar  (crates/nr-tensor/src/kernels.rs:72-82)
//   dot_q4k_scalar (crates/nr-tensor/src/kquant.rs:192-218)
//   dot_q6k_scalar (crates/nr-tensor/src/kquant.rs:220-250)
// inside the row loops of matvec_q8 (kernels.rs:36-70) and kquant_matvec!
// (kquant.rs:536-564).
//
// Work split. Each wave owns `rpw` consecutive rows. Their blocks are one
// contiguous byte range of W, cut into tiles of 64 lanes x BPL blocks. A tile
// moves HBM -> LDS with global_load_lds_dwordx4 (1 KiB per wave instruction)
// into one of NS per-wave stages, so up to NS tiles are in flight. A wave
// waits only on its own loads (s_waitcnt vmcnt); after the activation is
// staged, waves never wait for each other.
//
// Compute. Lane l of a tile forms the contribution of block l (+64k) exactly
// as the scalar kernel does: exact integer sub-dots with v_dot4_i32_i8 (and
// v_dot2_i32_i16 for the Q4_K min term), then the reference's f32 steps in
// its order. Contributions go to the wave's LDS slot u[b * rpw + r]; after
// the last tile, lane r adds row r's contributions in block order, the
// reference's `sumf +=` chain.
#include "nrq_device.h"
#include "nrq_launch.h"

namespace nrq {

namespace {

__device__ __forceinline__ void ws_dma4(const void* g, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off" : : "s"(m0), "v"(g) : "memory");
}

__device__ __forceinline__ void ws_dma16(const void* g, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" : : "s"(m0), "v"(g) : "memory");
}

template <int N>
__device__ __forceinline__ void ws_wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

__device__ __forceinline__ void ws_wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0x7f | (0 << 8) | (3 << 14)); }

// Workgroup barrier over LDS only; global loads in flight keep running.
__device__ __forceinline__ void ws_lds_barrier() {
  asm volatile("" ::: "memory");
  ws_wait_lgkm0();
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ uint32_t ws_lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)p;
}

// Per-format constants.
//   BS   weight block bytes       XB  activation block bytes
//   BPL  blocks per lane per tile NI  1 KiB DMA instructions per tile
//   XS   activation dwords per block in LDS
// Activation LDS layouts (dwords):
//   Q8_0 : [qs 8][d][pad 3]                                    stride 12
//   Q4_K : [qs 64][bsums 8][d][pad 11]                        stride 84
//          (placed by dword DMA straight from the Q8_K blocks, no repack)
//   Q6_K : [qs 64][-32 * group sums: 16][d][pad 3]             stride 84
// Strides 12 and 84 put the blocks read by one instruction on distinct
// 4-bank groups (84 = 20 mod 64).
template <int FMT>
struct WS;
template <>
struct WS<kQ8_0> {
  static constexpr int BS = kQ8_0Bytes, XB = kQ8_0Bytes, BPL = 4, NI = 9, XS = 12;
};
template <>
struct WS<kQ4K> {
  static constexpr int BS = kQ4KBytes, XB = kQ8KBytes, BPL = 1, NI = 9, XS = 84;
};
template <>
struct WS<kQ6K> {
  static constexpr int BS = kQ6KBytes, XB = kQ8KBytes, BPL = 1, NI = 14, XS = 84;
};

// Raw activation (already in LDS, `xskew` bytes into `raw`) -> padded layout.
template <int FMT>
__device__ void ws_repack(const uint32_t* raw, uint32_t xskew, int bpr, uint32_t* xl, int tid, int nt) {
  constexpr int XS = WS<FMT>::XS;
  if constexpr (FMT == kQ8_0) {
    for (int i = tid; i < bpr * 9; i += nt) {
      const int b = i / 9, t = i - b * 9;
      const uint32_t o = xskew + (uint32_t)b * kQ8_0Bytes;
      if (t < 8) xl[b * XS + t] = lds_u32_even(raw, o + 2 + 4 * t);
      else xl[b * XS + 8] = __float_as_uint(f16_bits_to_f32(lds_u16((const uint8_t*)raw, o)));
    }
  } else {
    // Q8_K block = 73 dwords: d @0, qs @1..64, bsums @65..72 (xskew is 4-aligned).
    const uint32_t* rw = raw + (xskew >> 2);
    for (int i = tid; i < bpr * 64; i += nt) {
      const int b = i >> 6, t = i & 63;
      xl[b * XS + t] = rw[b * 73 + 1 + t];
    }
    for (int i = tid; i < bpr * 16; i += nt) {
      const int b = i >> 4, g = i & 15;
      if constexpr (FMT == kQ6K) {
        int s = 0;  // -32 * (sum of the group's 16 quants): the (q - 32) term of the scalar dot
#pragma unroll
        for (int k = 0; k < 4; k++) s = sdot4(rw[b * 73 + 1 + 4 * g + k], 0xe0e0e0e0u, s);
        xl[b * XS + 64 + g] = (uint32_t)s;
        if (g == 0) xl[b * XS + 80] = rw[b * 73];
      }
    }
  }
}

// ---- per-block contributions (one lane, LDS in) --------------------------------------

// Q8_0 at even LDS byte offset o: (f32(acc) * dw) * dx (kernels.rs:75-79).
__device__ __forceinline__ float ws_q80(const uint32_t* w32, uint32_t o, const uint32_t* xb) {
  const uint32_t q0 = o + 2, base = q0 >> 2, sh = q0 & 3u;
  uint32_t D[9];
#pragma unroll
  for (int t = 0; t < 9; t++) D[t] = w32[base + t];
  const u32x4 xa = *(const u32x4*)xb, xc = *(const u32x4*)(xb + 4);
  const uint32_t X[8] = {xa.x, xa.y, xa.z, xa.w, xc.x, xc.y, xc.z, xc.w};
  int acc = 0;
#pragma unroll
  for (int t = 0; t < 8; t++) acc = sdot4(__builtin_amdgcn_alignbyte(D[t + 1], D[t], sh), X[t], acc);
  const uint32_t dbits = (o & 2) ? (w32[o >> 2] >> 16) : (w32[o >> 2] & 0xffffu);
  const float t1 = (float)acc * f16_bits_to_f32(dbits);
  return t1 * __uint_as_float(xb[8]);
}

// Q4_K at 16-byte-aligned LDS byte offset o (kquant.rs:195-215):
//   sub_j = sum of 32 q4*q8 (i32); sum_q += f32(sc_j) * f32(sub_j) in j order;
//   sum_m = sum_j m_j * (bsums[2j] + bsums[2j+1]);
//   contribution = d_all * sum_q - dmin_all * f32(sum_m).
// f32(sc) * f32(sub) == f32(sc * sub): |sc * sub| <= 63 * 61440 < 2^24, and the
// chain starts from +0.0, so a -0.0 product cannot change the sum.
__device__ __forceinline__ float ws_q4k(const uint8_t* lds_w, uint32_t o, const uint32_t* xb) {
  const u32x4 h = *(const u32x4*)(lds_w + o);
  // 6-bit scales and mins (kquant.rs:83-92), four per word:
  //   sc[0..4) = s[0..4] & 63             m[0..4) = s[4..8] & 63
  //   sc[4..8) = (s[8..12] & 15) | (s[0..4] >> 6) << 4
  //   m[4..8)  = (s[8..12] >> 4) | (s[4..8] >> 6) << 4
  const uint32_t s0 = h.y, s1 = h.z, s2 = h.w;
  const uint32_t scA = s0 & 0x3f3f3f3fu;
  const uint32_t mnA = s1 & 0x3f3f3f3fu;
  const uint32_t scB = (s2 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u);
  const uint32_t mnB = ((s2 >> 4) & 0x0f0f0f0fu) | ((s1 >> 2) & 0x30303030u);
  int sub[8];
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const u32x4 qa = *(const u32x4*)(lds_w + o + 16 + 32 * c);
    const u32x4 qb = *(const u32x4*)(lds_w + o + 32 + 32 * c);
    const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    const u32x4 x0 = *(const u32x4*)(xb + 16 * c), x1 = *(const u32x4*)(xb + 16 * c + 4);
    const u32x4 x2 = *(const u32x4*)(xb + 16 * c + 8), x3 = *(const u32x4*)(xb + 16 * c + 12);
    const uint32_t xl[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    const uint32_t xh[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
    int lo = 0, hi = 0;
#pragma unroll
    for (int t = 0; t < 8; t++) {
      lo = sdot4(q[t] & 0x0f0f0f0fu, xl[t], lo);
      hi = sdot4((q[t] >> 4) & 0x0f0f0f0fu, xh[t], hi);
    }
    sub[2 * c] = lo;
    sub[2 * c + 1] = hi;
  }
  // sc_j * sub_j on the 24-bit multiplier: |sc| < 64, |sub| <= 61440, so both
  // operands and the product fit 24 bits and the result is the exact product.
  float sum_q = (float)__mul24((int)(scA & 0xffu), sub[0]);
  sum_q = sum_q + (float)__mul24((int)((scA >> 8) & 0xffu), sub[1]);
  sum_q = sum_q + (float)__mul24((int)((scA >> 16) & 0xffu), sub[2]);
  sum_q = sum_q + (float)__mul24((int)(scA >> 24), sub[3]);
  sum_q = sum_q + (float)__mul24((int)(scB & 0xffu), sub[4]);
  sum_q = sum_q + (float)__mul24((int)((scB >> 8) & 0xffu), sub[5]);
  sum_q = sum_q + (float)__mul24((int)((scB >> 16) & 0xffu), sub[6]);
  sum_q = sum_q + (float)__mul24((int)(scB >> 24), sub[7]);
  // sum_m: m_j zero-extended into i16 pairs, dotted with the i16 pair sums.
  // m_j in both i16 halves against the activation's bsums[2j] | bsums[2j+1] << 16
  const u32x4 b0 = *(const u32x4*)(xb + 64), b1 = *(const u32x4*)(xb + 68);
  int sum_m = sdot2(__builtin_amdgcn_perm(0u, mnA, 0x0c000c00u), b0.x, 0);
  sum_m = sdot2(__builtin_amdgcn_perm(0u, mnA, 0x0c010c01u), b0.y, sum_m);
  sum_m = sdot2(__builtin_amdgcn_perm(0u, mnA, 0x0c020c02u), b0.z, sum_m);
  sum_m = sdot2(__builtin_amdgcn_perm(0u, mnA, 0x0c030c03u), b0.w, sum_m);
  sum_m = sdot2(__builtin_amdgcn_perm(0u, mnB, 0x0c000c00u), b1.x, sum_m);
  sum_m = sdot2(__builtin_amdgcn_perm(0u, mnB, 0x0c010c01u), b1.y, sum_m);
  sum_m = sdot2(__builtin_amdgcn_perm(0u, mnB, 0x0c020c02u), b1.z, sum_m);
  sum_m = sdot2(__builtin_amdgcn_perm(0u, mnB, 0x0c030c03u), b1.w, sum_m);
  const float xd = __uint_as_float(xb[72]);
  const float d_all = f16_bits_to_f32(h.x & 0xffffu) * xd;
  const float dmin_all = f16_bits_to_f32(h.x >> 16) * xd;
  const float a = d_all * sum_q;
  const float m = dmin_all * (float)sum_m;
  return a - m;
}

// Q6_K at even LDS byte offset o (kquant.rs:223-247): per half, the four
// planes of quants (q - 32), 16 group sums of (q - 32) * q8 (i32), then
// sum += f32(sc[g]) * f32(gs[g]) in g order and d_all * sum.
// f32(sc) * f32(gs) == f32(sc * gs): |sc * gs| <= 128 * 65536 < 2^24.
__device__ __forceinline__ float ws_q6k(const uint32_t* w32, uint32_t o, const uint32_t* xb) {
  const uint32_t sh = o & 3u, base = o >> 2;
  int gs[16];
  {
    const u32x4 c0 = *(const u32x4*)(xb + 64), c1 = *(const u32x4*)(xb + 68);
    const u32x4 c2 = *(const u32x4*)(xb + 72), c3 = *(const u32x4*)(xb + 76);
    const uint32_t C[16] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w,
                            c2.x, c2.y, c2.z, c2.w, c3.x, c3.y, c3.z, c3.w};
#pragma unroll
    for (int g = 0; g < 16; g++) gs[g] = (int)C[g];
  }
#pragma unroll
  for (int hh = 0; hh < 2; hh++) {
    uint32_t L[17], H[9];
#pragma unroll
    for (int t = 0; t < 17; t++) L[t] = w32[base + 16 * hh + t];       // ql[64hh ..]
#pragma unroll
    for (int t = 0; t < 9; t++) H[t] = w32[base + 32 + 8 * hh + t];    // qh[32hh ..]
    uint32_t X[32];
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const u32x4 v = *(const u32x4*)(xb + 32 * hh + 4 * k);
      X[4 * k] = v.x;
      X[4 * k + 1] = v.y;
      X[4 * k + 2] = v.z;
      X[4 * k + 3] = v.w;
    }
#pragma unroll
    for (int t = 0; t < 8; t++) {
      const uint32_t qlA = __builtin_amdgcn_alignbyte(L[t + 1], L[t], sh);
      const uint32_t qlB = __builtin_amdgcn_alignbyte(L[t + 9], L[t + 8], sh);
      const uint32_t qh = __builtin_amdgcn_alignbyte(H[t + 1], H[t], sh);
      uint32_t q6[4];
      q6k_planes(qlA, qlB, qh, q6);
#pragma unroll
      for (int n = 0; n < 4; n++) {
        const int g = 8 * hh + 2 * n + (t >> 2);
        gs[g] = sdot4(q6[n], X[8 * n + t], gs[g]);
      }
    }
  }
  const uint32_t S0 = __builtin_amdgcn_alignbyte(w32[base + 49], w32[base + 48], sh);  // scales[0..4)
  const uint32_t S1 = __builtin_amdgcn_alignbyte(w32[base + 50], w32[base + 49], sh);
  const uint32_t S2 = __builtin_amdgcn_alignbyte(w32[base + 51], w32[base + 50], sh);
  const uint32_t S3 = __builtin_amdgcn_alignbyte(w32[base + 52], w32[base + 51], sh);
  const uint32_t S[4] = {S0, S1, S2, S3};
  float sum = 0.0f;
#pragma unroll
  for (int g = 0; g < 16; g++) {
    const int s = (int)(int8_t)((S[g >> 2] >> (8 * (g & 3))) & 0xffu);
    sum = sum + (float)__mul24(s, gs[g]);  // |s| <= 128, |gs| <= 65536: exact in 24 bits
  }
  const uint32_t dw = w32[(o + 208) >> 2];
  const uint32_t dbits = ((o + 208) & 2) ? (dw >> 16) : (dw & 0xffffu);
  const float d_all = f16_bits_to_f32(dbits) * __uint_as_float(xb[80]);
  return d_all * sum;
}

}  // namespace

// LDS layout of one workgroup:
//   [activation, padded: bpr*XS dwords][raw activation window][per wave: NS stages | u]
// One launch: up to three matrices that share the activation.
struct WsArgs {
  const uint8_t* w[3];
  float* y[3];
  int rows[3];
  int wg_end[3];
  int nmat;
  const uint8_t* x;  // activation blocks (no fused norm)
  // fused norm (Q8_0 weights): residual in, pending residual (or null), their sum
  // (written by workgroup 0 when nadd != null), norm weight, epsilon
  const float* nx;
  const float* nadd;
  float* nx_out;
  const float* nw;
  float eps;
  float rscale;  // the pending residual is added as x + rscale * add (saxpy, vec.rs:68-72)
  // gate|up pair (nmat == 2, equal rows, multiple of 32): workgroup w computes
  // rows 32w .. 32w+31 of both (waves 0-1 gate, 2-3 up) and writes the Q8_0
  // blocks of swiglu(gate, up) (vec.rs:45-52, q8.rs:27-44) instead of y
  uint8_t* swiglu_q8;
  // fused norm, K-quant weights: workgroup 0 also stores the activation's Q8_K
  // blocks here (or null), for the next matvec over the same activation
  uint8_t* xq_out;
};

// Block contributions of a wave's rows wait in LDS for the per-row sum. Long
// rows (48+ blocks) are stored row-major with a padded stride, so each lane
// sums its own row with 16-byte pipelined reads; short rows block-major.
__host__ __device__ inline bool ws_u_rowmajor(int bpr) { return bpr >= 48; }

// Kernel variants, chosen at launch so that each instantiation carries only
// its own code: the fused rmsnorm prologue, the swiglu pair epilogue, and the
// row-major contribution layout.
enum { kWsNorm = 1, kWsSwiglu = 2, kWsRowMajorU = 4, kWsQuant = 8 };
__host__ __device__ inline int ws_u_stride(int bpr) { return ((bpr + 3) & ~3) + 4; }

template <int FMT>
struct WSGeom {
  size_t xl, xraw, stage, u, per_wave, total;
  __host__ __device__ WSGeom(int bpr, int rpw, int ns, int nw, bool urm) {
    if (FMT == kQ4K) {  // dword DMAs of 64 lanes write whole 256-byte runs
      xl = ((size_t)bpr * WS<FMT>::XS + 63) / 64 * 256;
      xraw = 0;
    } else {
      xl = ((size_t)bpr * WS<FMT>::XS * 4 + 15) & ~(size_t)15;
      // the DMA writes whole KiB per wave instruction
      xraw = ((size_t)bpr * WS<FMT>::XB + 15 + 15 + 1023) & ~(size_t)1023;
    }
    stage = (size_t)WS<FMT>::NI * 1024;
    u = (((size_t)rpw * (urm ? ws_u_stride(bpr) : bpr)) * 4 + 15) & ~(size_t)15;
    per_wave = (size_t)ns * stage + u;
    total = xl + xraw + (size_t)nw * per_wave;
  }
};

// Rmsnorm (vec.rs:4-14) after the pending residual add (vec.rs:63-67, scale
// 1.0), fused into a Q8_0 matvec's prologue: LDS holds x, add and the norm
// weight (DMA, issued before the weight tiles), then the squares; the result
// is quantized to Q8_0 (q8.rs:27-44) straight into the activation layout.
// One Q8_K block (kquant.rs:157-187) from a half-wave (q8k_half_lanes,
// nrq_device.h), written into the kernel's activation layout (Q4_K: qs,
// 16-value sums as i16 pairs, d; Q6_K: qs, -32 * 16-value sums, d) and, when
// gout != null, as the standard 292-byte block.
template <int FMT>
__device__ __forceinline__ void ws_q8k_half(const float o[8], int r, uint32_t* xb, uint8_t* gout) {
  uint32_t lo, hi, d_bits;
  int ps;
  q8k_half_lanes(o, r, &lo, &hi, &ps, &d_bits);
  const int ps2 = __shfl_down(ps, 2, 32);  // the next pair's sum
  ((uint2*)xb)[r] = make_uint2(lo, hi);
  if constexpr (FMT == kQ4K) {
    if ((r & 3) == 0) xb[64 + (r >> 2)] = ((uint32_t)ps & 0xffffu) | ((uint32_t)ps2 << 16);
    if (r == 0) xb[72] = d_bits;
  } else {
    if ((r & 1) == 0) xb[64 + (r >> 1)] = (uint32_t)(-32 * ps);
    if (r == 0) xb[80] = d_bits;
  }
  if (gout) q8k_half_store(gout, r, lo, hi, ps, d_bits);
}

constexpr int kFusedNormMax = 4096;
constexpr int kFusedNormPT = kFusedNormMax / 256;

// Fused-norm LDS, n floats per array: x (then its squares, in place) | norm
// weight | add. The add array (n >= 256 words) is the ordered sum's workspace
// (kWgChainWork words) once the squares exist.
static_assert(kWgChainWork <= 256, "the workspace fits the smallest add array");
__host__ __device__ inline size_t ws_norm_floats(int n) { return 3 * (size_t)n; }

__device__ __forceinline__ void ws_dma16_g(const void* g, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" : : "s"(m0), "v"(g) : "memory");
}

template <int FMT, int NW, int NS, int MODE>
__global__ __launch_bounds__(64 * NW) void wstream_matvec(WsArgs A, int bpr, int rpw, int nstages) {
  constexpr bool NORM = (MODE & kWsNorm) != 0, SWI = (MODE & kWsSwiglu) != 0, URM = (MODE & kWsRowMajorU) != 0;
  constexpr bool QNT = (MODE & kWsQuant) != 0;
  using F = WS<FMT>;
  static_assert(!QNT || (!NORM && FMT != kQ8_0), "the quantize prologue makes Q8_K blocks from an f32 activation");
  constexpr int NI = F::NI, BS = F::BS, TBK = 64 * F::BPL, STAGE = NI * 1024, NT = 64 * NW;
  static_assert(NS >= 1 && NS <= 4, "the vmcnt waits cover up to 4 stages");
  static_assert(!NORM || NW == 4, "the fused norm runs on 256 lanes");
  static_assert(!SWI || FMT == kQ8_0, "the swiglu pair writes Q8_0 blocks");
  static_assert(!SWI || NORM, "the swiglu pair is a fused-norm variant");
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  // workgroups [wg_end[i-1], wg_end[i]) take matrix i (the swiglu pair: waves 0-1 and 2-3)
  int mi = 0;
  if constexpr (SWI) {
    mi = wave >> 1;
  } else {
    while (mi + 1 < A.nmat && (int)blockIdx.x >= A.wg_end[mi]) mi++;
  }
  const int lwg = SWI ? 0 : (int)blockIdx.x - (mi ? A.wg_end[mi - 1] : 0);
  const uint8_t* __restrict__ W = A.w[mi];
  float* __restrict__ Y = A.y[mi];
  const int rows = A.rows[mi];
  const WSGeom<FMT> G(bpr, rpw, nstages, NW, URM);
  uint32_t* xl = (uint32_t*)smem;
  uint8_t* xraw = smem + G.xl;
  uint8_t* stages = xraw + G.xraw + (size_t)wave * G.per_wave;
  float* u = (float*)(stages + (size_t)nstages * STAGE);
  const uint32_t stage0 = ws_lds_addr(stages);

  const int row0 = SWI ? (int)blockIdx.x * 2 * rpw + (wave & 1) * rpw : (lwg * NW + wave) * rpw;
  const int nr = max(0, min(rpw, rows - row0));
  const int nb = nr * bpr;
  const size_t fbeg = (size_t)max(row0, 0) * bpr;  // first flat block of this wave
  const int ntiles = (nb + TBK - 1) / TBK;

  // Tile t: flat blocks [fbeg + t*TBK, ...) -> 16-byte window [a0, a0 + 16*n16), stage t % nstages.
  auto issue = [&](int t) {
    const size_t fb0 = fbeg + (size_t)t * TBK;
    const size_t fb1 = fbeg + (size_t)min(nb, (t + 1) * TBK);
    const size_t a0 = (fb0 * BS) & ~(size_t)15;
    const int n16 = (int)(((((fb1 * BS) + 15) & ~(size_t)15) - a0) >> 4);
    const uint32_t sbase = stage0 + (uint32_t)((t % nstages) * STAGE);
#pragma unroll
    for (int k = 0; k < NI; k++) {
      const int ci = min(k * 64 + lane, n16 - 1);  // past the window: reload its last chunk
      ws_dma16(W + a0 + 16 * (size_t)ci, sbase + (uint32_t)k * 1024u);
    }
  };

  // The activation (or the norm's inputs) first, so an in-order vmcnt wait below covers it.
  float* nxs = (float*)(smem + G.total);  // fused norm: x (then squares) | weight | add | pad | scale
  const int n = bpr * (FMT == kQ8_0 ? 32 : 256);
  if constexpr (QNT) {  // the f32 activation, quantized after the barrier below
    const uint32_t dst = ws_lds_addr(nxs);
    for (int k = wave; k < n / 256; k += NW) ws_dma16_g(A.nx + 256 * k + 4 * lane, dst + (uint32_t)k * 1024u);
  } else if constexpr (NORM) {
    const int nk = n / 256;  // 1 KiB DMAs per array
    const float* src[3] = {A.nx, A.nw, A.nadd};
#pragma unroll
    for (int a = 0; a < 3; a++) {
      if (a == 2 && !A.nadd) continue;
      const uint32_t dst = ws_lds_addr(nxs + (size_t)a * n);
      for (int k = wave; k < nk; k += NW) ws_dma16_g(src[a] + 256 * k + 4 * lane, dst + (uint32_t)k * 1024u);
    }
  } else if constexpr (FMT == kQ4K) {
    // LDS dword p of the padded layout = dword j = p % 84 of block b = p / 84:
    // qs and bsums (j < 72) are Q8_K dwords 1 + j, d (j = 72) is dword 0;
    // padding and the run past the last block load dword 0 of a block.
    const uint32_t* xw = (const uint32_t*)A.x;
    const int nins = (bpr * WS<FMT>::XS + 63) / 64;
    const uint32_t xbase = ws_lds_addr(xl);
    for (int k = wave; k < nins; k += NW) {
      const int p = 64 * k + lane;
      int b = p / WS<FMT>::XS;
      int j = p - b * WS<FMT>::XS;
      if (b >= bpr) {
        b = bpr - 1;
        j = 72;
      }
      ws_dma4(xw + (size_t)b * 73 + (j < 72 ? 1 + j : 0), xbase + (uint32_t)k * 256u);
    }
  } else {
    const uintptr_t xa = (uintptr_t)A.x;
    const uintptr_t xa0 = xa & ~(uintptr_t)15;
    const int n16x = (int)(((((xa + (size_t)bpr * F::XB) + 15) & ~(uintptr_t)15) - xa0) >> 4);
    const uint32_t rbase = ws_lds_addr(xraw);
    for (int grp = wave; grp * 64 < n16x; grp += NW) {
      const int ci = min(grp * 64 + lane, n16x - 1);
      ws_dma16((const uint8_t*)xa0 + 16 * (size_t)ci, rbase + (uint32_t)grp * 1024u);
    }
  }
  const int pro = min(nstages, ntiles);
  for (int t = 0; t < pro; t++) issue(t);
  // the activation landed once at most `pro` tiles' loads are outstanding
  switch (pro) {
    case 0: ws_wait_vm<0>(); break;
    case 1: ws_wait_vm<NI>(); break;
    case 2: ws_wait_vm<2 * NI>(); break;
    case 3: ws_wait_vm<3 * NI>(); break;
    default: ws_wait_vm<4 * NI>(); break;
  }
  ws_lds_barrier();
  if constexpr (NORM) {
    const float* xs = nxs;
    const float* wsn = nxs + n;
    const float* as = nxs + 2 * (size_t)n;
    // each run's squares overwrite its x, read just before by the same thread
    float* sq = nxs;
    // Thread t owns the 8-value runs j = t + NT*k; four consecutive runs (an
    // aligned lane quad) make one Q8_0 block.
    const int nrun = n >> 3;
    const float4* xs4 = (const float4*)xs;
    const float4* as4 = (const float4*)as;
    const float4* ws4 = (const float4*)wsn;
    float v[kFusedNormPT];
#pragma unroll
    for (int k = 0; k < kFusedNormPT / 8; k++) {
      const int j = tid + NT * k;
      if (j < nrun) {
        const float4 p0 = xs4[2 * j], p1 = xs4[2 * j + 1];
        float a[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
        if (A.nadd) {
          const float4 q0 = as4[2 * j], q1 = as4[2 * j + 1];
          const float b[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
          for (int e = 0; e < 8; e++) a[e] = a[e] + A.rscale * b[e];
          if (blockIdx.x == 0) {
            ((float4*)A.nx_out)[2 * j] = make_float4(a[0], a[1], a[2], a[3]);
            ((float4*)A.nx_out)[2 * j + 1] = make_float4(a[4], a[5], a[6], a[7]);
          }
        }
#pragma unroll
        for (int e = 0; e < 8; e++) v[8 * k + e] = a[e];
        ((float4*)sq)[2 * j] = make_float4(a[0] * a[0], a[1] * a[1], a[2] * a[2], a[3] * a[3]);
        ((float4*)sq)[2 * j + 1] = make_float4(a[4] * a[4], a[5] * a[5], a[6] * a[6], a[7] * a[7]);
      }
    }
    ws_lds_barrier();
    // every wave takes part in the ordered sum and gets its result; the add
    // array is dead here: the sum's workspace
    const float ss = wg_chain_nonneg<NW>(sq, n, 0.0f, (uint32_t*)(nxs + 2 * (size_t)n));
    const float scale = 1.0f / sqrtf(ss / (float)n + A.eps);
#pragma unroll
    for (int k = 0; k < kFusedNormPT / 8; k++) {
      const int j = tid + NT * k;
      if (j < nrun) {
        const float4 w0 = ws4[2 * j], w1 = ws4[2 * j + 1];
        const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] = v[8 * k + e] * scale * w[e];
        if constexpr (FMT == kQ8_0) {
          uint32_t lo, hi, d_bits;
          q8_0_quad8(o, &lo, &hi, &d_bits);
          uint32_t* xb = xl + (j >> 2) * WS<kQ8_0>::XS;
          ((uint2*)xb)[j & 3] = make_uint2(lo, hi);
          if ((j & 3) == 0) xb[8] = __float_as_uint(f16_bits_to_f32(d_bits));
        } else {
          // a Q8_K block is 32 runs, one aligned half-wave (nrun is a multiple of 32)
          ws_q8k_half<FMT>(o, j & 31, xl + (j >> 5) * WS<FMT>::XS,
                           (A.xq_out && blockIdx.x == 0) ? A.xq_out + (size_t)(j >> 5) * kQ8KBytes : nullptr);
        }
      }
    }
    ws_lds_barrier();
  } else if constexpr (QNT) {
    // Q8_K blocks of the activation (kquant.rs:157-187), a half-wave per block
    const float4* xs4 = (const float4*)nxs;
    for (int j = tid; j < (n >> 3); j += NT) {
      const float4 p0 = xs4[2 * j], p1 = xs4[2 * j + 1];
      const float o[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
      ws_q8k_half<FMT>(o, j & 31, xl + (j >> 5) * WS<FMT>::XS, nullptr);
    }
    ws_lds_barrier();
  } else if constexpr (FMT != kQ4K) {
    ws_repack<FMT>((const uint32_t*)xraw, (uint32_t)((uintptr_t)A.x & 15), bpr, xl, tid, NT);
    ws_lds_barrier();
  }

  // Lane l's k-th block of tile t is flat block fbeg + t*TBK + l + 64k; track its (row, block).
  int rr[F::BPL], bb[F::BPL];
#pragma unroll
  for (int k = 0; k < F::BPL; k++) {
    const int f = lane + 64 * k;
    rr[k] = f / bpr;
    bb[k] = f - rr[k] * bpr;
  }
  const int step_r = TBK / bpr, step_b = TBK - step_r * bpr;
  const int ust = ws_u_stride(bpr);

  for (int t = 0; t < ntiles; t++) {
    const int after = min(nstages - 1, ntiles - 1 - t);  // tiles issued after t
    switch (after) {  // tile t landed once `after` tiles' loads are outstanding
      case 0: ws_wait_vm<0>(); break;
      case 1: ws_wait_vm<NI>(); break;
      case 2: ws_wait_vm<2 * NI>(); break;
      default: ws_wait_vm<3 * NI>(); break;
    }
    asm volatile("" ::: "memory");
    const uint8_t* cur = stages + (t % nstages) * STAGE;
    const int tb0 = t * TBK;
    const uint32_t skew = (uint32_t)(((fbeg + tb0) * BS) & 15);
#pragma unroll
    for (int k = 0; k < F::BPL; k++) {
      const int i = lane + 64 * k;
      if (tb0 + i < nb) {
        // LDS offsets stay below 160 KiB, so the 24-bit multiplier is exact here
        const uint32_t o = skew + __umul24((uint32_t)i, (uint32_t)BS);
        const uint32_t* xb = xl + __umul24((uint32_t)bb[k], (uint32_t)F::XS);
        float c;
        if constexpr (FMT == kQ8_0) c = ws_q80((const uint32_t*)cur, o, xb);
        else if constexpr (FMT == kQ4K) c = ws_q4k(cur, o, xb);
        else c = ws_q6k((const uint32_t*)cur, o, xb);
        if constexpr (URM) u[__umul24((uint32_t)rr[k], (uint32_t)ust) + bb[k]] = c;
        else u[__umul24((uint32_t)bb[k], (uint32_t)rpw) + rr[k]] = c;
      }
      rr[k] += step_r;
      bb[k] += step_b;
      if (bb[k] >= bpr) {
        bb[k] -= bpr;
        rr[k] += 1;
      }
    }
    if (t + nstages < ntiles) {
      ws_wait_lgkm0();  // this stage's reads are done before the DMA refills it
      asm volatile("" ::: "memory");
      issue(t + nstages);
    }
  }
  ws_wait_lgkm0();
  asm volatile("" ::: "memory");
  // the reference's `sumf += contribution` chain, block order
  float s = 0.0f;
  if (lane < nr) {
    if constexpr (URM) {
      s = chain_from(u + lane * ust, bpr, 0.0f);
    } else {
      for (int b = 0; b < bpr; b++) s = s + u[b * rpw + lane];
    }
    if constexpr (!SWI) Y[row0 + lane] = s;
  }
  if constexpr (SWI) {
    // gate rows land in gu[0 .. 2 rpw), up rows in gu[2 rpw .. 4 rpw) (rpw = 16)
    float* gu = (float*)xl;  // the activation is no longer read
    ws_lds_barrier();
    if (lane < rpw) gu[(wave >> 1) * 2 * rpw + (wave & 1) * rpw + lane] = s;
    ws_lds_barrier();
    if (tid < 2 * rpw) {
      const float gv = gu[tid], uv = gu[2 * rpw + tid];
      const float silu = gv / (1.0f + dev_expf(-gv));
      const float v = silu * uv;
      uint32_t d_bits;
      const int q = q8_0_lane(v, &d_bits);
      uint8_t* blk = A.swiglu_q8 + (size_t)blockIdx.x * kQ8_0Bytes;
      blk[2 + tid] = (uint8_t)(int8_t)q;
      if (tid == 0) {
        blk[0] = (uint8_t)(d_bits & 0xff);
        blk[1] = (uint8_t)(d_bits >> 8);
      }
    }
  }
}

// ---- launch ----------------------------------------------------------------------------------

template <int FMT, int NW, int NS, int MODE>
static int launch_ws_t(WsArgs A, int bpr, int rpw, void* stream) {
  constexpr bool NORM = (MODE & kWsNorm) != 0, SWI = (MODE & kWsSwiglu) != 0, URM = (MODE & kWsRowMajorU) != 0;
  constexpr bool QNT = (MODE & kWsQuant) != 0;
  constexpr int TBK = 64 * WS<FMT>::BPL;
  int grid = 0;
  if constexpr (SWI) {
    grid = A.rows[0] / (2 * rpw);
    A.wg_end[0] = A.wg_end[1] = grid;
  } else {
    for (int i = 0; i < A.nmat; i++) {
      const long waves = (A.rows[i] + rpw - 1) / rpw;
      grid += (int)((waves + NW - 1) / NW);
      A.wg_end[i] = grid;
    }
  }
  const long tiles_per_wave = ((long)rpw * bpr + TBK - 1) / TBK;
  const int nstages = (int)(tiles_per_wave < NS ? tiles_per_wave : NS);
  const WSGeom<FMT> G(bpr, rpw, nstages, NW, URM);
  // fused norm: x, add, weight, squares (n floats each) and the scale
  const size_t lds = G.total + (NORM ? ws_norm_floats(bpr * (FMT == kQ8_0 ? 32 : 256)) * 4 : 0) +
                     (QNT ? (size_t)bpr * 256 * 4 : 0);
  if (lds > 160 * 1024) return NRQ_LAUNCH_TOO_WIDE;
  if (grid == 0) return 0;
  hipLaunchKernelGGL((wstream_matvec<FMT, NW, NS, MODE>), dim3(grid), dim3(64 * NW), lds, (hipStream_t)stream, A, bpr,
                     rpw, nstages);
  return hipGetLastError() == hipSuccess ? 0 : NRQ_LAUNCH_FAILED;
}

// Rows per wave: the smallest count whose blocks fill at least 85% of the
// lanes of the wave's tiles (a partly empty tile costs as much as a full one).
// Small counts also give the most waves, which short matrices need to cover
// every CU.
template <int FMT>
static int ws_rows_per_wave(int bpr, int cap) {
  constexpr int TBK = 64 * WS<FMT>::BPL;
  if (cap > 0) return cap < 64 ? cap : 64;
  int best = 1;
  double best_util = 0.0;
  for (int r = 1; r <= 64; r++) {
    const long blocks = (long)r * bpr;
    const long slots = (blocks + TBK - 1) / TBK * TBK;
    const double util = (double)blocks / (double)slots;
    if (util >= 0.85) return r;
    if (util > best_util) {
      best_util = util;
      best = r;
    }
  }
  return best;
}

static int ws_num_cus();

template <int FMT>
static int launch_ws(const MatvecLaunch& L) {
  int rpw = ws_rows_per_wave<FMT>(L.bpr, L.tile_rows);
  // Short matrices: half the rows per wave when that still fills half of each
  // tile and the default leaves SIMDs without a wave (the Llama-3.2-1B o
  // projection, 2048 x 2048 Q8_0: four rows per wave, 512 waves, 5.32 us; two
  // rows, 1024 waves, 4.98 us; single launches after the MALL flush)
  if (L.tile_rows == 0 && rpw % 2 == 0) {
    constexpr int TBK = 64 * WS<FMT>::BPL;
    const long waves = ((long)L.rows + rpw - 1) / rpw;
    if (waves < 4L * ws_num_cus() && 2L * (rpw / 2) * L.bpr >= TBK) rpw /= 2;
  }
  WsArgs A{};
  A.w[0] = (const uint8_t*)L.w;
  A.y[0] = L.y;
  A.rows[0] = L.rows;
  A.nmat = 1;
  A.x = (const uint8_t*)L.x;
  // NW waves share one activation copy; NS = 2 (double buffering) keeps a tile
  // in flight per wave while the other is computed, within the LDS of a CU.
  int rc;
  if (ws_u_rowmajor(L.bpr)) {
    rc = launch_ws_t<FMT, 4, 2, kWsRowMajorU>(A, L.bpr, rpw, L.stream);
    if (rc == NRQ_LAUNCH_TOO_WIDE) rc = launch_ws_t<FMT, 1, 2, kWsRowMajorU>(A, L.bpr, rpw, L.stream);
    if (rc == NRQ_LAUNCH_TOO_WIDE) rc = launch_ws_t<FMT, 1, 2, kWsRowMajorU>(A, L.bpr, 1, L.stream);
  } else {
    // Q4_K: eight waves share one activation copy (about 3% faster than four on
    // the 8192 x 3072 matvec, measured in one process; other formats gain nothing)
    rc = FMT == kQ4K ? launch_ws_t<FMT, 8, 2, 0>(A, L.bpr, rpw, L.stream) : NRQ_LAUNCH_TOO_WIDE;
    if (rc == NRQ_LAUNCH_TOO_WIDE) rc = launch_ws_t<FMT, 4, 2, 0>(A, L.bpr, rpw, L.stream);
    if (rc == NRQ_LAUNCH_TOO_WIDE) rc = launch_ws_t<FMT, 1, 2, 0>(A, L.bpr, rpw, L.stream);
    if (rc == NRQ_LAUNCH_TOO_WIDE) rc = launch_ws_t<FMT, 1, 2, 0>(A, L.bpr, 1, L.stream);
  }
  return rc;
}

static int ws_num_cus() {
  static int n = 0;
  if (n == 0) {
    int dev = 0, v = 0;
    n = (hipGetDevice(&dev) == hipSuccess &&
         hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            ? v
            : 256;
  }
  return n;
}

int launch_norm_matvec(int dtype, const NormMatvecLaunch& L) {
  if (dtype != kQ8_0 && dtype != kQ4K && dtype != kQ6K) return NRQ_LAUNCH_TOO_WIDE;
  const int qk = dtype == kQ8_0 ? 32 : 256;
  if (L.nmat < 1 || L.nmat > 3 || L.n <= 0 || L.n % 256 || L.n > kFusedNormMax) return NRQ_LAUNCH_TOO_WIDE;
  if (L.swiglu_q8 && dtype != kQ8_0) return NRQ_LAUNCH_TOO_WIDE;
  const int bpr = L.n / qk;
  // Every workgroup runs the norm's sequential sum once, and its LDS allows one
  // workgroup per CU, so the launch is sized to one workgroup per CU: rows per
  // wave grow (in steps that keep the tiles full) until the grid fits.
  const int rpw0 = dtype == kQ8_0 ? ws_rows_per_wave<kQ8_0>(bpr, 0)
                   : dtype == kQ4K ? ws_rows_per_wave<kQ4K>(bpr, 0)
                                   : ws_rows_per_wave<kQ6K>(bpr, 0);
  long total = 0;
  for (int i = 0; i < L.nmat; i++) total += L.rows[i];
  const long slots = 4L * ws_num_cus();
  // the fewest rows per wave whose workgroups (four waves, per matrix) fit one
  // per CU and whose blocks fill 85% of their tiles
  const int tbk = dtype == kQ8_0 ? 64 * WS<kQ8_0>::BPL : 64;
  int rpw = 0;
  for (int r = rpw0; r <= 64 && !rpw; r++) {
    long wgs = 0;
    for (int i = 0; i < L.nmat; i++) wgs += ((L.rows[i] + r - 1) / r + 3) / 4;
    const long tiles = ((long)r * bpr + tbk - 1) / tbk;
    if (4 * wgs <= slots && (double)r * bpr >= 0.85 * (double)(tiles * tbk)) rpw = r;
  }
  if (!rpw) {
    rpw = rpw0;
    while (rpw + rpw0 <= 64 && (total + rpw - 1) / rpw + 3L * L.nmat > slots) rpw += rpw0;
  }
  if (L.swiglu_q8) {  // 16 rows per wave: a workgroup owns 32 rows of gate and of up
    if (L.nmat != 2 || L.rows[0] != L.rows[1] || L.rows[0] % 32) return NRQ_LAUNCH_TOO_WIDE;
    rpw = 16;
  }
  WsArgs A{};
  for (int i = 0; i < L.nmat; i++) {
    A.w[i] = (const uint8_t*)L.w[i];
    A.y[i] = L.y[i];
    A.rows[i] = L.rows[i];
  }
  A.nmat = L.nmat;
  A.nx = L.x;
  A.nadd = L.add;
  A.nx_out = L.x_out;
  A.nw = L.norm_w;
  A.eps = L.eps;
  A.rscale = L.rscale;
  A.swiglu_q8 = L.swiglu_q8;
  A.xq_out = L.xq_out;
  const bool urm = ws_u_rowmajor(bpr);
  if (dtype == kQ4K) {
    // three stages where the LDS has room: a wave's tiles in flight during the norm
    int rc = urm ? launch_ws_t<kQ4K, 4, 3, kWsNorm | kWsRowMajorU>(A, bpr, rpw, L.stream)
                 : launch_ws_t<kQ4K, 4, 3, kWsNorm>(A, bpr, rpw, L.stream);
    if (rc == NRQ_LAUNCH_TOO_WIDE)
      rc = urm ? launch_ws_t<kQ4K, 4, 2, kWsNorm | kWsRowMajorU>(A, bpr, rpw, L.stream)
               : launch_ws_t<kQ4K, 4, 2, kWsNorm>(A, bpr, rpw, L.stream);
    return rc;
  }
  if (dtype == kQ6K)
    return urm ? launch_ws_t<kQ6K, 4, 2, kWsNorm | kWsRowMajorU>(A, bpr, rpw, L.stream)
               : launch_ws_t<kQ6K, 4, 2, kWsNorm>(A, bpr, rpw, L.stream);
  if (L.swiglu_q8)
    return urm ? launch_ws_t<kQ8_0, 4, 2, kWsNorm | kWsSwiglu | kWsRowMajorU>(A, bpr, rpw, L.stream)
               : launch_ws_t<kQ8_0, 4, 2, kWsNorm | kWsSwiglu>(A, bpr, rpw, L.stream);
  return urm ? launch_ws_t<kQ8_0, 4, 2, kWsNorm | kWsRowMajorU>(A, bpr, rpw, L.stream)
             : launch_ws_t<kQ8_0, 4, 2, kWsNorm>(A, bpr, rpw, L.stream);
}

int launch_quant_matvec(int dtype, const float* x, int n, const void* w, float* y, int rows, void* stream) {
  if ((dtype != kQ4K && dtype != kQ6K) || n <= 0 || n % 256 || rows <= 0) return NRQ_LAUNCH_TOO_WIDE;
  const int bpr = n / 256;
  WsArgs A{};
  A.w[0] = (const uint8_t*)w;
  A.y[0] = y;
  A.rows[0] = rows;
  A.nmat = 1;
  A.nx = x;
  const bool urm = ws_u_rowmajor(bpr);
  if (dtype == kQ4K) {
    const int rpw = ws_rows_per_wave<kQ4K>(bpr, 0);
    return urm ? launch_ws_t<kQ4K, 4, 2, kWsQuant | kWsRowMajorU>(A, bpr, rpw, stream)
               : launch_ws_t<kQ4K, 4, 2, kWsQuant>(A, bpr, rpw, stream);
  }
  const int rpw = ws_rows_per_wave<kQ6K>(bpr, 0);
  return urm ? launch_ws_t<kQ6K, 4, 2, kWsQuant | kWsRowMajorU>(A, bpr, rpw, stream)
             : launch_ws_t<kQ6K, 4, 2, kWsQuant>(A, bpr, rpw, stream);
}

// Up to three matrices of one format over one activation in one launch
// (q|k, gate|up in a K-quant layer): workgroups are laid out matrix after
// matrix, each row computed as launch_ws computes it.
template <int FMT>
static int launch_ws_group(const void* const* w, float* const* y, const int* rows, int n, const void* x, int bpr,
                           void* stream) {
  const int rpw = ws_rows_per_wave<FMT>(bpr, 0);
  WsArgs A{};
  for (int i = 0; i < n; i++) {
    A.w[i] = (const uint8_t*)w[i];
    A.y[i] = y[i];
    A.rows[i] = rows[i];
  }
  A.nmat = n;
  A.x = (const uint8_t*)x;
  int rc;
  if (ws_u_rowmajor(bpr)) {
    rc = launch_ws_t<FMT, 4, 2, kWsRowMajorU>(A, bpr, rpw, stream);
    if (rc == NRQ_LAUNCH_TOO_WIDE) rc = launch_ws_t<FMT, 1, 2, kWsRowMajorU>(A, bpr, rpw, stream);
    if (rc == NRQ_LAUNCH_TOO_WIDE) rc = launch_ws_t<FMT, 1, 2, kWsRowMajorU>(A, bpr, 1, stream);
  } else {
    rc = FMT == kQ4K ? launch_ws_t<FMT, 8, 2, 0>(A, bpr, rpw, stream) : NRQ_LAUNCH_TOO_WIDE;
    if (rc == NRQ_LAUNCH_TOO_WIDE) rc = launch_ws_t<FMT, 4, 2, 0>(A, bpr, rpw, stream);
    if (rc == NRQ_LAUNCH_TOO_WIDE) rc = launch_ws_t<FMT, 1, 2, 0>(A, bpr, rpw, stream);
    if (rc == NRQ_LAUNCH_TOO_WIDE) rc = launch_ws_t<FMT, 1, 2, 0>(A, bpr, 1, stream);
  }
  return rc;
}

int launch_wstream_group(int dtype, const void* const* w, float* const* y, const int* rows, int n, const void* x,
                         int bpr, void* stream) {
  if (n < 1 || n > 3 || bpr <= 0) return NRQ_LAUNCH_BAD_ARG;
  for (int i = 0; i < n; i++)
    if (rows[i] <= 0) return NRQ_LAUNCH_BAD_ARG;
  if (dtype == kQ8_0) return launch_ws_group<kQ8_0>(w, y, rows, n, x, bpr, stream);
  if (dtype == kQ4K) return launch_ws_group<kQ4K>(w, y, rows, n, x, bpr, stream);
  if (dtype == kQ6K) return launch_ws_group<kQ6K>(w, y, rows, n, x, bpr, stream);
  return NRQ_LAUNCH_BAD_ARG;
}

int launch_wstream_scalar(int dtype, const MatvecLaunch& L) {
  if (L.rows <= 0 || L.bpr <= 0) return 0;
  if (dtype == kQ8_0) return launch_ws<kQ8_0>(L);
  if (dtype == kQ4K) return launch_ws<kQ4K>(L);
  if (dtype == kQ6K) return launch_ws<kQ6K>(L);
  return NRQ_LAUNCH_BAD_ARG;
}

}  // namespace nrq
