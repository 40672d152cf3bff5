// Decode matvec, scalar f32 order: HBM -> LDS streaming with asynchronous
// direct-to-LDS loads. Bit-identical to the reference's scalar kernels
//   dot_q8_scalar  (crates/nr-tensor/src/kernels.rs:72-82)
//   dot_q4k_scalar (crates/nr-tensor/src/kquant.rs:192-218)
//   dot_q6k_scalar (crates/nr-tensor/src/kquant.rs:220-250)
// inside the row loops of matvec_q8 (kernels.rs:36-70) and kquant_matvec!
// (kquant.rs:536-564).
//
// Work split. Workgroup g owns rows [g*R, g*R + R); their blocks are one
// contiguous byte range of W, cut into tiles of up to TB whole blocks (one
// 16-byte-aligned window of at most NI*4 KiB each). Tiles stream through NS
// LDS stages with global_load_lds_dwordx4: every wave instruction moves 1 KiB
// of consecutive HBM straight into LDS, no VGPRs involved, and up to NS-1
// tiles are in flight while one is computed. Completion is tracked with
// explicit s_waitcnt vmcnt(n) (loads retire in order) and raw s_barrier, so
// a barrier never drains the loads still in flight.
//
// Compute. Phase 1 (per tile): each (row, block) contribution, formed
// exactly as the reference forms it — exact integer sub-dots with v_dot4,
// then its f32 steps: Q8_0 one lane per block; Q4_K / Q6_K one lane quad per
// block with partial sums joined by quad_perm DPP. Contributions go to LDS
// u[b*R + r]. Phase 2 (after the last tile): one lane per row adds its
// contributions in block order, the reference's `sumf +=` chain.
//
// The activation is staged once per workgroup in padded LDS layouts that put
// the 8 lanes served together by a 16-byte LDS read on 8 distinct bank groups.
#include "nrq_device.h"
#include "nrq_launch.h"

namespace nrq {

namespace {

template <int K>
__device__ __forceinline__ int qbcast(int v) {  // lane K of this quad
  return __builtin_amdgcn_mov_dpp(v, K * 0x55, 0xF, 0xF, false);
}

__device__ __forceinline__ int qsum(int v) {
  v += __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);  // quad_perm(1,0,3,2)
  v += __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);  // quad_perm(2,3,0,1)
  return v;
}

// 16 bytes per lane from global `g` into LDS at m0 + 16*lane.
__device__ __forceinline__ void dma16(const void* g, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" : : "s"(m0), "v"(g) : "memory");
}

// s_waitcnt vmcnt(N) leaving expcnt and lgkmcnt unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0x7f | (0 << 8) | (3 << 14)); }

// Workgroup barrier that orders LDS only: every wave's LDS operations are
// complete, outstanding global loads are left running.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  wait_lgkm0();
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)p;
}

// Activation layouts in LDS, dwords per block:
//   Q8_0 : [qs 8][d][pad 3]                                                  12
//   Q4_K : chunk c at 40c: [qs 16 (x elements 64c..64c+64)][bsum pair 2c][pair 2c+1];
//          d at 160; stride 164 (= 4 mod 32)                                  164
//   Q6_K : half h at 40h: [qs 32]; group corrections -32*sum16 at 80+g; d at 96;
//          stride 112 (= 16 mod 32)                                           112
template <int FMT>
__host__ __device__ constexpr int xs_stride() {
  return FMT == kQ8_0 ? 12 : (FMT == kQ4K ? 164 : 112);
}
template <int FMT>
__host__ __device__ constexpr int wbytes() {
  return FMT == kQ8_0 ? kQ8_0Bytes : (FMT == kQ4K ? kQ4KBytes : kQ6KBytes);
}
template <int FMT>
__host__ __device__ constexpr int xbytes() {
  return FMT == kQ8_0 ? kQ8_0Bytes : kQ8KBytes;
}

// Repacks the raw activation (already in LDS, `xskew` bytes into `raw`) into
// the padded layout.
template <int FMT, int NT>
__device__ void repack_act(const uint32_t* raw, uint32_t xskew, int bpr, uint32_t* xl) {
  const int tid = threadIdx.x;
  constexpr int XS = xs_stride<FMT>();
  if constexpr (FMT == kQ8_0) {
    const uint8_t* rb = (const uint8_t*)raw;
    for (int i = tid; i < bpr * 9; i += NT) {
      int b = i / 9, t = i - b * 9;
      uint32_t o = xskew + (uint32_t)b * kQ8_0Bytes;
      if (t < 8) xl[b * XS + t] = lds_u32_even(raw, o + 2 + 4 * t);
      else xl[b * XS + 8] = __float_as_uint(f16_bits_to_f32(lds_u16(rb, o)));
    }
  } else {
    // Q8_K block = 73 dwords: d @0, qs @1..64, bsums @65..72 (xskew is a multiple of 4).
    const uint32_t* rw = raw + (xskew >> 2);
    for (int i = tid; i < bpr * 64; i += NT) {
      int b = i >> 6, t = i & 63;
      uint32_t v = rw[b * 73 + 1 + t];
      if constexpr (FMT == kQ4K) xl[b * XS + (t >> 4) * 40 + (t & 15)] = v;
      else xl[b * XS + (t >> 5) * 40 + (t & 31)] = v;
    }
    for (int i = tid; i < bpr * 16; i += NT) {
      int b = i >> 4, g = i & 15;
      if constexpr (FMT == kQ4K) {
        if (g < 8) {  // bsums[2g] + bsums[2g+1]: sub-block g, stored beside chunk g/2
          uint32_t v = rw[b * 73 + 65 + g];
          int s = (int)(int16_t)(v & 0xffffu) + (int)(int16_t)(v >> 16);
          xl[b * XS + (g >> 1) * 40 + 16 + (g & 1)] = (uint32_t)s;
        } else if (g == 8) {
          xl[b * XS + 160] = rw[b * 73];
        }
      } else {
        // -32 * (sum of the group's 16 quants): the (q - 32) term of the scalar dot
        int s = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) s = sdot4(rw[b * 73 + 1 + 4 * g + k], 0xe0e0e0e0u, s);
        xl[b * XS + 80 + g] = (uint32_t)s;
        if (g == 0) xl[b * XS + 96] = rw[b * 73];
      }
    }
  }
}

// ---- per-block contributions from an LDS stage --------------------------------------

// Q8_0, one lane per block at even LDS byte offset o: (f32(acc) * dw) * dx
// (kernels.rs:75-79).
__device__ __forceinline__ float q80_contrib(const uint32_t* w32, uint32_t o, const uint32_t* xb) {
  const uint32_t q0 = o + 2, base = q0 >> 2, sh = q0 & 3u;
  uint32_t D[9];
#pragma unroll
  for (int t = 0; t < 9; t++) D[t] = w32[base + t];
  int acc = 0;
#pragma unroll
  for (int t = 0; t < 8; t++) acc = sdot4(__builtin_amdgcn_alignbyte(D[t + 1], D[t], sh), xb[t], acc);
  const uint32_t dbits = (o & 2) ? (w32[o >> 2] >> 16) : (w32[o >> 2] & 0xffffu);
  const float t1 = (float)acc * f16_bits_to_f32(dbits);
  return t1 * __uint_as_float(xb[8]);
}

// Q4_K, quad lane c at 16-byte-aligned LDS byte offset o: lane c owns qs chunk c
// (sub-blocks 2c, 2c+1). Returns d_all*sum_q - dmin_all*f32(sum_m)
// (kquant.rs:195-215) in every lane of the quad.
__device__ __forceinline__ float q4k_contrib(const uint8_t* lds_w, uint32_t o, int c, const uint32_t* xb) {
  const u32x4 h = *(const u32x4*)(lds_w + o);
  const u32x4 qa = *(const u32x4*)(lds_w + o + 16 + 32 * c);
  const u32x4 qb = *(const u32x4*)(lds_w + o + 32 + 32 * c);
  const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
  const uint32_t* xc = xb + 40 * c;
  int lo = 0, hi = 0;
#pragma unroll
  for (int t = 0; t < 8; t++) {
    lo = sdot4(q[t] & 0x0f0f0f0fu, xc[t], lo);
    hi = sdot4((q[t] >> 4) & 0x0f0f0f0fu, xc[8 + t], hi);
  }
  int sc[8], mn[8];
  q4k_unpack_scales(h.y, h.z, h.w, sc, mn);
  const int sl = c == 0 ? sc[0] : c == 1 ? sc[2] : c == 2 ? sc[4] : sc[6];
  const int sh = c == 0 ? sc[1] : c == 1 ? sc[3] : c == 2 ? sc[5] : sc[7];
  const int ml = c == 0 ? mn[0] : c == 1 ? mn[2] : c == 2 ? mn[4] : mn[6];
  const int mh = c == 0 ? mn[1] : c == 1 ? mn[3] : c == 2 ? mn[5] : mn[7];
  // f32(sc) * f32(sub) == f32(sc * sub): |sc * sub| <= 63 * 61440 < 2^24
  const int tl = sl * lo, th = sh * hi;
  const int sum_m = qsum(ml * (int)xc[16] + mh * (int)xc[17]);
  const int T[8] = {qbcast<0>(tl), qbcast<0>(th), qbcast<1>(tl), qbcast<1>(th),
                    qbcast<2>(tl), qbcast<2>(th), qbcast<3>(tl), qbcast<3>(th)};
  float sum_q = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; j++) sum_q = sum_q + (float)T[j];
  const float xd = __uint_as_float(xb[160]);
  const float d_all = f16_bits_to_f32(h.x & 0xffffu) * xd;
  const float dmin_all = f16_bits_to_f32(h.x >> 16) * xd;
  const float a = d_all * sum_q;
  const float m = dmin_all * (float)sum_m;
  return a - m;
}

// Q6_K, quad lane c = (half hh, parity u) at even LDS byte offset o: the lane owns
// the 16 quants of groups 8hh+2n+u (n = 0..3). Returns d_all * sum
// (kquant.rs:223-247) in every lane of the quad.
__device__ __forceinline__ float q6k_contrib(const uint32_t* w32, uint32_t o, int hh, int u, const uint32_t* xb) {
  const uint32_t sh = o & 3u;
  const uint32_t ba = (o >> 2) + 16 * hh + 4 * u;      // ql[64hh+16u ..]
  const uint32_t bb = ba + 8;                           // ql[64hh+32+16u ..]
  const uint32_t bh = (o >> 2) + 32 + 8 * hh + 4 * u;  // qh[32hh+16u ..]
  uint32_t A[5], B[5], H[5];
#pragma unroll
  for (int t = 0; t < 5; t++) {
    A[t] = w32[ba + t];
    B[t] = w32[bb + t];
    H[t] = w32[bh + t];
  }
  const uint32_t* xh = xb + 40 * hh;
  int gs[4];
#pragma unroll
  for (int n = 0; n < 4; n++) gs[n] = (int)xb[80 + 8 * hh + 2 * n + u];
#pragma unroll
  for (int t = 0; t < 4; t++) {
    uint32_t q6[4];
    q6k_planes(__builtin_amdgcn_alignbyte(A[t + 1], A[t], sh), __builtin_amdgcn_alignbyte(B[t + 1], B[t], sh),
               __builtin_amdgcn_alignbyte(H[t + 1], H[t], sh), q6);
#pragma unroll
    for (int n = 0; n < 4; n++) gs[n] = sdot4(q6[n], xh[8 * n + 4 * u + t], gs[n]);
  }
  const uint32_t bs = (o >> 2) + 48 + 2 * hh;  // scales[8hh ..]
  const uint32_t s0 = __builtin_amdgcn_alignbyte(w32[bs + 1], w32[bs], sh);
  const uint32_t s1 = __builtin_amdgcn_alignbyte(w32[bs + 2], w32[bs + 1], sh);
  // f32(sc) * f32(gs) == f32(sc * gs): |sc * gs| <= 128 * 65536 < 2^24
  int T[4];
  T[0] = (int)(int8_t)((s0 >> (8 * u)) & 0xffu) * gs[0];
  T[1] = (int)(int8_t)((s0 >> (8 * u + 16)) & 0xffu) * gs[1];
  T[2] = (int)(int8_t)((s1 >> (8 * u)) & 0xffu) * gs[2];
  T[3] = (int)(int8_t)((s1 >> (8 * u + 16)) & 0xffu) * gs[3];
  // group g = 8h + 2n + u lives in lane 2h + u, slot n: add in g order
  float sum = 0.0f;
#pragma unroll
  for (int n = 0; n < 4; n++) {
    sum = sum + (float)qbcast<0>(T[n]);
    sum = sum + (float)qbcast<1>(T[n]);
  }
#pragma unroll
  for (int n = 0; n < 4; n++) {
    sum = sum + (float)qbcast<2>(T[n]);
    sum = sum + (float)qbcast<3>(T[n]);
  }
  const uint32_t dw = w32[(o + 208) >> 2];
  const uint32_t dbits = ((o + 208) & 2) ? (dw >> 16) : (dw & 0xffffu);
  const float d_all = f16_bits_to_f32(dbits) * __uint_as_float(xb[96]);
  return d_all * sum;
}

}  // namespace

// ---- the kernel ------------------------------------------------------------------------

constexpr int kStreamNT = 256;  // 4 waves
constexpr int kStreamNS = 4;    // LDS stages: up to 3 tiles in flight
constexpr int kStreamNI = 3;    // 4 KiB wave-group loads per tile: 12 KiB tiles

template <int FMT>
__host__ __device__ constexpr int tile_blocks() {  // whole blocks per tile window
  return (kStreamNI * 4096 - 30) / wbytes<FMT>();
}

template <int FMT>
__global__ __launch_bounds__(kStreamNT) void stream_matvec(const uint8_t* __restrict__ W,
                                                           const uint8_t* __restrict__ X, float* __restrict__ Y,
                                                           int rows, int bpr, int R, int nstages) {
  constexpr int NT = kStreamNT, NS = kStreamNS, NI = kStreamNI, XS = xs_stride<FMT>(), BS = wbytes<FMT>();
  constexpr int TB = tile_blocks<FMT>(), STAGE = NI * 4096;
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int r0 = blockIdx.x * R;
  const int nr = min(R, rows - r0);
  const int nb = nr * bpr;
  const size_t fbeg = (size_t)r0 * bpr;  // first flat block of this workgroup
  const int ntiles = (nb + TB - 1) / TB;

  uint32_t* xl = (uint32_t*)smem;
  uint8_t* stages = smem + ((bpr * XS * 4 + 15) & ~15);
  // u[b * R + r]; first the activation scratch. A workgroup whose rows span
  // fewer than NS tiles gets only that many stages (tile t always uses stage t).
  float* u = (float*)(stages + nstages * STAGE);
  const uint32_t stage0 = lds_addr(stages);

  // Tile t: flat blocks [fbeg + t*TB, ...) -> 16-byte window [a0, a0 + 16*n16).
  auto issue = [&](int t) {
    const size_t fb0 = fbeg + (size_t)t * TB;
    const size_t fb1 = fbeg + (size_t)min(nb, (t + 1) * TB);
    const size_t a0 = (fb0 * BS) & ~(size_t)15;
    const int n16 = (int)((((fb1 * BS) + 15) & ~(size_t)15) - a0) >> 4;
    const uint32_t sbase = stage0 + (uint32_t)((t % NS) * STAGE);
#pragma unroll
    for (int k = 0; k < NI; k++) {
      const int grp = 4 * k + wave;
      const int ci = min(grp * 64 + lane, n16 - 1);  // past the window: reload its last chunk
      dma16(W + a0 + 16 * (size_t)ci, sbase + (uint32_t)grp * 1024u);
    }
  };

  // Activation: its 16-byte window goes to the u region by the same DMA, issued
  // first so that its completion is implied by an in-order vmcnt below.
  {
    const uintptr_t xa = (uintptr_t)X;
    const uintptr_t xa0 = xa & ~(uintptr_t)15;
    const int n16x = (int)((((xa + (size_t)bpr * xbytes<FMT>()) + 15) & ~(uintptr_t)15) - xa0) >> 4;
    const uint32_t ubase = lds_addr(u);
    for (int grp = wave; grp * 64 < n16x; grp += 4) {
      const int ci = min(grp * 64 + lane, n16x - 1);
      dma16((const uint8_t*)xa0 + 16 * (size_t)ci, ubase + (uint32_t)grp * 1024u);
    }
  }
  const int pro = min(NS - 1, ntiles);
#pragma unroll
  for (int t = 0; t < NS - 1; t++)
    if (t < ntiles) issue(t);
  // the activation landed once at most `pro` tiles' loads are outstanding
  if (pro >= 3) wait_vm<3 * NI>();
  else if (pro == 2) wait_vm<2 * NI>();
  else if (pro == 1) wait_vm<NI>();
  else wait_vm<0>();
  lds_barrier();
  repack_act<FMT, NT>((const uint32_t*)u, (uint32_t)((uintptr_t)X & 15), bpr, xl);
  lds_barrier();

  for (int t = 0; t < ntiles; t++) {
    const int after = min(NS - 2, ntiles - 1 - t);  // tiles this wave issued after t
    if (after >= 2) wait_vm<2 * NI>();
    else if (after == 1) wait_vm<NI>();
    else wait_vm<0>();
    lds_barrier();
    if (t + NS - 1 < ntiles) issue(t + NS - 1);

    const uint8_t* cur = stages + (t % NS) * STAGE;
    const int tb0 = t * TB;  // first block of the tile, relative to fbeg
    const int items = min(nb - tb0, TB);
    const uint32_t skew = (uint32_t)(((fbeg + tb0) * BS) & 15);
    if constexpr (FMT == kQ8_0) {
      for (int i = tid; i < items; i += NT) {
        const int f = tb0 + i, r = f / bpr, b = f - r * bpr;
        u[b * R + r] = q80_contrib((const uint32_t*)cur, skew + (uint32_t)i * BS, xl + b * XS);
      }
    } else {
      const int q = tid >> 2, c = tid & 3;
      for (int i0 = 0; i0 < items; i0 += NT / 4) {
        const int i = min(i0 + q, items - 1);  // whole quads stay active for the DPP
        const int f = tb0 + i, r = f / bpr, b = f - r * bpr;
        const uint32_t o = skew + (uint32_t)i * BS;
        float cb;
        if constexpr (FMT == kQ4K) cb = q4k_contrib(cur, o, c, xl + b * XS);
        else cb = q6k_contrib((const uint32_t*)cur, o, c >> 1, c & 1, xl + b * XS);
        if (c == 0 && i0 + q < items) u[b * R + r] = cb;
      }
    }
  }
  lds_barrier();
  // phase 2: the reference's `sumf += contribution` chain, block order
  for (int r = tid; r < nr; r += NT) {
    float s = 0.0f;
    for (int b = 0; b < bpr; b++) s = s + u[b * R + r];
    Y[r0 + r] = s;
  }
}

// ---- launch ---------------------------------------------------------------------------------

template <int FMT>
static int launch_stream_t(const MatvecLaunch& L, int num_cus) {
  constexpr int XS = xs_stride<FMT>(), TB = tile_blocks<FMT>();
  constexpr size_t STAGE = (size_t)kStreamNI * 4096;
  const int bpr = L.bpr;
  const size_t xl = ((size_t)bpr * XS * 4 + 15) & ~(size_t)15;
  // activation window as the DMA writes it: whole KiB per wave instruction
  const size_t raw = ((size_t)bpr * xbytes<FMT>() + 15 + 15 + 1023) & ~(size_t)1023;
  // Rows per workgroup: about four workgroups per CU, within an LDS budget
  // that keeps them resident.
  int R = (L.rows + 4 * num_cus - 1) / (4 * num_cus);
  if (L.tile_rows > 0) R = L.tile_rows;
  if (R < 1) R = 1;
  auto nstages_for = [&](int r) {
    const long tiles = ((long)r * bpr + TB - 1) / TB;
    return (int)(tiles < kStreamNS ? tiles : kStreamNS);
  };
  auto lds_for = [&](int r) {
    const size_t ub = (size_t)r * bpr * 4;
    return xl + (size_t)nstages_for(r) * STAGE + (ub > raw ? ub : raw);
  };
  while (R > 1 && lds_for(R) > 80 * 1024) R--;
  const size_t lds = lds_for(R);
  const int nstages = nstages_for(R);
  if (lds > 160 * 1024) return NRQ_LAUNCH_TOO_WIDE;
  const int grid = (L.rows + R - 1) / R;
  hipLaunchKernelGGL(stream_matvec<FMT>, dim3(grid), dim3(kStreamNT), lds, (hipStream_t)L.stream,
                     (const uint8_t*)L.w, (const uint8_t*)L.x, L.y, L.rows, bpr, R, nstages);
  return hipGetLastError() == hipSuccess ? 0 : NRQ_LAUNCH_FAILED;
}

int launch_stream_scalar(int dtype, const MatvecLaunch& L) {
  if (L.rows <= 0 || L.bpr <= 0) return 0;
  static int num_cus = 0;
  if (num_cus == 0) {
    int dev = 0;
    int n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      num_cus = n;
    else
      num_cus = 256;
  }
  if (dtype == kQ8_0) return launch_stream_t<kQ8_0>(L, num_cus);
  if (dtype == kQ4K) return launch_stream_t<kQ4K>(L, num_cus);
  if (dtype == kQ6K) return launch_stream_t<kQ6K>(L, num_cus);
  return NRQ_LAUNCH_BAD_ARG;
}

}  // namespace nrq
