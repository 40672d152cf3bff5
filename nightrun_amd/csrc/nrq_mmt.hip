// Batched prefill matmul on int8 MFMA, in the reference's scalar f32 order:
//   Q4_K x Q8_K: dot_q4k_scalar (crates/nr-tensor/src/kquant.rs:192-218)
//   Q6_K x Q8_K: dot_q6k_scalar (crates/nr-tensor/src/kquant.rs:220-250)
//   Q8_0 x Q8_0: dot_q8_scalar (crates/nr-tensor/src/kernels.rs:72-82)
// so y[t][r] equals the per-token matvec bit for bit, as kquant_matmul! and
// matmul_q8 guarantee (kquant.rs:566-639, kernels.rs:91-143).
//
// Tiles. A wave owns 32 weight rows x 32 tokens (32x32 int8 MFMA: lane l holds
// row l % 32 and 16 tokens, so a row's scales stay in one lane and one
// unpacked weight operand serves 16 outputs per lane). A workgroup is KS waves
// over the same tile, splitting its blocks: in round k, wave s takes block
// KS*k + s. With KS = 1 the reference's `sumf +=` chain runs in registers; with
// KS > 1 each wave writes its round's contributions to LDS and, after the next
// round's barrier, the wave that owns an element adds the KS contributions in
// block order.
//
// Loads, one block ahead of use (from a second register buffer, or into the
// current one once its operands are consumed). Weights: each lane reads its
// row's bytes for its MFMA K positions straight into registers. K-quant
// activations: the wave reads its 32 tokens' Q8_K blocks as consecutive
// 16-byte windows (about three whole blocks per load instruction, where one
// 16-byte operand per lane would touch 32 tokens' lines) and writes them to
// its LDS stage, from where each lane reads its operands: 16 bytes per Q4_K
// sub-block, one v_mfma_i32_32x32x32_i8 step, or 8 bytes per Q6_K group, one
// v_mfma_i32_32x32x16_i8 step. A and B take the same K positions per lane
// half, so a step sums exactly the sub-block's (group's) products. The token
// values the f32 steps need per output element (d) pass through a small
// per-wave LDS table, from the lane that read the token to the lanes that
// hold its outputs.
//
// f32 steps. Q4_K's sum_q += f32(sc_j) * f32(sub_j): each product is an
// integer below 63 * 61440 < 2^22, so the first four partial sums are exact
// integers below 2^24 and are formed on the 24-bit integer multiplier; the
// remaining four steps are f32 (fmaf with an exact product rounds like the
// reference's multiply-then-add). sum_m = sum of m_{k/2} * bsums[k] is two
// more MFMA steps (the bsums split exactly into low 7 bits and a signed high
// part). Q6_K: sum += f32(sc) * f32(gs) in group
// order, gs = sum((q - 32) * q8) from one MFMA step per 16-quant group.
// Q8_0: a 32-value block is two MFMA steps (lane half kg takes bytes
// 16kg .. +16 of both operands), then sum += (f32(acc) * dw) * dx.
#include "nrq_device.h"
#include "nrq_launch.h"

#include <stdio.h>
#include <stdlib.h>

namespace nrq {

namespace {

typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x3a __attribute__((ext_vector_type(3), aligned(4)));
typedef uint32_t u32x2a __attribute__((ext_vector_type(2), aligned(4)));

__device__ __forceinline__ i32x16 md_mfma(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1, i32x16 c) {
  const long a = (long)(((uint64_t)a1 << 32) | a0);
  const long b = (long)(((uint64_t)b1 << 32) | b0);
  return __builtin_amdgcn_mfma_i32_32x32x16_i8(a, b, c, 0, 0, 0);
}

// One 32-value Q4_K sub-block per step (gfx950 v_mfma_i32_32x32x32_i8): lane
// half kg supplies the same 16 K positions of both operands, so the step sums
// exactly the sub-block's 32 products.
typedef int i32x4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x16 md_mfma32(const u32x4& a, uint32_t b0, uint32_t b1, uint32_t b2, uint32_t b3,
                                            i32x16 c) {
  const i32x4v av = {(int)a.x, (int)a.y, (int)a.z, (int)a.w};
  const i32x4v bv = {(int)b0, (int)b1, (int)b2, (int)b3};
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, c, 0, 0, 0);
}

__device__ __forceinline__ void md_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x7f | (0 << 8) | (3 << 14));  // this wave's LDS accesses are done
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// `v`, ordered after all 16 values of `dep` are computed. MFMA steps have no
// side effects, so the compiler would otherwise issue a block's steps far
// ahead of the f32 chains that consume them and hold every result (16
// registers each); tying each step's operand to the chains of two steps back
// keeps two results live.
__device__ __forceinline__ uint32_t md_after(uint32_t v, const float dep[16]) {
  asm volatile("" : "+v"(v) : "v"(dep[0]), "v"(dep[1]), "v"(dep[2]), "v"(dep[3]), "v"(dep[4]), "v"(dep[5]),
               "v"(dep[6]), "v"(dep[7]), "v"(dep[8]), "v"(dep[9]), "v"(dep[10]), "v"(dep[11]), "v"(dep[12]),
               "v"(dep[13]), "v"(dep[14]), "v"(dep[15]));
  return v;
}

// (q - 32) as int8 for four 6-bit quants whose bit 5 is already inverted
// (q ^ 32, so bit 5 set means negative): (v + 0x60) ^ 0x60 copies bit 5 into
// bits 6-7, with no carry between bytes.
__device__ __forceinline__ uint32_t md_q6_signed(uint32_t v) { return (v + 0x60606060u) ^ 0x60606060u; }

// Per-wave table of the tile's 32 token values (dword 128 + t: d of token t).
constexpr int kMdScalDw = 160;

// Registers one block needs, loaded one block ahead of use.
template <int FMT>
struct MdLoad;
// K-quant activation tiles move as 16-byte windows: 19 per token (qs in 16,
// then bsums in 2, then one holding d), window i of lane l being number
// 64i + l of the tile's 32 x 19, so that each load instruction reads about
// three whole token blocks. The wave writes them to its LDS stage in the same
// order (token t at 304t: qs at +0, bsums at +256, d at +288), from where
// every lane reads its MFMA operands.
constexpr int kMdWin = 19, kMdTokB = 16 * kMdWin, kMdStage = 32 * kMdTokB;
constexpr int kMdXi = (32 * kMdWin + 63) / 64;  // window loads per lane (10)

template <>
struct MdLoad<kQ4K> {
  u32x4a x[kMdXi];  // activation windows
  u32x4 h;          // weight header: d | dmin, scales[12]
  u32x4 q[4];       // qs bytes 32cc + 16kg .. +16
};
template <>
struct MdLoad<kQ8_0> {
  // per operand: an aligned 16-byte window at or just before this lane's 16
  // qs bytes, the 2 bytes after it, and the dword holding the block's d
  u32x4 a;
  uint32_t a4, ad, ao;  // ao: byte offsets (bits 0-1: qs window, bits 2-3: d)
  u32x4 w;
  uint32_t w4, wd, wo;
};
template <>
struct MdLoad<kQ6K> {
  u32x4a x[kMdXi];  // activation windows, as for Q4_K
  u32x3a w[12];  // aligned 12-byte windows [hh][u][ql low planes, ql high planes, qh]
  u32x4a s;      // aligned window over scales[16] ...
  uint32_t s4;   // ... and d
};

// xb: Q8_0 — this lane's token's block; K-quants — the tile's block column
// (its first token's block), with xo the lane's window offsets from it.
template <int FMT>
__device__ __forceinline__ void md_load(MdLoad<FMT>& L, const uint8_t* __restrict__ xb, const uint8_t* __restrict__ wb,
                                        int kg, const uint32_t* xo);

__device__ __forceinline__ void md_load_windows(u32x4a (&x)[kMdXi], const uint8_t* __restrict__ xb,
                                                const uint32_t* xo) {
#pragma unroll
  for (int i = 0; i < kMdXi; i++) x[i] = *(const u32x4a*)(xb + xo[i]);
}

// The lane's windows into the wave's stage (the last load's upper half-wave
// holds repeats and is not written).
// Lanes then read windows other lanes wrote: the wave's LDS accesses run in
// program order, and the compiler barriers keep that order in the code (the
// previous block's reads before these writes, these writes before the reads).
__device__ __forceinline__ void md_stage(const u32x4a (&x)[kMdXi], uint8_t* stg, int lane) {
  asm volatile("" ::: "memory");
#pragma unroll
  for (int i = 0; i < kMdXi; i++) {
    const int idx = 64 * i + lane;
    if (i < kMdXi - 1 || idx < 32 * kMdWin) *(u32x4*)(stg + 16 * idx) = (u32x4)x[i];
  }
  asm volatile("" ::: "memory");
}

// Byte offsets of the lane's windows from the tile's block column: token
// min(t, last) of the tile, window c of its block.
__device__ __forceinline__ void md_window_offsets(uint32_t* xo, int lane, int last, int bpr) {
#pragma unroll
  for (int i = 0; i < kMdXi; i++) {
    int idx = 64 * i + lane;
    if (idx >= 32 * kMdWin) idx -= 32;
    const int t = idx / kMdWin, c = idx - t * kMdWin;
    const uint32_t off = c < 16 ? 4u + 16u * (uint32_t)c : c == 16 ? 260u : c == 17 ? 276u : 0u;
    xo[i] = (uint32_t)min(t, last) * (uint32_t)bpr * (uint32_t)kQ8KBytes + off;
  }
}

template <>
__device__ __forceinline__ void md_load<kQ4K>(MdLoad<kQ4K>& L, const uint8_t* __restrict__ xb,
                                              const uint8_t* __restrict__ wb, int kg, const uint32_t* xo) {
  md_load_windows(L.x, xb, xo);
  L.h = *(const u32x4*)wb;
#pragma unroll
  for (int cc = 0; cc < 4; cc++) L.q[cc] = *(const u32x4*)(wb + 16 + 32 * cc + 16 * kg);
}

// A Q8_0 block (34 bytes, 2-byte aligned) as whole dwords that never leave it,
// except the d dword of a block starting 2 bytes past a dword, which begins 2
// bytes before it (such a block is never a buffer's first, the buffers being
// 4-byte aligned). qs bytes 16kg .. +16 start at p = (2 + 16kg + block) & 3 past
// an aligned window V; with p = 2 the last two bytes follow V.
__device__ __forceinline__ void md_q8_window(const uint8_t* __restrict__ blk, int kg, u32x4& v, uint32_t& v4,
                                             uint32_t& d, uint32_t& off) {
  const uint8_t* q = blk + 2 + 16 * kg;
  const uint32_t p = (uint32_t)((uintptr_t)q & 3u);
  const uint8_t* a = q - p;
  v = *(const u32x4*)a;
  v4 = *(const uint16_t*)(a + (p ? 16 : 14));  // p = 0: an in-block halfword, unused
  const uint32_t pd = (uint32_t)((uintptr_t)blk & 3u);
  d = *(const uint32_t*)(blk - pd);
  off = p | (pd << 2);
}

// A Q8_0 block's window, as md_q8_window, from a copy of its row in LDS whose
// start keeps the row's alignment mod 16 (reads of 4-byte alignment only).
__device__ __forceinline__ void md_q8_window_lds(const uint8_t* blk, int kg, u32x4& v, uint32_t& v4, uint32_t& d,
                                                 uint32_t& off) {
  const uint8_t* q = blk + 2 + 16 * kg;
  const uint32_t p = (uint32_t)((uintptr_t)q & 3u);
  const uint8_t* a = q - p;
  v = (u32x4)(*(const u32x4a*)a);
  v4 = *(const uint16_t*)(a + (p ? 16 : 14));
  const uint32_t pd = (uint32_t)((uintptr_t)blk & 3u);
  d = *(const uint32_t*)(blk - pd);
  off = p | (pd << 2);
}

// Q8_0 spans: 8 blocks of a row, 272 bytes, 17 aligned 16-byte windows when
// rows are 8-block multiples on 16-byte aligned bases. A tile's span is 32 x 17
// windows per operand, window i of the tile being row i / 17, piece i % 17.
constexpr int kMdSpanB = 8 * 34, kMdSpanWin = 17, kMdSpanLd = (32 * kMdSpanWin + 63) / 64;  // 9 loads per lane

template <>
__device__ __forceinline__ void md_load<kQ8_0>(MdLoad<kQ8_0>& L, const uint8_t* __restrict__ xb,
                                               const uint8_t* __restrict__ wb, int kg, const uint32_t* xo) {
  (void)xo;
  md_q8_window(xb, kg, L.a, L.a4, L.ad, L.ao);
  md_q8_window(wb, kg, L.w, L.w4, L.wd, L.wo);
}

// Q6_K loads by half: half 0 = groups 0-7 and their weights, plus d and the
// scales (read at the block's start); half 1 = groups 8-15.
__device__ __forceinline__ void md_load_q6k_half(MdLoad<kQ6K>& L, const uint8_t* __restrict__ xb,
                                                 const uint8_t* __restrict__ wb, int kg, int hh, const uint32_t* xo,
                                                 bool windows = true) {
  if (hh == 0 && windows) md_load_windows(L.x, xb, xo);
  const uint8_t* w4 = wb - ((uintptr_t)wb & 3u);  // the block is 2-byte aligned
#pragma unroll
  for (int u = 0; u < 2; u++) {
    const int l0 = 16 * u + 8 * kg;
    L.w[6 * hh + 3 * u + 0] = *(const u32x3a*)(w4 + 64 * hh + l0);        // ql[64hh + l]: planes 0, 2
    L.w[6 * hh + 3 * u + 1] = *(const u32x3a*)(w4 + 64 * hh + 32 + l0);   // ql[64hh + 32 + l]: planes 1, 3
    L.w[6 * hh + 3 * u + 2] = *(const u32x3a*)(w4 + 128 + 32 * hh + l0);  // qh[32hh + l]
  }
  if (hh == 0) {
    L.s = *(const u32x4a*)(w4 + 192);
    L.s4 = *(const uint32_t*)(w4 + 208);
  }
}

template <>
__device__ __forceinline__ void md_load<kQ6K>(MdLoad<kQ6K>& L, const uint8_t* __restrict__ xb,
                                              const uint8_t* __restrict__ wb, int kg, const uint32_t* xo) {
  md_load_q6k_half(L, xb, wb, kg, 0, xo);
  md_load_q6k_half(L, xb, wb, kg, 1, xo);
}

// Q4_K block: contributions c[e] of this lane's 16 outputs (row l % 32,
// tile tokens 8(e/4) + 4kg + e%4). `ta` is this lane's operand token.
// prefetch() runs once L is no longer read (it loads the next block into L).
template <typename PF, typename PX>
__device__ __forceinline__ void md_q4k(MdLoad<kQ4K>& L, uint8_t* stg, uint32_t* scal, int ta, int kg, float c[16],
                                       PF prefetch, PX prefetch_x) {
  md_stage(L.x, stg, ta + 32 * kg);
  prefetch_x();  // the windows are in the stage: the next block's may load into L.x now
  const uint8_t* at = stg + ta * kMdTokB;  // operand token ta in the stage
  if (kg == 0) scal[128 + ta] = *(const uint32_t*)(at + 288);  // token ta's d
  const u32x4 h = L.h;
  // kquant.rs:83-92, four scales or mins per word
  const uint32_t scA = h.y & 0x3f3f3f3fu, mnA = h.z & 0x3f3f3f3fu;
  const uint32_t scB = (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
  const uint32_t mnB = ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
  // kquant.rs:209-213: sum_m = sum_k m_{k/2} * bsums[k] over the 16 bsums, as two
  // MFMA steps (K = 16): lane half kg holds bsums 8kg .. 8kg+7 of token ta,
  // split exactly as bsum = 128 * hi + lo (lo = low 7 bits, hi in [-16, 15]),
  // against m_{4kg}, m_{4kg}, m_{4kg+1}, ... of row l % 32.
  // (the two steps issue after the sub-block loop, whose results they would otherwise sit beside)
  const u32x4 bsv = *(const u32x4*)(at + 256 + 16 * kg);
  const uint32_t sb0 = bsv.x, sb1 = bsv.y, sb2 = bsv.z, sb3 = bsv.w;
  const uint32_t mn = kg ? mnB : mnA;
  const float dw = f16_bits_to_f32(h.x & 0xffffu), dmw = f16_bits_to_f32(h.x >> 16);
  int S[16];
  float sq[16];
  auto sub_of = [&](int j, const float dep[16]) {
    const u32x4 q = L.q[j >> 1];
    const uint32_t sh = (j & 1) ? 4u : 0u;
    const uint32_t b0 = (q.x >> sh) & 0x0f0f0f0fu, b1 = (q.y >> sh) & 0x0f0f0f0fu;
    const uint32_t b2 = (q.z >> sh) & 0x0f0f0f0fu, b3 = (q.w >> sh) & 0x0f0f0f0fu;
    const i32x16 z = {};
    u32x4 a = *(const u32x4*)(at + 32 * j + 16 * kg);
    a.x = md_after(a.x, dep);
    return md_mfma32(a, b0, b1, b2, b3, z);
  };
  float dep[16];
#pragma unroll
  for (int e = 0; e < 16; e++) dep[e] = 0.0f;
  i32x16 nsub = sub_of(0, dep);
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const i32x16 sub = nsub;
    // the next sub-block's steps wait for this lane's chains after sub-block j - 1
    if (j >= 1) {
#pragma unroll
      for (int e = 0; e < 16; e++) dep[e] = j <= 4 ? __int_as_float(S[e]) : sq[e];
    }
    if (j + 1 < 8) nsub = sub_of(j + 1, dep);
    if (j < 4) {
      // kquant.rs:207, j = 0..3: exact integer partial sums (|sum| <= 4 * 63 * 61440 < 2^24)
      const int sc = (int)((scA >> (8 * j)) & 0xffu);
#pragma unroll
      for (int e = 0; e < 16; e++) S[e] = j == 0 ? __mul24(sc, sub[e]) : S[e] + __mul24(sc, sub[e]);
      if (j == 3) {
#pragma unroll
        for (int e = 0; e < 16; e++) sq[e] = (float)S[e];
      }
    } else {
      const float sc = (float)((scB >> (8 * (j - 4))) & 0xffu);
#pragma unroll
      for (int e = 0; e < 16; e++) sq[e] = fmaf(sc, (float)sub[e], sq[e]);  // j = 4..7, f32
    }
  }
  i32x16 smlo, smhi;
  {
    const uint32_t lo0 = md_after(__builtin_amdgcn_perm(sb1, sb0, 0x06040200u) & 0x7f7f7f7fu, sq);
    const uint32_t lo1 = __builtin_amdgcn_perm(sb3, sb2, 0x06040200u) & 0x7f7f7f7fu;
    const uint32_t hi0 = __builtin_amdgcn_perm((sb1 >> 7) & 0x00ff00ffu, (sb0 >> 7) & 0x00ff00ffu, 0x06040200u);
    const uint32_t hi1 = __builtin_amdgcn_perm((sb3 >> 7) & 0x00ff00ffu, (sb2 >> 7) & 0x00ff00ffu, 0x06040200u);
    const uint32_t m0 = __builtin_amdgcn_perm(mn, mn, 0x01010000u), m1 = __builtin_amdgcn_perm(mn, mn, 0x03030202u);
    const i32x16 z = {};
    smlo = md_mfma(lo0, lo1, m0, m1, z);
    smhi = md_mfma(md_after(hi0, sq), hi1, m0, m1, z);
  }
  prefetch();  // the block's operands are consumed: the next block's loads may reuse L
#pragma unroll
  for (int qq = 0; qq < 4; qq++) {
    const int t4 = 8 * qq + 4 * kg;  // tile tokens t4 .. t4 + 3
    const u32x4 XD = *(const u32x4*)(scal + 128 + t4);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int e = 4 * qq + i;
      const int sm = (int)(((uint32_t)smhi[e] << 7) + (uint32_t)smlo[e]);  // exact: |sum_m| < 2^22
      const float xd = __uint_as_float(XD[i]);
      const float d_all = dw * xd, dmin_all = dmw * xd;
      const float av = d_all * sq[e];
      const float mv = dmin_all * (float)sm;
      c[e] = av - mv;  // kquant.rs:215
    }
  }
}

// The 16 qs bytes of a Q8_0 window, realigned, and the block's d as f32.
__device__ __forceinline__ void md_q8_bytes(const u32x4& v, uint32_t v4, uint32_t d, uint32_t off, uint32_t q[4],
                                            float* df) {
  const uint32_t sh = off & 3u;
  q[0] = __builtin_amdgcn_alignbyte(v.y, v.x, sh);
  q[1] = __builtin_amdgcn_alignbyte(v.z, v.y, sh);
  q[2] = __builtin_amdgcn_alignbyte(v.w, v.z, sh);
  q[3] = __builtin_amdgcn_alignbyte(v4, v.w, sh);
  *df = f16_bits_to_f32((d >> (8u * (off >> 2))) & 0xffffu);
}

// Q8_0 block: kernels.rs:77-79, acc = integer dot; sum += (f32(acc) * dw) * dx.
template <typename PF>
__device__ __forceinline__ void md_q8(MdLoad<kQ8_0>& L, uint32_t* scal, int ta, int kg, float c[16], PF prefetch) {
  uint32_t xa[4], wq[4];
  float dx, dw;
  md_q8_bytes(L.a, L.a4, L.ad, L.ao, xa, &dx);
  md_q8_bytes(L.w, L.w4, L.wd, L.wo, wq, &dw);
  if (kg == 0) scal[128 + ta] = __float_as_uint(dx);  // token ta's d
  const i32x16 z = {};
  const i32x16 acc = md_mfma(xa[2], xa[3], wq[2], wq[3], md_mfma(xa[0], xa[1], wq[0], wq[1], z));
  prefetch();  // the block's operands are consumed
#pragma unroll
  for (int qq = 0; qq < 4; qq++) {
    const int t4 = 8 * qq + 4 * kg;  // tile tokens t4 .. t4 + 3
    const u32x4 XD = *(const u32x4*)(scal + 128 + t4);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float t1 = (float)acc[4 * qq + i] * dw;
      c[4 * qq + i] = t1 * __uint_as_float(XD[i]);
    }
  }
}

// Q6_K block, `sh` = its start's byte offset (0 or 2) past the aligned windows.
// prefetch(half) runs once that half of L is no longer read.
template <typename PF, typename PX>
__device__ __forceinline__ void md_q6k(MdLoad<kQ6K>& L, uint32_t sh, uint8_t* stg, uint32_t* scal, int ta, int kg,
                                       float c[16], PF prefetch, PX prefetch_x) {
  md_stage(L.x, stg, ta + 32 * kg);
  prefetch_x();  // the windows are in the stage: the next block's may load into L.x now
  const uint8_t* at = stg + ta * kMdTokB;  // operand token ta in the stage
  if (kg == 0) scal[128 + ta] = *(const uint32_t*)(at + 288);
  uint32_t S[4];  // scales[16], realigned
  {
    const uint32_t sw[5] = {L.s.x, L.s.y, L.s.z, L.s.w, L.s4};
#pragma unroll
    for (int t = 0; t < 4; t++) S[t] = __builtin_amdgcn_alignbyte(sw[t + 1], sw[t], sh);
  }
  const uint32_t dbits = sh ? (L.s4 >> 16) : (L.s4 & 0xffffu);
  const float dw = f16_bits_to_f32(dbits);
  float sum[16];
#pragma unroll
  for (int e = 0; e < 16; e++) sum[e] = 0.0f;
#pragma unroll
  for (int hh = 0; hh < 2; hh++) {
    // this half's ql and qh dwords for quants l = 16u + 8kg + 0..7, realigned;
    // qh ^ 0xaa inverts bit 5 of every quant (see md_q6_signed)
    uint32_t QA[2][2], QB[2][2], QH[2][2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const u32x3a wa = L.w[6 * hh + 3 * u], wb = L.w[6 * hh + 3 * u + 1], wq = L.w[6 * hh + 3 * u + 2];
      QA[u][0] = __builtin_amdgcn_alignbyte(wa.y, wa.x, sh);
      QA[u][1] = __builtin_amdgcn_alignbyte(wa.z, wa.y, sh);
      QB[u][0] = __builtin_amdgcn_alignbyte(wb.y, wb.x, sh);
      QB[u][1] = __builtin_amdgcn_alignbyte(wb.z, wb.y, sh);
      QH[u][0] = __builtin_amdgcn_alignbyte(wq.y, wq.x, sh) ^ 0xaaaaaaaau;
      QH[u][1] = __builtin_amdgcn_alignbyte(wq.z, wq.y, sh) ^ 0xaaaaaaaau;
    }
    // group G = 8hh + 2pn + u: (q - 32) of plane pn (kquant.rs:233-237), formed when its step issues
    auto step = [&](int g8, const float dep[16]) {
      const int pn = g8 >> 1, u = g8 & 1, G = 8 * hh + g8;
      uint32_t bq[2];
#pragma unroll
      for (int k = 0; k < 2; k++) {
        const uint32_t ql = (pn & 1) ? QB[u][k] : QA[u][k];
        const uint32_t lo = (pn >> 1) ? ((ql >> 4) & 0x0f0f0f0fu) : (ql & 0x0f0f0f0fu);
        const uint32_t hi = (pn == 0 ? (QH[u][k] << 4) : pn == 1 ? (QH[u][k] << 2) : pn == 2 ? QH[u][k] : (QH[u][k] >> 2)) &
                            0x30303030u;
        bq[k] = md_q6_signed(md_after(lo | hi, dep));
      }
      const i32x16 z = {};
      const uint2 a = *(const uint2*)(at + 16 * G + 8 * kg);
      return md_mfma(a.x, a.y, bq[0], bq[1], z);
    };
    i32x16 ngs = step(0, sum);
#pragma unroll
    for (int g8 = 0; g8 < 8; g8++) {
      const int G = 8 * hh + g8;  // kquant.rs:238-246: groups in order (g8 = 2pn + u)
      const i32x16 gs = ngs;
      if (g8 + 1 < 8) ngs = step(g8 + 1, sum);  // waits for this lane's chains after group G - 1
      const float sc = (float)(int)(int8_t)((S[G >> 2] >> (8 * (G & 3))) & 0xffu);
      // kquant.rs:244: sum += f32(sc) * f32(gs); |sc * gs| <= 128 * 65536, exact
#pragma unroll
      for (int e = 0; e < 16; e++) sum[e] = fmaf(sc, (float)gs[e], sum[e]);
    }
    prefetch(hh);
  }
#pragma unroll
  for (int qq = 0; qq < 4; qq++) {
    const u32x4 XD = *(const u32x4*)(scal + 128 + 8 * qq + 4 * kg);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float d_all = dw * __uint_as_float(XD[i]);
      c[4 * qq + i] = d_all * sum[4 * qq + i];  // kquant.rs:246-247
    }
  }
}

}  // namespace

// The matrices of one launch: up to three of one format and width that share
// the activation (q|k|v, gate|up), their row tiles laid end to end; matrix m
// owns row tiles tile0_m .. tile0_{m+1} - 1. Separate fields, selected with
// uniform conditions (an indexed array would live in private memory).
struct MdMats {
  const uint8_t *w0, *w1, *w2;
  float *y0, *y1, *y2;
  int rows0, rows1, rows2;
  int tile1, tile2;  // first row tile of matrices 1 and 2
};

// NB register buffers of block loads: NB = 1 reloads the one buffer as soon as
// its operands are consumed; NB = 2 or 4 is a ring whose loads run NB - 1
// rounds ahead of the block being computed.
template <int FMT, int KS, int NB>
__device__ __forceinline__ void mmd_body(const int wg, const MdMats& M, const uint8_t* __restrict__ X, int bpr,
                                         int batch, int ntt, int nrt, int early_x) {
  constexpr int OWN = 16 / KS;  // chain elements per lane when KS > 1
  constexpr size_t BS = FMT == kQ4K ? kQ4KBytes : FMT == kQ6K ? kQ6KBytes : kQ8_0Bytes;
  constexpr size_t XS = FMT == kQ8_0 ? kQ8_0Bytes : kQ8KBytes;  // activation block bytes
  extern __shared__ __align__(16) uint32_t lds[];
  // XCD-aware numbering: the token tiles of one row tile share an XCD and its L2.
  const int xcd = wg & 7, slot = wg >> 3;
  const int tt = slot % ntt;
  const int rt = (slot / ntt) * 8 + xcd;
  if (rt >= nrt) return;  // padding workgroup (uniform, before any barrier)
  const int m = rt >= M.tile2 ? 2 : rt >= M.tile1 ? 1 : 0;
  const uint8_t* __restrict__ W = m == 2 ? M.w2 : m == 1 ? M.w1 : M.w0;
  float* __restrict__ Y = m == 2 ? M.y2 : m == 1 ? M.y1 : M.y0;
  const int rows = m == 2 ? M.rows2 : m == 1 ? M.rows1 : M.rows0;
  const int lane = threadIdx.x & 63;
  const int ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ta = lane & 31, kg = lane >> 5;
  const int r0 = (rt - (m == 2 ? M.tile2 : m == 1 ? M.tile1 : 0)) * 32, t0 = tt * 32;
  // rows and tokens past the end load valid memory (the last row / token) and store nothing;
  // K-quants: xrow is the tile's first token's row, the lanes' windows offsets from it
  const uint8_t* xrow = X + (size_t)min(t0 + (FMT == kQ8_0 ? ta : 0), batch - 1) * bpr * XS;
  const uint8_t* wrow = W + (size_t)min(r0 + ta, rows - 1) * bpr * BS;
  uint32_t xo[FMT == kQ8_0 ? 1 : kMdXi];
  if constexpr (FMT != kQ8_0) md_window_offsets(xo, lane, batch - 1 - t0, bpr);
  uint32_t* scal = lds + ks * kMdScalDw;
  float* xch = (float*)(lds + KS * kMdScalDw);  // KS > 1: [2][KS][1024], producer-lane-major
  // K-quants: this wave's activation stage, after the exchange buffers
  uint8_t* stg = (uint8_t*)(lds + KS * kMdScalDw + (KS > 1 ? 2 * KS * 1024 : 0)) + ks * kMdStage;
  const int nrounds = (bpr + KS - 1) / KS;

  float acc[KS == 1 ? 16 : OWN];
#pragma unroll
  for (int e = 0; e < (KS == 1 ? 16 : OWN); e++) acc[e] = 0.0f;
  auto chain_add = [&](int r) {
#pragma unroll
    for (int s = 0; s < KS; s++) {
      if (KS * r + s < bpr) {
        const float* src = xch + ((r & 1) * KS + s) * 1024 + ks * (1024 / KS) + lane * OWN;
#pragma unroll
        for (int u = 0; u < OWN; u++) acc[u] = acc[u] + src[u];  // block order
      }
    }
  };
  // Loads are unconditional (past the last block they repeat it: valid memory,
  // never used), so the registers hold one block's values, never a choice of two.
  auto finish = [&](int k, const float c[16]) {
    if constexpr (KS == 1) {
#pragma unroll
      for (int e = 0; e < 16; e++) acc[e] = acc[e] + c[e];  // block order
    } else {
      float* dst = xch + ((k & 1) * KS + ks) * 1024 + lane * 16;
#pragma unroll
      for (int e = 0; e < 16; e += 4) *(float4*)(dst + e) = make_float4(c[e], c[e + 1], c[e + 2], c[e + 3]);
    }
  };
  if constexpr (NB == 8) {
    // Spans through LDS (Q8_0, whole rows per wave): the wave reads a span of
    // its 32 weight rows and 32 tokens as consecutive 16-byte windows (about 4
    // rows per load instruction, where one operand per lane touches 32 rows'
    // lines), writes them to its stages, and takes each block's operands from
    // there; the next span's windows load during the current span's blocks.
    static_assert(FMT == kQ8_0 && KS == 1, "spans: Q8_0, whole rows");
    uint8_t* sw = (uint8_t*)(lds + kMdScalDw);  // 32 rows x 272 bytes
    uint8_t* sx = sw + 32 * kMdSpanB;           // 32 tokens x 272 bytes
    size_t wro[kMdSpanLd], xro[kMdSpanLd];  // window offsets at span 0
#pragma unroll
    for (int j = 0; j < kMdSpanLd; j++) {
      const int i = min(64 * j + lane, 32 * kMdSpanWin - 1);
      const int rr = i / kMdSpanWin, pc = i - rr * kMdSpanWin;
      wro[j] = (size_t)min(r0 + rr, rows - 1) * bpr * BS + 16 * pc;
      xro[j] = (size_t)min(t0 + rr, batch - 1) * bpr * XS + 16 * pc;
    }
    const int nspan = bpr / 8;
    u32x4 gw[kMdSpanLd], gx[kMdSpanLd];
#pragma unroll
    for (int j = 0; j < kMdSpanLd; j++) {
      gw[j] = *(const u32x4*)(W + wro[j]);
      gx[j] = *(const u32x4*)(X + xro[j]);
    }
    for (int sp = 0; sp < nspan; sp++) {
#pragma unroll
      for (int j = 0; j < kMdSpanLd; j++) {
        const int i = 64 * j + lane;
        if (j < kMdSpanLd - 1 || i < 32 * kMdSpanWin) {
          *(u32x4*)(sw + 16 * i) = gw[j];
          *(u32x4*)(sx + 16 * i) = gx[j];
        }
      }
      // lanes read other lanes' windows: the wave's LDS accesses run in program
      // order, and these compiler barriers keep that order in the code
      asm volatile("" ::: "memory");
      const size_t nxt = (size_t)min(sp + 1, nspan - 1) * kMdSpanB;  // the last span reloads itself
#pragma unroll
      for (int j = 0; j < kMdSpanLd; j++) {
        gw[j] = *(const u32x4*)(W + wro[j] + nxt);
        gx[j] = *(const u32x4*)(X + xro[j] + nxt);
      }
#pragma unroll 2
      for (int jb = 0; jb < 8; jb++) {
        MdLoad<kQ8_0> L;
        md_q8_window_lds(sx + ta * kMdSpanB + 34 * jb, kg, L.a, L.a4, L.ad, L.ao);
        md_q8_window_lds(sw + ta * kMdSpanB + 34 * jb, kg, L.w, L.w4, L.wd, L.wo);
        float c[16];
        md_q8(L, scal, ta, kg, c, [&]() {});
        finish(8 * sp + jb, c);
      }
      asm volatile("" ::: "memory");  // the span's reads come before the next span's writes
    }
  } else if constexpr (NB == 4) {
    // four register buffers in a ring: round k's block is loaded at round k - 3
    MdLoad<FMT> L0, L1, L2, L3;
    {
      const int b0 = min(ks, bpr - 1), b1 = min(KS + ks, bpr - 1), b2 = min(2 * KS + ks, bpr - 1);
      md_load<FMT>(L0, xrow + (size_t)b0 * XS, wrow + (size_t)b0 * BS, kg, xo);
      md_load<FMT>(L1, xrow + (size_t)b1 * XS, wrow + (size_t)b1 * BS, kg, xo);
      md_load<FMT>(L2, xrow + (size_t)b2 * XS, wrow + (size_t)b2 * BS, kg, xo);
    }
    auto body = [&](int k, MdLoad<FMT>& cur, MdLoad<FMT>& nxt) {
      const int b = KS * k + ks;
      const int bn = min(b + 3 * KS, bpr - 1);
      md_load<FMT>(nxt, xrow + (size_t)bn * XS, wrow + (size_t)bn * BS, kg, xo);
      asm volatile("" ::: "memory");  // the loads issue here, ahead of the block's compute
      if constexpr (KS > 1) {
        md_barrier();
        if (k > 0) chain_add(k - 1);
      }
      if (b < bpr) {
        float c[16];
        if constexpr (FMT == kQ8_0) {
          md_q8(cur, scal, ta, kg, c, [&]() {});
        } else if constexpr (FMT == kQ4K) {
          md_q4k(cur, stg, scal, ta, kg, c, [&]() {}, [&]() {});
        } else {
          md_q6k(cur, (uint32_t)((uintptr_t)(wrow + (size_t)b * BS) & 3u), stg, scal, ta, kg, c, [&](int) {},
                 [&]() {});
        }
        finish(k, c);
      }
    };
    int k = 0;
    for (; k + 4 <= nrounds; k += 4) {
      body(k, L0, L3);
      body(k + 1, L1, L0);
      body(k + 2, L2, L1);
      body(k + 3, L3, L2);
    }
    if (k < nrounds) body(k, L0, L3);  // at most three rounds remain
    if (k + 1 < nrounds) body(k + 1, L1, L0);
    if (k + 2 < nrounds) body(k + 2, L2, L1);
  } else if constexpr (NB == 2) {
    // two register buffers: a block's loads are issued a whole block ahead
    MdLoad<FMT> La, Lb;
    {
      const int b0 = min(ks, bpr - 1);
      md_load<FMT>(La, xrow + (size_t)b0 * XS, wrow + (size_t)b0 * BS, kg, xo);
    }
    auto body = [&](int k, MdLoad<FMT>& cur, MdLoad<FMT>& nxt) {
      const int b = KS * k + ks;
      const int bn = min(b + KS, bpr - 1);
      md_load<FMT>(nxt, xrow + (size_t)bn * XS, wrow + (size_t)bn * BS, kg, xo);
      asm volatile("" ::: "memory");  // the loads issue here, ahead of the block's compute
      if constexpr (KS > 1) {
        md_barrier();
        if (k > 0) chain_add(k - 1);
      }
      if (b < bpr) {
        float c[16];
        if constexpr (FMT == kQ8_0) {
          md_q8(cur, scal, ta, kg, c, [&]() {});
        } else if constexpr (FMT == kQ4K) {
          md_q4k(cur, stg, scal, ta, kg, c, [&]() {}, [&]() {});
        } else {
          md_q6k(cur, (uint32_t)((uintptr_t)(wrow + (size_t)b * BS) & 3u), stg, scal, ta, kg, c, [&](int) {},
                 [&]() {});
        }
        finish(k, c);
      }
    };
    int k = 0;
    for (; k + 1 < nrounds; k += 2) {
      body(k, La, Lb);
      body(k + 1, Lb, La);
    }
    if (k < nrounds) body(k, La, Lb);
  } else {
    // one register buffer: the next block's loads are issued as soon as the
    // current block's operands are consumed
    MdLoad<FMT> L;
    {
      const int b0 = min(ks, bpr - 1);
      md_load<FMT>(L, xrow + (size_t)b0 * XS, wrow + (size_t)b0 * BS, kg, xo);
    }
    for (int k = 0; k < nrounds; k++) {
      const int b = KS * k + ks;
      const int bn = min(b + KS, bpr - 1);
      if constexpr (KS > 1) {
        md_barrier();
        if (k > 0) chain_add(k - 1);
      }
      if (b < bpr) {
        float c[16];
        const uint8_t* xn = xrow + (size_t)bn * XS;
        const uint8_t* wn = wrow + (size_t)bn * BS;
        if constexpr (FMT == kQ8_0) {
          md_q8(L, scal, ta, kg, c, [&]() { md_load<kQ8_0>(L, xn, wn, kg, xo); });
        } else if constexpr (FMT == kQ4K) {
          // the next block's activation windows as soon as this block's are staged,
          // its weights once this block's are consumed
          // (early_x, uniform: the windows with the weights instead, once all are consumed)
          md_q4k(L, stg, scal, ta, kg, c, [&]() {
            if (!early_x) md_load_windows(L.x, xn, xo);
            L.h = *(const u32x4*)wn;
#pragma unroll
            for (int cc = 0; cc < 4; cc++) L.q[cc] = *(const u32x4*)(wn + 16 + 32 * cc + 16 * kg);
          }, [&]() {
            if (early_x) md_load_windows(L.x, xn, xo);
          });
        } else {
          md_q6k(L, (uint32_t)((uintptr_t)(wrow + (size_t)b * BS) & 3u), stg, scal, ta, kg, c,
                 [&](int hh) { md_load_q6k_half(L, xn, wn, kg, hh, xo, !early_x); },
                 [&]() {
                   if (early_x) md_load_windows(L.x, xn, xo);
                 });
        }
        finish(k, c);
      }
    }
  }
  if constexpr (KS == 1) {
    const int row = r0 + ta;
#pragma unroll
    for (int e = 0; e < 16; e++) {
      const int tok = t0 + 8 * (e >> 2) + 4 * kg + (e & 3);
      if (row < rows && tok < batch) Y[(size_t)tok * rows + row] = acc[e];
    }
  } else {
    md_barrier();
    chain_add(nrounds - 1);
#pragma unroll
    for (int u = 0; u < OWN; u++) {
      const int f = ks * (1024 / KS) + lane * OWN + u;  // producer lane f / 16, its element f % 16
      const int pl = f >> 4, e = f & 15;
      const int row = r0 + (pl & 31), tok = t0 + 8 * (e >> 2) + 4 * (pl >> 5) + (e & 3);
      if (row < rows && tok < batch) Y[(size_t)tok * rows + row] = acc[u];
    }
  }
}

template <int FMT, int KS, int NB>
__global__ __launch_bounds__(64 * KS) void mmd_kernel(MdMats M, const uint8_t* __restrict__ X, int bpr, int batch,
                                                      int ntt, int nrt, int early_x) {
  mmd_body<FMT, KS, NB>((int)blockIdx.x, M, X, bpr, batch, ntt, nrt, early_x);
}

// Two K-quant groups of different formats over one activation (Qwen3 Q4_K_M:
// q|k in Q4_K and v in Q6_K) in one launch: workgroups below nwg0 run the F0
// group's tiles, the others the F1 group's, each numbered as in its own launch.
template <int F0, int F1, int KS>
__global__ __launch_bounds__(64 * KS) void mmd2_kernel(MdMats M0, MdMats M1, const uint8_t* __restrict__ X, int bpr,
                                                       int batch, int ntt, int nrt0, int nrt1, int nwg0, int early0,
                                                       int early1) {
  const int wg = (int)blockIdx.x;
  if (wg < nwg0) mmd_body<F0, KS, 1>(wg, M0, X, bpr, batch, ntt, nrt0, early0);
  else mmd_body<F1, KS, 1>(wg - nwg0, M1, X, bpr, batch, ntt, nrt1, early1);
}

// ---- launch ----------------------------------------------------------------------------------

namespace {

// A launch's matrices, and its total row tiles.
MdMats md_mats(const MatmulGroupLaunch& G, int* nrt) {
  MdMats M{};
  const int t0 = (G.rows[0] + 31) / 32;
  const int t1 = G.nmat > 1 ? (G.rows[1] + 31) / 32 : 0;
  const int t2 = G.nmat > 2 ? (G.rows[2] + 31) / 32 : 0;
  M.w0 = (const uint8_t*)G.w[0];
  M.y0 = G.y[0];
  M.rows0 = G.rows[0];
  M.w1 = G.nmat > 1 ? (const uint8_t*)G.w[1] : M.w0;
  M.y1 = G.nmat > 1 ? G.y[1] : M.y0;
  M.rows1 = G.nmat > 1 ? G.rows[1] : M.rows0;
  M.w2 = G.nmat > 2 ? (const uint8_t*)G.w[2] : M.w0;
  M.y2 = G.nmat > 2 ? G.y[2] : M.y0;
  M.rows2 = G.nmat > 2 ? G.rows[2] : M.rows0;
  M.tile1 = G.nmat > 1 ? t0 : 0x7fffffff;
  M.tile2 = G.nmat > 2 ? t0 + t1 : 0x7fffffff;
  *nrt = t0 + t1 + t2;
  return M;
}

template <int FMT, int KS, int NB>
int md_launch_t(const MatmulGroupLaunch& G) {
  int nrt = 0;
  const MdMats M = md_mats(G, &nrt);
  const int ntt = (G.batch + 31) / 32;
  const long rt_pad = (long)((nrt + 7) / 8) * 8;
  const long nwg = rt_pad * ntt;
  if (nwg > 0x7fffffffL) return NRQ_LAUNCH_BAD_ARG;
  const size_t lds = (size_t)KS * kMdScalDw * 4 + (KS > 1 ? (size_t)2 * KS * 1024 * 4 : 0) +
                     (FMT == kQ8_0 ? (NB == 8 ? (size_t)2 * 32 * kMdSpanB : 0) : (size_t)KS * kMdStage);
  // one buffer: the next block's activation windows load as soon as the
  // current block's are staged (Q6_K, and Q4_K rows of 16+ blocks: down 30.5 ->
  // 27.7 us, o 13.4 -> 12.4 us on the Qwen3-4B layer at M = 64; q|k|v, 10
  // blocks, 13.4 -> 13.8 us, so not there), else with its weights
  const char* ex = getenv("NRQ_MMT_EARLY_X");
  const int early_x = ex && ex[0] ? ex[0] == '1' : (FMT == kQ6K || (FMT == kQ4K && G.bpr >= 16));
  hipLaunchKernelGGL((mmd_kernel<FMT, KS, NB>), dim3((unsigned)nwg), dim3(64 * KS), lds, (hipStream_t)G.stream, M,
                     (const uint8_t*)G.xs, G.bpr, G.batch, ntt, nrt, early_x);
  return hipGetLastError() == hipSuccess ? 0 : NRQ_LAUNCH_FAILED;
}

template <int FMT, int NB>
int md_launch_ks(const MatmulGroupLaunch& L, int ks) {
  if (ks >= 8) return md_launch_t<FMT, 8, NB>(L);
  if (ks == 4) return md_launch_t<FMT, 4, NB>(L);
  if (ks == 2) return md_launch_t<FMT, 2, NB>(L);
  return md_launch_t<FMT, 1, NB>(L);
}

// K-quant blocks (256 values) need one or two buffers; Q8_0 blocks (32
// values) take a ring of four to keep enough loads in flight.
template <int FMT>
int md_launch(const MatmulGroupLaunch& L, int ks, int nb) {
  if constexpr (FMT == kQ8_0) {
    if (nb == 8 && ks == 1) return md_launch_t<FMT, 1, 8>(L);
    if (nb >= 4) return md_launch_ks<FMT, 4>(L, ks);
  }
  return nb >= 2 ? md_launch_ks<FMT, 2>(L, ks) : md_launch_ks<FMT, 1>(L, ks);
}

// Block splits per tile: none when the tiles alone give four waves per CU
// (sixteen for rows of 32+ blocks; a whole row of blocks per wave,
// double-buffered, beat two splits by 3-6% on 9728 x 2560 at M = 64); else the
// fewest that give about two waves per SIMD (four for rows of 32+ blocks), and
// at most 4 for rows of fewer than 16 blocks (more splits leave each wave one
// or two blocks; the o projection's 16-block rows take 8 with the early
// activation loads, 12.4 -> 12.0 us). Measured on the Qwen3-4B layer shapes
// at M = 64 and M = 512.
int md_choose(int dtype, long row_tiles, int batch, int bpr) {
  const char* env = getenv("NRQ_MMT_SPLITS");  // tuning override: 1, 2, 4 or 8
  if (env && env[0]) {
    const int ks = atoi(env);
    if (ks == 1 || ks == 2 || ks == 4 || ks == 8) return ks;
  }
  const long tiles = row_tiles * ((batch + 31) / 32);
  // Q8_0 past 64 tokens, rows of 8-block multiples: whole rows in 8-block
  // spans from 1024 tiles (Llama-3.2-1B at M = 512: q|k|v 72 -> 39 us, o 48
  // -> 34, down 174 -> 117, gate 181 -> 82; at M = 128 gate's 1024 tiles 49 ->
  // 34, while q|k|v's 384 tiles keep 2 splits, 25 against 27)
  if (dtype == kQ8_0 && batch > 64 && bpr % 8 == 0 && tiles >= 1024) return 1;
  const int cap = bpr < 16 ? 4 : 8;
  // Q8_0 blocks are an eighth of a K-quant block's work: aim for twice the
  // waves. K-quants: splits until about 8 (rows of 32+ blocks: 16) tiles per
  // CU; at M = 512 the Qwen3-4B down (80 row tiles, 38 blocks) takes 117 us in
  // 4 splits against 158 in none, v (32 row tiles) 12 against 17; gate|up
  // (608 row tiles) and q|k keep whole rows.
  const long want = dtype == kQ8_0 ? 8L * 256 : (bpr >= 32 ? 16L : 8L) * 256;
  if (dtype != kQ8_0 && tiles >= (bpr >= 32 ? 16L : 4L) * 256) return 1;
  int ks = 1;
  while (ks < cap && ks < bpr && tiles * ks < want) ks *= 2;
  return ks;
}

int md_buffers(int dtype, int ks, int batch, int bpr);

// the early activation loads of md_launch_t, by format and row length
int md_early_x(int fmt, int bpr) {
  const char* ex = getenv("NRQ_MMT_EARLY_X");
  return ex && ex[0] ? ex[0] == '1' : (fmt == kQ6K || (fmt == kQ4K && bpr >= 16));
}

template <int F0, int F1, int KS>
int md2_launch_t(const MatmulGroupLaunch& G0, const MatmulGroupLaunch& G1) {
  int nrt0 = 0, nrt1 = 0;
  const MdMats M0 = md_mats(G0, &nrt0), M1 = md_mats(G1, &nrt1);
  const int ntt = (G0.batch + 31) / 32;
  const long nwg0 = (long)((nrt0 + 7) / 8) * 8 * ntt, nwg1 = (long)((nrt1 + 7) / 8) * 8 * ntt;
  if (nwg0 + nwg1 > 0x7fffffffL) return NRQ_LAUNCH_BAD_ARG;
  const size_t lds = (size_t)KS * kMdScalDw * 4 + (size_t)2 * KS * 1024 * 4 + (size_t)KS * kMdStage;
  hipLaunchKernelGGL((mmd2_kernel<F0, F1, KS>), dim3((unsigned)(nwg0 + nwg1)), dim3(64 * KS), lds,
                     (hipStream_t)G0.stream, M0, M1, (const uint8_t*)G0.xs, G0.bpr, G0.batch, ntt, nrt0, nrt1,
                     (int)nwg0, md_early_x(F0, G0.bpr), md_early_x(F1, G1.bpr));
  return hipGetLastError() == hipSuccess ? 0 : NRQ_LAUNCH_FAILED;
}

template <int F0, int F1>
int md2_launch_ks(const MatmulGroupLaunch& G0, const MatmulGroupLaunch& G1, int ks) {
  if (ks >= 8) return md2_launch_t<F0, F1, 8>(G0, G1);
  if (ks == 4) return md2_launch_t<F0, F1, 4>(G0, G1);
  return md2_launch_t<F0, F1, 2>(G0, G1);
}

int md_group(int dtype, const MatmulGroupLaunch& G) {
  long row_tiles = 0;
  for (int i = 0; i < G.nmat; i++) row_tiles += (G.rows[i] + 31) / 32;
  const int ks = md_choose(dtype, row_tiles, G.batch, G.bpr);
  int nb = md_buffers(dtype, ks, G.batch, G.bpr);
  if (nb == 8) {  // spans need 8-block rows on 16-byte aligned bases
    uintptr_t a = (uintptr_t)G.xs;
    for (int i = 0; i < G.nmat; i++) a |= (uintptr_t)G.w[i];
    if (ks != 1 || G.bpr % 8 != 0 || (a & 15u) != 0) nb = 1;
  }
  if (dtype == kQ8_0) return md_launch<kQ8_0>(G, ks, nb);
  return dtype == kQ4K ? md_launch<kQ4K>(G, ks, nb) : md_launch<kQ6K>(G, ks, nb);
}

// Register buffers of block loads. K-quants: two (a block's loads issued a
// whole block ahead) where waves are fewest per SIMD, one split; else one
// (eight splits of the Qwen3-4B down projection: 30.4 us on one buffer, 34.1
// on two, which spill). Q8_0: one (on the Llama-3.2-1B shapes at M = 64 one
// buffer beat two and a ring of four by 4-20%).
int md_buffers(int dtype, int ks, int batch, int bpr) {
  const char* nb = getenv("NRQ_MMT_NB");  // tuning override: 1, 2, 4 or 8 (4, 8: Q8_0 only)
  if (nb && nb[0]) return atoi(nb);
  const char* env = getenv("NRQ_MMT_DB");  // tuning override: 0 (one buffer) or 1 (two)
  if (env && env[0]) return env[0] == '1' ? 2 : 1;
  // Q8_0 whole rows past 64 tokens: 8-block spans through LDS (Llama-3.2-1B
  // gate|up, 16384 x 2048 at M = 512: see the staging branch of mmd_body)
  if (dtype == kQ8_0) return ks == 1 && batch > 64 && bpr % 8 == 0 ? 8 : 1;
  // whole rows: two buffers, except for rows of fewer than 16 blocks at more
  // than 64 tokens (Qwen3-4B gate and up at M = 512: 58 against 63 us; o's 16
  // blocks: 40 against 37)
  return ks == 1 && (batch <= 64 || bpr >= 16) ? 2 : 1;
}

}  // namespace

// Q8_0 takes the 32 x 32 tiles from 1024 rows (gate/up 8192 x 2048 at M = 64:
// 25 us against 52 on 16 x 16 tiles; k/v 512 x 2048: 13.6 against 10.6), with
// 4-byte aligned bases for its dword windows.
bool mmt_fits(int dtype, const MatmulLaunch& L) {
  if (dtype == kQ8_0) return L.rows >= 1024 && (((uintptr_t)L.w | (uintptr_t)L.xs) & 3u) == 0;
  return dtype == kQ4K || dtype == kQ6K;
}

int launch_mmt(int dtype, const MatmulLaunch& L) {
  if (L.rows <= 0 || L.bpr <= 0 || L.batch <= 0) return 0;
  MatmulGroupLaunch G{};
  G.w[0] = L.w;
  G.y[0] = L.y;
  G.rows[0] = L.rows;
  G.nmat = 1;
  G.xs = L.xs;
  G.bpr = L.bpr;
  G.batch = L.batch;
  G.stream = L.stream;
  return md_group(dtype, G);
}

// Every matrix of the group in one launch when the 32 x 32 kernel takes their
// format and the group's rows (Q8_0: 1024 in all, 4-byte aligned bases).
int launch_mmt_group(int dtype, const MatmulGroupLaunch& G) {
  if (G.nmat < 1 || G.nmat > 3 || G.bpr <= 0 || G.batch <= 0) return NRQ_LAUNCH_BAD_ARG;
  if (dtype != kQ8_0 && dtype != kQ4K && dtype != kQ6K) return NRQ_LAUNCH_BAD_ARG;
  int total = 0;
  uintptr_t bases = (uintptr_t)G.xs;
  for (int i = 0; i < G.nmat; i++) {
    if (G.rows[i] <= 0) return NRQ_LAUNCH_BAD_ARG;
    total += G.rows[i];
    bases |= (uintptr_t)G.w[i];
  }
  if (dtype == kQ8_0 && (total < 1024 || (bases & 3u))) return NRQ_LAUNCH_BAD_ARG;
  return md_group(dtype, G);
}

// Two groups of different K-quant formats over one activation in one launch,
// when the split rule gives both more than one split (so that both take one
// load buffer, as their own launches would); else NRQ_LAUNCH_BAD_ARG.
int launch_mmt_group2(int dt0, const MatmulGroupLaunch& G0, int dt1, const MatmulGroupLaunch& G1) {
  const bool kq0 = dt0 == kQ4K || dt0 == kQ6K, kq1 = dt1 == kQ4K || dt1 == kQ6K;
  if (!kq0 || !kq1 || dt0 == dt1 || G0.xs != G1.xs || G0.bpr != G1.bpr || G0.batch != G1.batch) return NRQ_LAUNCH_BAD_ARG;
  for (const MatmulGroupLaunch* G : {&G0, &G1}) {
    if (G->nmat < 1 || G->nmat > 3 || G->bpr <= 0 || G->batch <= 0) return NRQ_LAUNCH_BAD_ARG;
    for (int i = 0; i < G->nmat; i++)
      if (G->rows[i] <= 0) return NRQ_LAUNCH_BAD_ARG;
  }
  long row_tiles = 0;
  for (const MatmulGroupLaunch* G : {&G0, &G1})
    for (int i = 0; i < G->nmat; i++) row_tiles += (G->rows[i] + 31) / 32;
  const int ks = md_choose(dt0, row_tiles, G0.batch, G0.bpr);
  if (ks < 2 || md_buffers(dt0, ks, G0.batch, G0.bpr) != 1 || md_buffers(dt1, ks, G1.batch, G1.bpr) != 1) return NRQ_LAUNCH_BAD_ARG;
  return dt0 == kQ4K ? md2_launch_ks<kQ4K, kQ6K>(G0, G1, ks) : md2_launch_ks<kQ6K, kQ4K>(G0, G1, ks);
}

}  // namespace nrq
