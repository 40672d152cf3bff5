// Batched prefill matmul on int8 MFMA in the reference's AVX2 f32 order:
//   Q4_K x Q8_K: dot_q4k_avx2 / dot_q4k_avx2_x4 (crates/nr-tensor/src/kquant.rs:260-374)
//   Q6_K x Q8_K: dot_q6k_avx2 / dot_q6k_avx2_x4 (kquant.rs:383-510)
//   Q8_0 x Q8_0: dot_q8_avx2 / dot_q8_avx2_x4 (crates/nr-tensor/src/kernels.rs:229-286)
// so y[t][r] equals the AVX2-order decode matvec (nrq_matvec.hip) bit for bit,
// as the reference's 4-wide tiles equal its 1-wide dots (kquant.rs:307-310).
//
// The reference keeps eight f32 accumulators per (row, token), the lanes k of
// an __m256, each fed once per block by acc_k = fma(d, f32(sumi_k), acc_k).
// The i32 sumi_k sums the block's products over bytes 4k..4k+3 of every
// 32-byte vector ("class k"), each scaled inside the integer sum by its
// sub-block's (Q4_K) or group's (Q6_K) scale. The lanes meet at the end in
// hsum256's order ((a0+a4)+(a2+a6))+((a1+a5)+(a3+a7)).
//
// K-quants. A class is 32 of a block's 256 values (4 bytes of each of its 8
// vectors), so one v_mfma_i32_32x32x32_i8 step over them gives sumi_k exactly
// once the scale is folded into the weight operand: lane half kg supplies the
// class's 4 bytes of vectors 4kg..4kg+3 (Q4_K sub-blocks; Q6_K: the planes of
// half kg) in both operands. The scaled weight does not fit an int8 (Q4_K
// sc*q up to 63*15, Q6_K sc*(q-32) up to 4096), so it is split exactly into
// two operands, two steps and an exact i32 combine (|sumi| <= 2^24):
//   Q4_K: sc = 8*sh + sl with sl, sh in 0..7; sl*q and sh*q are at most 105,
//         byte products formed four at a time with no carry between bytes;
//         sumi = 8*C(sh*q) + C(sl*q).
//   Q6_K: P = sc*(q-32) in 16-bit lanes, lo = P & 127, hi = P >> 7 (in
//         -32..32); sumi = 128*C(hi) + C(lo).
// A workgroup of 4 waves owns a 32-row x 32-token tile. Wave w owns classes
// 2w and 2w+1 (8 contiguous bytes per vector, one load each) and runs their
// fma chains over the row's blocks in order; at the end the waves meet in
// LDS, and wave w sums the 8 lanes of its quarter of the tile's outputs.
// Q4_K's acc_min (acc_min += (dmin*x.d) * f32(min_sum) per block, subtracted
// after the hsum) takes min_sum from two MFMA steps over the bsums, split
// exactly into low 7 bits and a signed high part.
//
// Q8_0. A class is 4 bytes of a 32-value block. One MFMA step over a block,
// with output columns taken as (row, class) pairs (4 rows x 8 classes) and
// the weight operand masked to the column's class, gives every class's
// 4-byte dot; the hsum runs across the 8 class lanes (xor 4, 2, 1). The
// activations are q8::quantize's, in [-127, 127], where the reference's
// sign_epi8 / maddubs pair is the plain product (as in the decode kernel).
#include "nrq_device.h"
#include "nrq_launch.h"

namespace nrq {

namespace {

typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2a __attribute__((ext_vector_type(2), aligned(4)));
typedef uint32_t u32x3a __attribute__((ext_vector_type(3), aligned(4)));
typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef short s16x2 __attribute__((ext_vector_type(2)));

// 32 x 32 x 32 int8 step: lane l supplies row l % 32 of A (tokens) and
// column l % 32 of B (weight rows, or (row, class) pairs) at the same 16 K
// positions of lane half l / 32; lane l receives column l % 32, rows
// 8(e/4) + 4(l/32) + e%4 for e = 0..15.
__device__ __forceinline__ i32x16 ma_mfma32(const uint32_t a[4], const uint32_t b[4], i32x16 c) {
  const i32x4v av = {(int)a[0], (int)a[1], (int)a[2], (int)a[3]};
  const i32x4v bv = {(int)b[0], (int)b[1], (int)b[2], (int)b[3]};
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, c, 0, 0, 0);
}

// 32 x 32 x 16 int8 step (8 K positions per lane half).
__device__ __forceinline__ i32x16 ma_mfma16(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1, i32x16 c) {
  const long a = (long)(((uint64_t)a1 << 32) | a0);
  const long b = (long)(((uint64_t)b1 << 32) | b0);
  return __builtin_amdgcn_mfma_i32_32x32x16_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ u16x2 as_u16x2(uint32_t v) {
  u16x2 r;
  __builtin_memcpy(&r, &v, 4);
  return r;
}
__device__ __forceinline__ uint32_t from_u16x2(u16x2 v) {
  uint32_t r;
  __builtin_memcpy(&r, &v, 4);
  return r;
}
__device__ __forceinline__ s16x2 as_s16x2(uint32_t v) {
  s16x2 r;
  __builtin_memcpy(&r, &v, 4);
  return r;
}
__device__ __forceinline__ uint32_t from_s16x2(s16x2 v) {
  uint32_t r;
  __builtin_memcpy(&r, &v, 4);
  return r;
}

// Four bytes of at most 15 times s <= 7: 16-bit lane products, no carry
// between bytes (each byte product is at most 105).
__device__ __forceinline__ uint32_t mul_nibbles(uint32_t v, uint32_t s) {
  const u16x2 m = {(unsigned short)s, (unsigned short)s};
  return from_u16x2(as_u16x2(v) * m);
}

// Q6_K: the four products P = sc * (q - 32) of a dword of 6-bit quants, in
// 16-bit lanes (s16 = sc and c16 = -32 * sc in both halves, mod 2^16), split
// exactly into lo = P & 127 and hi = P >> 7, one int8 per quant, in byte order.
__device__ __forceinline__ void q6_scaled_split(uint32_t q6, uint32_t s16, uint32_t c16, uint32_t& lo,
                                                uint32_t& hi) {
  const uint32_t ev = __builtin_amdgcn_perm(0u, q6, 0x0c020c00u);  // quants 0, 2 as 16-bit lanes
  const uint32_t od = __builtin_amdgcn_perm(0u, q6, 0x0c030c01u);  // quants 1, 3
  const uint32_t pe = from_u16x2(as_u16x2(ev) * as_u16x2(s16) + as_u16x2(c16));
  const uint32_t po = from_u16x2(as_u16x2(od) * as_u16x2(s16) + as_u16x2(c16));
  lo = __builtin_amdgcn_perm(po, pe, 0x06020400u) & 0x7f7f7f7fu;  // low bytes: P0, P1, P2, P3
  const uint32_t he = from_s16x2(as_s16x2(pe) >> (short)7), ho = from_s16x2(as_s16x2(po) >> (short)7);
  hi = __builtin_amdgcn_perm(ho, he, 0x06020400u);
}

// XCD-aware tile numbering (workgroups go round-robin over the 8 XCDs): the
// token tiles of one row tile run on one XCD and share its L2.
__device__ __forceinline__ bool ma_tile(int ntt, int nrt, int& rt, int& tt) {
  const int wg = blockIdx.x;
  const int xcd = wg & 7, slot = wg >> 3;
  tt = slot % ntt;
  rt = (slot / ntt) * 8 + xcd;
  return rt < nrt;
}

// ---- K-quants ----------------------------------------------------------------------

template <int FMT>
struct KqLoad;
template <>
struct KqLoad<kQ4K> {
  u32x4 h;       // d | dmin, scales[12]
  u32x2a q[2];   // qs dwords 2w, 2w+1 of 32-byte groups 2kg, 2kg+1
  u32x2a x[4];   // activation qs dwords 2w, 2w+1 of sub-blocks 4kg .. 4kg+3
  u32x4a bs;     // bsums 8kg .. 8kg+7 of token ta ^ 8w (see kq_block)
  uint32_t xd;   // activation d (f32 bits)
};
template <>
struct KqLoad<kQ6K> {
  u32x3a ql[2];  // aligned windows over ql[64kg + 8w ..+8] and ql[64kg + 32 + 8w ..+8]
  u32x3a qh;     // over qh[32kg + 8w ..+8]
  u32x2a sc;     // over scales[8kg ..+8] ...
  uint32_t sc2;  // ... (its third dword)
  uint32_t d;    // f16 bits of d
  uint32_t sh;   // the block's byte offset past the aligned windows (0 or 2)
  u32x2a x[4];   // activation qs dwords 2w, 2w+1 of vectors (kg, n), n = 0..3
  uint32_t xd;
};

__device__ __forceinline__ void kq_load(KqLoad<kQ4K>& L, const uint8_t* __restrict__ wb,
                                        const uint8_t* __restrict__ xb, const uint8_t* __restrict__ xbm, int kg,
                                        int w) {
  L.h = *(const u32x4*)wb;
  L.q[0] = *(const u32x2a*)(wb + 16 + 64 * kg + 8 * w);
  L.q[1] = *(const u32x2a*)(wb + 16 + 64 * kg + 32 + 8 * w);
#pragma unroll
  for (int i = 0; i < 4; i++) L.x[i] = *(const u32x2a*)(xb + 4 + 32 * (4 * kg + i) + 8 * w);
  L.bs = *(const u32x4a*)(xbm + 260 + 16 * kg);
  L.xd = *(const uint32_t*)xb;
}

// Q6_K blocks (210 bytes) start 2-byte aligned: every window is an aligned
// 12-byte read covering the 8 bytes wanted, inside the block (the scale
// window's third dword is re-pointed inside the block when the block is
// 4-byte aligned, where it is not used).
__device__ __forceinline__ void kq_load(KqLoad<kQ6K>& L, const uint8_t* __restrict__ wb,
                                        const uint8_t* __restrict__ xb, const uint8_t* __restrict__ xbm, int kg,
                                        int w) {
  (void)xbm;
  const uint32_t sh = (uint32_t)((uintptr_t)wb & 3u);
  const uint8_t* w4 = wb - sh;
  L.sh = sh;
  L.ql[0] = *(const u32x3a*)(w4 + 64 * kg + 8 * w);
  L.ql[1] = *(const u32x3a*)(w4 + 64 * kg + 32 + 8 * w);
  L.qh = *(const u32x3a*)(w4 + 128 + 32 * kg + 8 * w);
  L.sc = *(const u32x2a*)(w4 + 192 + 8 * kg);
  L.sc2 = *(const uint32_t*)(w4 + 196 + 8 * kg + (sh ? 4 : 0));
  L.d = *(const uint16_t*)(wb + 208);
#pragma unroll
  for (int n = 0; n < 4; n++) L.x[n] = *(const u32x2a*)(xb + 4 + 128 * kg + 32 * n + 8 * w);
  L.xd = *(const uint32_t*)xb;
}

// One Q4_K block: acc[c][e] for the wave's classes, and acc_min[i] for
// tokens 8w + 4kg + i, the elements this wave sums at the end. xd[e]: the
// tokens' d; xdm[i]: those of tokens 8w + 4kg + i.
__device__ __forceinline__ void kq_block(const KqLoad<kQ4K>& L, const float xd[16], const float xdm[4], int kg,
                                         int w, float acc[2][16], float acc_min[4]) {
  const u32x4 h = L.h;
  // kquant.rs:83-92: the 6-bit scales and mins of sub-blocks 4kg .. 4kg+3, one per byte
  const uint32_t scw = kg ? ((h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u)) : (h.y & 0x3f3f3f3fu);
  const uint32_t mnw = kg ? (((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u)) : (h.z & 0x3f3f3f3fu);
  const uint32_t SL = scw & 0x07070707u, SH = (scw >> 3) & 0x07070707u;
  const float dw = f16_bits_to_f32(h.x & 0xffffu), dmw = f16_bits_to_f32(h.x >> 16);
  const i32x16 z = {};
  // kquant.rs:283-287: min_sum = sum_j mins[j] * (bsums[2j] + bsums[2j+1]), exact,
  // as two K = 16 steps: bsums 8kg .. 8kg+7 = 128 * hi + lo (lo in 0..127, hi in
  // -16..15) against m_{4kg}, m_{4kg}, m_{4kg+1}, ... Lane l supplies token
  // (l % 32) ^ 8w, so output element i (step row 4kg + i) is token 8w + 4kg + i:
  // the wave's own elements sit at static register positions.
  i32x16 smlo, smhi;
  {
    const uint32_t sb0 = L.bs.x, sb1 = L.bs.y, sb2 = L.bs.z, sb3 = L.bs.w;
    const uint32_t lo0 = __builtin_amdgcn_perm(sb1, sb0, 0x06040200u) & 0x7f7f7f7fu;
    const uint32_t lo1 = __builtin_amdgcn_perm(sb3, sb2, 0x06040200u) & 0x7f7f7f7fu;
    const uint32_t hi0 = __builtin_amdgcn_perm((sb1 >> 7) & 0x00ff00ffu, (sb0 >> 7) & 0x00ff00ffu, 0x06040200u);
    const uint32_t hi1 = __builtin_amdgcn_perm((sb3 >> 7) & 0x00ff00ffu, (sb2 >> 7) & 0x00ff00ffu, 0x06040200u);
    const uint32_t m0 = __builtin_amdgcn_perm(mnw, mnw, 0x01010000u), m1 = __builtin_amdgcn_perm(mnw, mnw, 0x03030202u);
    smlo = ma_mfma16(lo0, lo1, m0, m1, z);
    smhi = ma_mfma16(hi0, hi1, m0, m1, z);
  }
#pragma unroll
  for (int c = 0; c < 2; c++) {
    // kquant.rs:289-301: the class's bytes of sub-blocks 4kg+i (group 2kg + i/2,
    // low nibbles for even sub-blocks, high for odd), scaled by sc = 8*sh + sl
    const uint32_t qa = L.q[0][c], qb = L.q[1][c];
    const uint32_t nb[4] = {qa & 0x0f0f0f0fu, (qa >> 4) & 0x0f0f0f0fu, qb & 0x0f0f0f0fu, (qb >> 4) & 0x0f0f0f0fu};
    uint32_t alo[4], ahi[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      alo[i] = mul_nibbles(nb[i], (SL >> (8 * i)) & 0xffu);
      ahi[i] = mul_nibbles(nb[i], (SH >> (8 * i)) & 0xffu);
    }
    const uint32_t xa[4] = {L.x[0][c], L.x[1][c], L.x[2][c], L.x[3][c]};
    const i32x16 clo = ma_mfma32(xa, alo, z);
    const i32x16 chi = ma_mfma32(xa, ahi, z);
#pragma unroll
    for (int e = 0; e < 16; e++) {
      const int sumi = (int)(((uint32_t)chi[e] << 3) + (uint32_t)clo[e]);
      acc[c][e] = fmaf(dw * xd[e], (float)sumi, acc[c][e]);  // kquant.rs:302
    }
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int sm = (int)(((uint32_t)smhi[i] << 7) + (uint32_t)smlo[i]);  // exact: |min_sum| < 2^22
    const float dmin = dmw * xdm[i];
    acc_min[i] = acc_min[i] + dmin * (float)sm;  // kquant.rs:288
  }
}

// One Q6_K block: acc[c][e] for the wave's classes.
__device__ __forceinline__ void kq_block(const KqLoad<kQ6K>& L, const float xd[16], const float xdm[4], int kg,
                                         int w, float acc[2][16], float acc_min[4]) {
  (void)xdm;
  (void)kg;
  (void)acc_min;
  const uint32_t sh = L.sh;
  uint32_t QA[2], QB[2], QH[2];
  QA[0] = __builtin_amdgcn_alignbyte(L.ql[0].y, L.ql[0].x, sh);
  QA[1] = __builtin_amdgcn_alignbyte(L.ql[0].z, L.ql[0].y, sh);
  QB[0] = __builtin_amdgcn_alignbyte(L.ql[1].y, L.ql[1].x, sh);
  QB[1] = __builtin_amdgcn_alignbyte(L.ql[1].z, L.ql[1].y, sh);
  QH[0] = __builtin_amdgcn_alignbyte(L.qh.y, L.qh.x, sh);
  QH[1] = __builtin_amdgcn_alignbyte(L.qh.z, L.qh.y, sh);
  // scales[8kg .. 8kg+8); plane n of classes 0-3 takes sc[8kg + 2n], of 4-7
  // sc[8kg + 2n + 1] (kquant.rs:474-479): the wave's two classes share it
  const uint32_t S0 = __builtin_amdgcn_alignbyte(L.sc.y, L.sc.x, sh);
  const uint32_t S1 = __builtin_amdgcn_alignbyte(L.sc2, L.sc.y, sh);
  const int up = w >= 2 ? 8 : 0;
  const float dw = f16_bits_to_f32(L.d);
  uint32_t s16[4], c16[4];
#pragma unroll
  for (int n = 0; n < 4; n++) {
    const uint32_t word = n < 2 ? S0 : S1;
    const int s = (int)(int8_t)((word >> (16 * (n & 1) + up)) & 0xffu);
    s16[n] = ((uint32_t)s & 0xffffu) * 0x00010001u;
    c16[n] = ((uint32_t)(-32 * s) & 0xffffu) * 0x00010001u;
  }
  const i32x16 z = {};
#pragma unroll
  for (int c = 0; c < 2; c++) {
    uint32_t alo[4], ahi[4];
#pragma unroll
    for (int n = 0; n < 4; n++) {
      // kquant.rs:485-493: plane n = ql (n odd: ql[32..]) nibble (n >= 2: high)
      // | qh bits 2n, 2n+1 << 4
      const uint32_t ql = (n & 1) ? QB[c] : QA[c];
      const uint32_t nib = (n >> 1) ? ((ql >> 4) & 0x0f0f0f0fu) : (ql & 0x0f0f0f0fu);
      const uint32_t q6 = nib | (((QH[c] >> (2 * n)) & 0x03030303u) << 4);
      q6_scaled_split(q6, s16[n], c16[n], alo[n], ahi[n]);
    }
    const uint32_t xa[4] = {L.x[0][c], L.x[1][c], L.x[2][c], L.x[3][c]};
    const i32x16 clo = ma_mfma32(xa, alo, z);
    const i32x16 chi = ma_mfma32(xa, ahi, z);
#pragma unroll
    for (int e = 0; e < 16; e++) {
      const int sumi = (int)(((uint32_t)chi[e] << 7) + (uint32_t)clo[e]);
      acc[c][e] = fmaf(dw * xd[e], (float)sumi, acc[c][e]);  // kquant.rs:505
    }
  }
}

constexpr int kMaFinDw = 8 * 16 * 64;  // [class][e][lane] f32 at the end

template <int FMT>
__global__ __launch_bounds__(256) void mma_kq_kernel(const uint8_t* __restrict__ W, const uint8_t* __restrict__ X,
                                                     float* __restrict__ Y, int rows, int bpr, int batch, int ntt,
                                                     int nrt) {
  constexpr size_t BS = FMT == kQ4K ? kQ4KBytes : kQ6KBytes;
  extern __shared__ __align__(16) uint32_t lds[];
  int rt, tt;
  if (!ma_tile(ntt, nrt, rt, tt)) return;  // padding workgroup (uniform, before any barrier)
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ta = lane & 31, kg = lane >> 5;
  const int r0 = rt * 32, t0 = tt * 32;
  // rows and tokens past the end load the last one's blocks and store nothing
  const uint8_t* wrow = W + (size_t)min(r0 + ta, rows - 1) * bpr * BS;
  const uint8_t* xrow = X + (size_t)min(t0 + ta, batch - 1) * bpr * kQ8KBytes;
  const uint8_t* xrowm = X + (size_t)min(t0 + (ta ^ (8 * w)), batch - 1) * bpr * kQ8KBytes;  // Q4_K bsums
  uint32_t* tab = lds + 32 * w;  // this wave's table of the tile's 32 token d

  float acc[2][16], acc_min[4];
#pragma unroll
  for (int e = 0; e < 16; e++) acc[0][e] = acc[1][e] = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; i++) acc_min[i] = 0.0f;

  KqLoad<FMT> L[2];
  kq_load(L[0], wrow, xrow, xrowm, kg, w);
  auto body = [&](int b, KqLoad<FMT>& cur, KqLoad<FMT>& nxt) {
    const int bn = min(b + 1, bpr - 1);  // past the last block: a repeat, never used
    kq_load(nxt, wrow + (size_t)bn * BS, xrow + (size_t)bn * kQ8KBytes, xrowm + (size_t)bn * kQ8KBytes, kg, w);
    asm volatile("" ::: "memory");  // the next block's loads issue ahead of this block's compute
    if (kg == 0) tab[ta] = cur.xd;
    float xd[16];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const u32x4 v = *(const u32x4*)(tab + 8 * q + 4 * kg);  // tokens 8q + 4kg .. +3
      xd[4 * q + 0] = __uint_as_float(v.x);
      xd[4 * q + 1] = __uint_as_float(v.y);
      xd[4 * q + 2] = __uint_as_float(v.z);
      xd[4 * q + 3] = __uint_as_float(v.w);
    }
    float xdm[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (FMT == kQ4K) {
      const u32x4 v = *(const u32x4*)(tab + 8 * w + 4 * kg);  // tokens 8w + 4kg .. +3
      xdm[0] = __uint_as_float(v.x);
      xdm[1] = __uint_as_float(v.y);
      xdm[2] = __uint_as_float(v.z);
      xdm[3] = __uint_as_float(v.w);
    }
    kq_block(cur, xd, xdm, kg, w, acc, acc_min);
  };
  int b = 0;
  for (; b + 1 < bpr; b += 2) {
    body(b, L[0], L[1]);
    body(b + 1, L[1], L[0]);
  }
  if (b < bpr) body(b, L[0], L[1]);

  // hsum256 across the waves (kquant.rs:514-522): wave w sums elements 4w .. 4w+3
  float* fin = (float*)(lds + 4 * 32);
#pragma unroll
  for (int c = 0; c < 2; c++) {
#pragma unroll
    for (int e = 0; e < 16; e++) fin[((2 * w + c) * 16 + e) * 64 + lane] = acc[c][e];
  }
  __syncthreads();
  const int row = r0 + ta;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int e = 4 * w + i;
    float a[8];
#pragma unroll
    for (int c = 0; c < 8; c++) a[c] = fin[(c * 16 + e) * 64 + lane];
    float s = ((a[0] + a[4]) + (a[2] + a[6])) + ((a[1] + a[5]) + (a[3] + a[7]));
    if constexpr (FMT == kQ4K) s = s - acc_min[i];  // kquant.rs:304
    const int tok = t0 + 8 * w + 4 * kg + i;       // e = 4w + i
    if (row < rows && tok < batch) Y[(size_t)tok * rows + row] = s;
  }
}

// ---- Q8_0 ----------------------------------------------------------------------------

// qs bytes 16kg .. 16kg+15 of a Q8_0 block (34 bytes, 2-byte aligned) from an
// aligned 16-byte window inside the block (and the two bytes after it when the
// bytes start 2 past a dword), and d's f16 bits.
__device__ __forceinline__ void q8_half(const uint8_t* __restrict__ blk, int kg, uint32_t q[4], uint32_t& dbits) {
  const uint8_t* qp = blk + 2 + 16 * kg;
  const uint32_t p = (uint32_t)((uintptr_t)qp & 3u);
  const uint8_t* a = qp - p;
  const u32x4a v = *(const u32x4a*)a;
  const uint32_t v4 = *(const uint16_t*)(a + (p ? 16 : 14));  // p = 0: an in-block halfword, unused
  q[0] = __builtin_amdgcn_alignbyte(v.y, v.x, p);
  q[1] = __builtin_amdgcn_alignbyte(v.z, v.y, p);
  q[2] = __builtin_amdgcn_alignbyte(v.w, v.z, p);
  q[3] = __builtin_amdgcn_alignbyte(v4, v.w, p);
  dbits = *(const uint16_t*)blk;
}

// A wave owns 4*MT rows x 32 tokens: MT steps per block, each over 4 rows x 8
// classes (column l % 32 = 8 * row + class).
template <int MT>
__global__ __launch_bounds__(64) void mma_q8_kernel(const uint8_t* __restrict__ W, const uint8_t* __restrict__ X,
                                                    float* __restrict__ Y, int rows, int bpr, int batch, int ntt,
                                                    int nrt) {
  __shared__ __align__(16) uint32_t tab[32];  // the tile's 32 token d (f32 bits)
  int rt, tt;
  if (!ma_tile(ntt, nrt, rt, tt)) return;
  const int lane = threadIdx.x;
  const int ta = lane & 31, kg = lane >> 5;
  const int rr = ta >> 3, cls = ta & 7;
  const int r0 = rt * 4 * MT, t0 = tt * 32;
  const uint8_t* xrow = X + (size_t)min(t0 + ta, batch - 1) * bpr * kQ8_0Bytes;
  const uint8_t* wrow[MT];
#pragma unroll
  for (int m = 0; m < MT; m++) wrow[m] = W + (size_t)min(r0 + 4 * m + rr, rows - 1) * bpr * kQ8_0Bytes;
  // the column's class: dword cls & 3 of lane half cls >> 2 (kernels.rs:276-277)
  const int keep = kg == (cls >> 2) ? (cls & 3) : 4;

  float acc[MT][16];
#pragma unroll
  for (int m = 0; m < MT; m++) {
#pragma unroll
    for (int e = 0; e < 16; e++) acc[m][e] = 0.0f;
  }
  struct Ld {
    uint32_t x[4], xd;
    uint32_t q[MT][4], wd[MT];
  };
  auto load = [&](Ld& L, int b) {
    q8_half(xrow + (size_t)b * kQ8_0Bytes, kg, L.x, L.xd);
#pragma unroll
    for (int m = 0; m < MT; m++) q8_half(wrow[m] + (size_t)b * kQ8_0Bytes, kg, L.q[m], L.wd[m]);
  };
  auto body = [&](int b, Ld& cur, Ld& nxt) {
    load(nxt, min(b + 1, bpr - 1));
    asm volatile("" ::: "memory");
    if (kg == 0) tab[ta] = __float_as_uint(f16_bits_to_f32(cur.xd));
    float xd[16];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const u32x4 v = *(const u32x4*)(tab + 8 * q + 4 * kg);
      xd[4 * q + 0] = __uint_as_float(v.x);
      xd[4 * q + 1] = __uint_as_float(v.y);
      xd[4 * q + 2] = __uint_as_float(v.z);
      xd[4 * q + 3] = __uint_as_float(v.w);
    }
    const i32x16 z = {};
#pragma unroll
    for (int m = 0; m < MT; m++) {
      uint32_t bq[4];
#pragma unroll
      for (int j = 0; j < 4; j++) bq[j] = j == keep ? cur.q[m][j] : 0u;
      const i32x16 p = ma_mfma32(cur.x, bq, z);
      const float dw = f16_bits_to_f32(cur.wd[m]);
#pragma unroll
      for (int e = 0; e < 16; e++) acc[m][e] = fmaf(dw * xd[e], (float)p[e], acc[m][e]);  // kernels.rs:278
    }
  };
  Ld L0, L1;
  load(L0, 0);
  int b = 0;
  for (; b + 1 < bpr; b += 2) {
    body(b, L0, L1);
    body(b + 1, L1, L0);
  }
  if (b < bpr) body(b, L0, L1);
  // hsum (kernels.rs:279-285) over the 8 class lanes of each row: xor 4 pairs
  // a_k with a_(k+4), xor 2 then xor 1 finish ((s0+s2)+(s1+s3))
#pragma unroll
  for (int m = 0; m < MT; m++) {
    const int row = r0 + 4 * m + rr;
#pragma unroll
    for (int e = 0; e < 16; e++) {
      float v = acc[m][e];
      v = v + __shfl_xor(v, 4);
      v = v + __shfl_xor(v, 2);
      v = v + __shfl_xor(v, 1);
      const int tok = t0 + 8 * (e >> 2) + 4 * kg + (e & 3);
      if (cls == 0 && row < rows && tok < batch) Y[(size_t)tok * rows + row] = v;
    }
  }
}

constexpr int kMaQ8Rows = 8;  // rows per Q8_0 wave (MT = 2)

}  // namespace

int launch_mma(int dtype, const MatmulLaunch& L) {
  if (L.rows <= 0 || L.bpr <= 0 || L.batch <= 0) return 0;
  const int ntt = (L.batch + 31) / 32;
  const int tile_rows = dtype == kQ8_0 ? kMaQ8Rows : 32;
  const int nrt = (L.rows + tile_rows - 1) / tile_rows;
  const long nwg = (long)((nrt + 7) / 8) * 8 * ntt;
  if (nwg > 0x7fffffffL) return NRQ_LAUNCH_BAD_ARG;
  const hipStream_t st = (hipStream_t)L.stream;
  const uint8_t* w = (const uint8_t*)L.w;
  const uint8_t* x = (const uint8_t*)L.xs;
  if (dtype == kQ8_0) {
    hipLaunchKernelGGL((mma_q8_kernel<kMaQ8Rows / 4>), dim3((unsigned)nwg), dim3(64), 0, st, w, x, L.y, L.rows,
                       L.bpr, L.batch, ntt, nrt);
  } else {
    const size_t lds = (size_t)(4 * 32 + kMaFinDw) * 4;
    if (dtype == kQ4K)
      hipLaunchKernelGGL((mma_kq_kernel<kQ4K>), dim3((unsigned)nwg), dim3(256), lds, st, w, x, L.y, L.rows, L.bpr,
                         L.batch, ntt, nrt);
    else if (dtype == kQ6K)
      hipLaunchKernelGGL((mma_kq_kernel<kQ6K>), dim3((unsigned)nwg), dim3(256), lds, st, w, x, L.y, L.rows, L.bpr,
                         L.batch, ntt, nrt);
    else
      return NRQ_LAUNCH_BAD_ARG;
  }
  return hipGetLastError() == hipSuccess ? 0 : NRQ_LAUNCH_FAILED;
}

}  // namespace nrq
