// Device-side building blocks shared by the gfx950 kernels of libnrq.
//
// Block layouts are the reference's GGUF-compatible ones, read in place:
//   Q8_0 : d:f16@0  qs:i8[32]@2                                   34 B  (q8.rs:9-17)
//   Q4_K : d:f16@0  dmin:f16@2  scales:u8[12]@4  qs:u8[128]@16     144 B (kquant.rs:26-31)
//   Q6_K : ql:u8[128]@0  qh:u8[64]@128  scales:i8[16]@192  d:f16@208 210 B (kquant.rs:37-42)
//   Q8_K : d:f32@0  qs:i8[256]@4  bsums:i16[16]@260               292 B (kquant.rs:48-52)
//
// All f32 arithmetic in these kernels is written out operation by operation;
// the library is compiled with -ffp-contract=off so a*b+c stays two rounded
// operations wherever the reference has two, and fmaf() is used exactly where
// the reference's AVX2 kernels use _mm256_fmadd_ps.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nrq {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef short short2_t __attribute__((ext_vector_type(2)));

constexpr int kQ8_0 = 1;  // TensorDtype ids (crates/nr-model/src/format.rs:97-102)
constexpr int kQ4K = 2;
constexpr int kQ6K = 3;

constexpr int kOrderScalar = 0;  // dot_*_scalar (and the NEON kernels, bit for bit)
constexpr int kOrderAvx2 = 1;    // dot_*_avx2 / dot_*_avx2_x4

constexpr int kQ8_0Bytes = 34;
constexpr int kQ4KBytes = 144;
constexpr int kQ6KBytes = 210;
constexpr int kQ8KBytes = 292;

// IEEE binary16 -> f32. The hardware conversion is exact for every finite
// and infinite f16 (f16 denormals are enabled in the kernel float mode), so it
// equals the reference's softfloat f16_to_f32 (f16.rs:3-23) bit for bit on
// all non-NaN inputs; NaNs stay NaN.
__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits16) {
  _Float16 h;
  uint16_t b = (uint16_t)bits16;
  __builtin_memcpy(&h, &b, 2);
  return (float)h;
}

// Exact 4-way int8 dot product with accumulate (v_dot4_i32_i8).
__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Exact dot of two i16 pairs packed in dwords, with accumulate (v_dot2_i32_i16).
// The operands are taken by value as plain dwords: a bit cast applied
// directly to an ext-vector element can read the wrong element.
__device__ __forceinline__ int sdot2(uint32_t a, uint32_t b, int c) {
  short2_t sa, sb;
  __builtin_memcpy(&sa, &a, 4);
  __builtin_memcpy(&sb, &b, 4);
  return __builtin_amdgcn_sdot2(sa, sb, c, false);
}

// Dword starting at an even LDS byte offset `off` (2- or 4-aligned):
// two aligned reads and a byte funnel shift.
__device__ __forceinline__ uint32_t lds_u32_even(const uint32_t* lds32, uint32_t off) {
  uint32_t w = off >> 2;
  return __builtin_amdgcn_alignbyte(lds32[w + 1], lds32[w], off & 3u);
}

__device__ __forceinline__ uint32_t lds_u16(const uint8_t* lds, uint32_t off) {
  return *(const uint16_t*)(lds + off);
}

// Q4_K 6-bit (scale, min) unpack for all j = 0..7 (kquant.rs:83-92).
// s0,s1,s2 hold scales[0..4], scales[4..8], scales[8..12] little-endian.
__device__ __forceinline__ void q4k_unpack_scales(uint32_t s0, uint32_t s1, uint32_t s2, int sc[8], int mn[8]) {
#pragma unroll
  for (int j = 0; j < 4; j++) {
    uint32_t a = (s0 >> (8 * j)) & 0xffu;  // scales[j]
    uint32_t b = (s1 >> (8 * j)) & 0xffu;  // scales[j+4]
    uint32_t c = (s2 >> (8 * j)) & 0xffu;  // scales[j+8]
    sc[j] = (int)(a & 63u);
    mn[j] = (int)(b & 63u);
    sc[j + 4] = (int)((c & 0x0fu) | ((a >> 6) << 4));
    mn[j + 4] = (int)((c >> 4) | ((b >> 6) << 4));
  }
}

// The four 6-bit planes of a Q6_K half for one l-dword (4 consecutive l),
// following the scalar unpack of kquant.rs:233-237: plane n holds quants
// n*32 + l of the half.
__device__ __forceinline__ void q6k_planes(uint32_t qlA, uint32_t qlB, uint32_t qh, uint32_t q6[4]) {
  const uint32_t m4 = 0x0f0f0f0fu, m2h = 0x30303030u;
  q6[0] = (qlA & m4) | ((qh << 4) & m2h);
  q6[1] = (qlB & m4) | ((qh << 2) & m2h);
  q6[2] = ((qlA >> 4) & m4) | (qh & m2h);
  q6[3] = ((qlB >> 4) & m4) | ((qh >> 2) & m2h);
}

// f16.rs:25-56: round to nearest even for normal results, round half up
// for subnormal ones, a quiet NaN without payload. Every case is formed and
// the result picked by selects: no divergent branches.
__device__ __forceinline__ uint32_t f32_to_f16_bits(float v) {
  const uint32_t bits = __float_as_uint(v);
  const uint32_t sign = (bits >> 16) & 0x8000u;
  const int exp = (int)((bits >> 23) & 0xffu);
  const uint32_t frac = bits & 0x7fffffu;
  const int e = exp - 127 + 15;
  // e in 1 .. 30: the top ten fraction bits, then the 13 dropped ones round
  uint32_t nrm = sign | ((uint32_t)e << 10) | (frac >> 13);
  const uint32_t rnd = frac & 0x1fffu;
  nrm += (rnd > 0x1000u || (rnd == 0x1000u && (nrm & 1u) != 0)) ? 1u : 0u;
  // e in -10 .. 0: the significand shifted right by 14 - e, half up
  const uint32_t sh = (uint32_t)min(max(14 - e, 14), 24);
  const uint32_t sub = sign | (((frac | 0x800000u) + (1u << (sh - 1))) >> sh);
  // e >= 31: infinity, or a quiet NaN for exp 0xff with a nonzero fraction
  const uint32_t big = sign | 0x7c00u | (exp == 0xff && frac != 0 ? 0x200u : 0u);
  uint32_t out = e <= 0 ? (e < -10 ? sign : sub) : nrm;
  out = e >= 0x1f ? big : out;
  return out & 0xffffu;
}

// Rust `f as i32`: truncate toward zero, saturate to [i32::MIN, i32::MAX],
// NaN -> 0. That is what v_cvt_i32_f32 does; checked against the three-way
// restatement of those rules on all 2^32 f32 inputs on gfx950.
__device__ __forceinline__ int rust_f32_to_i32(float f) {
  int r;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(f));
  return r;
}

// kquant.rs:145-153 (the two sums formed, one picked: no branch)
__device__ __forceinline__ int nearest_int(float v) {
  const float up = v + 0.5f, down = v - 0.5f;
  return rust_f32_to_i32(v >= 0.0f ? up : down);
}

// One Q8_K block (kquant.rs:157-187) from 32 lanes of a half-wave, lane r
// holding values 8r .. 8r+7 of the block: the first index of the largest |v|
// (a strict `>` scan; NaN never wins), iscale = -128 / v[that index],
// q = min(nearest_int(iscale * v), 127), d = 1 / iscale, an all-zero block
// when the largest |v| is not > 0. Returns lane r's 8 quants (lo, hi), the
// 16-value sum of lanes r & ~1 and r | 1 (ps), and d's f32 bits.
__device__ __forceinline__ void q8k_half_lanes(const float o[8], int r, uint32_t* lo_out, uint32_t* hi_out,
                                               int* ps_out, uint32_t* d_bits_out) {
  // this lane's largest |v| and its first value holding it
  float al = -1.0f, mine = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; e++) {
    float ae = fabsf(o[e]);
    if (ae != ae) ae = -1.0f;
    if (ae > al) {
      al = ae;
      mine = o[e];
    }
  }
  // the half-wave's largest: max over quads and 16-lane rows (DPP), then the
  // row pair; no NaN is left, so the max is exact in any order
  float a = al;
  a = fmaxf(a, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0xB1, 0xF, 0xF, false)));
  a = fmaxf(a, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x4E, 0xF, 0xF, false)));
  a = fmaxf(a, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x124, 0xF, 0xF, false)));
  a = fmaxf(a, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x128, 0xF, 0xF, false)));
  a = fmaxf(a, __shfl_xor(a, 16, 32));
  // the first index holding it: the first such lane of the half-wave, its first such value
  const unsigned long long has = __ballot(al == a);
  const uint32_t hw = (uint32_t)(has >> (__lane_id() & 32));
  const float mx = __shfl(mine, (int)__builtin_ctz(hw | 0x80000000u), 32);
  const bool zero = !(a > 0.0f);
  const float iscale = -128.0f / mx;
  int q[8];
  int p = 0;
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const int t = nearest_int(iscale * o[e]);
    q[e] = zero ? 0 : (t > 127 ? 127 : t);
    p += q[e];
  }
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    lo |= (uint32_t)(q[e] & 0xff) << (8 * e);
    hi |= (uint32_t)(q[4 + e] & 0xff) << (8 * e);
  }
  *lo_out = lo;
  *hi_out = hi;
  *ps_out = p + __builtin_amdgcn_update_dpp(0, p, 0xB1, 0xF, 0xF, false);  // lane r ^ 1 (quad_perm [1,0,3,2])
  *d_bits_out = zero ? 0u : __float_as_uint(1.0f / iscale);
}

// Lane r's part of the 292-byte Q8_K block at gout (4-byte aligned): its 8
// quants, bsums[r / 2] from the even lanes, d from lane 0.
__device__ __forceinline__ void q8k_half_store(uint8_t* gout, int r, uint32_t lo, uint32_t hi, int ps,
                                               uint32_t d_bits) {
  *(uint32_t*)(gout + 4 + 8 * r) = lo;
  *(uint32_t*)(gout + 8 + 8 * r) = hi;
  if ((r & 1) == 0) *(int16_t*)(gout + 260 + r) = (int16_t)ps;
  if (r == 0) *(uint32_t*)gout = d_bits;
}

// q8::quantize (q8.rs:27-44) of one 32-value block held one value per lane of
// a 32-lane group: amax over the group, d = f16(amax / 127), round half away
// from zero, clamp to [-127, 127]. Returns this lane's quant and the f16 bits of d.
__device__ __forceinline__ int q8_0_lane(float v, uint32_t* d_bits_out) {
  // max over quads (DPP quad_perm), then over each 16-lane row (DPP row_ror
  // 4 and 8), then across the two rows of the group: max is exact in any order
  float amax = fabsf(v);
  amax = fmaxf(amax, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(amax), 0xB1, 0xF, 0xF, false)));
  amax = fmaxf(amax, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(amax), 0x4E, 0xF, 0xF, false)));
  amax = fmaxf(amax, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(amax), 0x124, 0xF, 0xF, false)));
  amax = fmaxf(amax, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(amax), 0x128, 0xF, 0xF, false)));
  amax = fmaxf(amax, __shfl_xor(amax, 16, 32));
  amax = fmaxf(0.0f, amax);
  const uint32_t d_bits = f32_to_f16_bits(amax / 127.0f);
  const float d = f16_bits_to_f32(d_bits);
  const float inv = d > 0.0f ? 1.0f / d : 0.0f;
  const float xi = v * inv;
  const float r = xi >= 0.0f ? xi + 0.5f : xi - 0.5f;
  int q = rust_f32_to_i32(r);
  q = q < -127 ? -127 : (q > 127 ? 127 : q);
  *d_bits_out = d_bits;
  return q;
}

// q8::quantize (q8.rs:27-44) of one 32-value block held as eight consecutive
// values in each lane of an aligned lane quad (lane & 3 = eighth of the block).
// The block amax is exact in any order, so a quad DPP max reduction gives the
// reference's value. Returns the eight quants packed little-endian in two
// dwords and the f16 bits of d.
__device__ __forceinline__ float dpp_quad_xor1(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));  // [1,0,3,2]
}
__device__ __forceinline__ float dpp_quad_xor2(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));  // [2,3,0,1]
}
// Max over the 64 lanes of a wave (every lane active), in every lane: DPP
// within quads and 16-lane rows, then two cross-row exchanges. fmaxf is
// exact and ignores NaN in any order.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_quad_xor1(v));
  v = fmaxf(v, dpp_quad_xor2(v));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false)));
  v = fmaxf(v, __shfl_xor(v, 16));
  v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}
__device__ __forceinline__ void q8_0_quad8(const float o[8], uint32_t* lo, uint32_t* hi, uint32_t* d_bits_out) {
  float amax = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(o[e]));
  amax = fmaxf(amax, dpp_quad_xor1(amax));
  amax = fmaxf(amax, dpp_quad_xor2(amax));
  const uint32_t d_bits = f32_to_f16_bits(amax / 127.0f);
  const float d = f16_bits_to_f32(d_bits);
  const float inv = d > 0.0f ? 1.0f / d : 0.0f;
  uint32_t w[2] = {0u, 0u};
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const float xi = o[e] * inv;
    const float r = xi >= 0.0f ? xi + 0.5f : xi - 0.5f;
    int q = rust_f32_to_i32(r);
    q = q < -127 ? -127 : (q > 127 ? 127 : q);
    w[e >> 2] |= ((uint32_t)q & 0xffu) << (8 * (e & 3));
  }
  *lo = w[0];
  *hi = w[1];
  *d_bits_out = d_bits;
}

// Sequential f32 sum s + a[0] + a[1] + ... + a[n-1], in index order, by
// one lane: the reference's `s += v` loops. Three banks of four 16-byte LDS
// loads rotate: a bank is refilled 48 values ahead right after it is added, so
// the dependent adds rarely wait on a load. a is 16-byte aligned.
__device__ inline float chain_from(const float* __restrict__ a, int n, float s) {
  const float4* a4 = (const float4*)a;
  const int n16 = n >> 4;  // groups of 16 values
  int g = 0;
  if (n16 >= 3) {
    float4 R0[4], R1[4], R2[4];
    // The running sum passes through the empty asm statements around each
    // group's loads, so the loads stay right after the adds that free their
    // registers: left alone, the compiler moves them next to their first use
    // and the whole load latency is paid once per group.
    auto ld = [&](float4* R, int gg) {
      asm volatile("" : "+v"(s) : : "memory");
#pragma unroll
      for (int k = 0; k < 4; k++) R[k] = a4[4 * gg + k];
      asm volatile("" : "+v"(s) : : "memory");
    };
    auto add = [&](const float4* R) {
#pragma unroll
      for (int k = 0; k < 4; k++) {
        s = s + R[k].x;
        s = s + R[k].y;
        s = s + R[k].z;
        s = s + R[k].w;
      }
    };
    ld(R0, 0);
    ld(R1, 1);
    ld(R2, 2);
    for (; g + 6 <= n16; g += 3) {  // groups g .. g+2 are loaded
      add(R0);
      ld(R0, g + 3);
      add(R1);
      ld(R1, g + 4);
      add(R2);
      ld(R2, g + 5);
    }
    // groups g .. g+2 loaded, fewer than three groups left after them
    add(R0);
    if (g + 3 < n16) ld(R0, g + 3);
    add(R1);
    if (g + 4 < n16) ld(R1, g + 4);
    add(R2);
    if (g + 5 < n16) ld(R2, g + 5);
    if (g + 3 < n16) add(R0);
    if (g + 4 < n16) add(R1);
    if (g + 5 < n16) add(R2);
    g = n16;
  }
  for (int i = 16 * g; i < n; i++) s = s + a[i];
  return s;
}
__device__ inline float chain_sum(const float* __restrict__ a, int n) { return chain_from(a, n, 0.0f); }

// The same sequential sum, s + a[0] + ... + a[n-1] in index order, run by a
// whole wave (all 64 lanes active, a in LDS, 4-byte aligned); the result is
// valid in lane 0. Lanes 0-15 load 16 consecutive values into one VGPR and
// lane 0 adds them in order, reading lane k through a DPP row shift
// (row_shl:k). Eight such VGPRs keep 128 values in flight ahead of the adds.
// The first n & ~127 values take this path, the rest a plain loop.
#define NRQ_DPP_ADD(b, k) "v_add_f32_dpp %0, %" #b ", %0 row_shl:" #k " row_mask:0xf bank_mask:0xf\n"
#define NRQ_DPP_ADD16(b)                                                                                 \
  "v_add_f32_e32 %0, %" #b ", %0\n" NRQ_DPP_ADD(b, 1) NRQ_DPP_ADD(b, 2) NRQ_DPP_ADD(b, 3) NRQ_DPP_ADD(b, 4) \
      NRQ_DPP_ADD(b, 5) NRQ_DPP_ADD(b, 6) NRQ_DPP_ADD(b, 7) NRQ_DPP_ADD(b, 8) NRQ_DPP_ADD(b, 9)              \
          NRQ_DPP_ADD(b, 10) NRQ_DPP_ADD(b, 11) NRQ_DPP_ADD(b, 12) NRQ_DPP_ADD(b, 13) NRQ_DPP_ADD(b, 14)     \
              NRQ_DPP_ADD(b, 15)
#define NRQ_DPP_LD(b, off) "ds_read_b32 %" #b ", %10 offset:" #off "\n"
__device__ inline float wave_chain_from(const float* __restrict__ a, int n, float s) {
  const int n128 = n & ~127;
  if (n128 > 0) {
    uint32_t addr = (uint32_t)(uintptr_t)a + 4u * (uint32_t)(threadIdx.x & 15);
    int iters = __builtin_amdgcn_readfirstlane(n128 >> 7);
    float b0, b1, b2, b3, b4, b5, b6, b7;
    // Iteration i adds values 128i .. 128i+127 (VGPR b holds 128i + 16b + lane)
    // and, unless it is the last, refills each VGPR for iteration i + 1 right
    // after adding it; LDS reads return in order, so lgkmcnt(7) means the
    // oldest of the eight outstanding reads has landed.
    asm volatile(
        NRQ_DPP_LD(1, 0) NRQ_DPP_LD(2, 64) NRQ_DPP_LD(3, 128) NRQ_DPP_LD(4, 192) NRQ_DPP_LD(5, 256)
            NRQ_DPP_LD(6, 320) NRQ_DPP_LD(7, 384) NRQ_DPP_LD(8, 448)
        "s_nop 4\n"
        "1:\n"
        "s_sub_u32 %9, %9, 1\n"
        "s_cmp_eq_u32 %9, 0\n"
        "s_cbranch_scc1 2f\n"
        "s_waitcnt lgkmcnt(7)\n" NRQ_DPP_ADD16(1) NRQ_DPP_LD(1, 512)
        "s_waitcnt lgkmcnt(7)\n" NRQ_DPP_ADD16(2) NRQ_DPP_LD(2, 576)
        "s_waitcnt lgkmcnt(7)\n" NRQ_DPP_ADD16(3) NRQ_DPP_LD(3, 640)
        "s_waitcnt lgkmcnt(7)\n" NRQ_DPP_ADD16(4) NRQ_DPP_LD(4, 704)
        "s_waitcnt lgkmcnt(7)\n" NRQ_DPP_ADD16(5) NRQ_DPP_LD(5, 768)
        "s_waitcnt lgkmcnt(7)\n" NRQ_DPP_ADD16(6) NRQ_DPP_LD(6, 832)
        "s_waitcnt lgkmcnt(7)\n" NRQ_DPP_ADD16(7) NRQ_DPP_LD(7, 896)
        "s_waitcnt lgkmcnt(7)\n" NRQ_DPP_ADD16(8) NRQ_DPP_LD(8, 960)
        "v_add_u32_e32 %10, 0x200, %10\n"
        "s_branch 1b\n"
        "2:\n"
        "s_waitcnt lgkmcnt(7)\n" NRQ_DPP_ADD16(1)
        "s_waitcnt lgkmcnt(6)\n" NRQ_DPP_ADD16(2)
        "s_waitcnt lgkmcnt(5)\n" NRQ_DPP_ADD16(3)
        "s_waitcnt lgkmcnt(4)\n" NRQ_DPP_ADD16(4)
        "s_waitcnt lgkmcnt(3)\n" NRQ_DPP_ADD16(5)
        "s_waitcnt lgkmcnt(2)\n" NRQ_DPP_ADD16(6)
        "s_waitcnt lgkmcnt(1)\n" NRQ_DPP_ADD16(7)
        "s_waitcnt lgkmcnt(0)\n" NRQ_DPP_ADD16(8)
        : "+v"(s), "=&v"(b0), "=&v"(b1), "=&v"(b2), "=&v"(b3), "=&v"(b4), "=&v"(b5), "=&v"(b6), "=&v"(b7),
          "+s"(iters), "+v"(addr)
        :
        : "memory", "scc");
  }
  for (int i = n128; i < n; i++) s = s + a[i];
  return s;
}
#undef NRQ_DPP_LD
#undef NRQ_DPP_ADD16
#undef NRQ_DPP_ADD

// Inclusive prefix sum over the wave's 64 lanes (all active): row shifts
// within each 16-lane row, then the row totals through row_bcast:15/31.
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t x) {
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xf, 0xf, false);  // row_shr:1
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xf, 0xf, false);  // row_shr:2
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xf, 0xf, false);  // row_shr:4
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xf, 0xf, false);  // row_shr:8
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xa, 0xf, false);  // row_bcast:15 -> rows 1, 3
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xc, 0xf, false);  // row_bcast:31 -> rows 2, 3
  return x;
}

// Inclusive prefix sum of f32 over the wave (any association: a prediction only).
__device__ __forceinline__ float wave_incl_scan_f32(float x) {
  x = x + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x111, 0xf, 0xf, false));
  x = x + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x112, 0xf, 0xf, false));
  x = x + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x114, 0xf, 0xf, false));
  x = x + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x118, 0xf, 0xf, false));
  x = x + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x142, 0xa, 0xf, false));
  x = x + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x143, 0xc, 0xf, false));
  return x;
}

__device__ __forceinline__ int f32_exp(float x) { return (int)((__float_as_uint(x) >> 23) & 0xffu) - 127; }

// One pass of wg_chain_nonneg over a[0 .. m), m <= 64 * NW * RL, run by all NW
// waves of a workgroup with the same s: s <- s + a[0] + ... + a[m-1] exactly as
// the sequential f32 chain gives it, the same value in every lane of every
// wave. Returns false in every wave (s unchanged) when the pass cannot vouch
// for its result; the caller then runs the plain chain over the same terms.
//
// While the running sum s is a normal float in one binade [2^E, 2^(E+1)), it is
// a multiple of the binade's unit u = 2^(E-23), and so is every rounded s + a.
// Round-to-nearest-even of s + a then equals s + (a rounded to a multiple of u)
// as long as the exact s + a stays below 2^(E+1), except when a is an odd half
// of u away from a multiple (a tie, whose direction depends on s). So with
// S = s / u, an integer in [2^23, 2^24], a run of terms in one binade is S plus
// an integer prefix sum of the terms' roundings, exact in 32-bit integers.
//
// Lane g = 64 * wave + lane takes terms RL*g .. RL*g + RL-1. An approximate f32
// prefix sum (its association does not matter) predicts the binade each term
// is added in. Each term is rounded with the unit of its predicted binade,
// except the terms after which the predicted binade changes (crossings) and
// ties: those "special" terms count 0 in the integer prefix sum and are added
// as ordinary f32 adds, in order, by a chain that checks each prediction
// against the exact sum: each run of terms between special ones must end below
// 2^(E+1) in the binade predicted for it, and each special term must land in
// the binade predicted after it. (The binade predicted before a special term is
// the one predicted after the previous special term, or s's own for the first:
// lane 0 predicts from s itself, and the predicted binade only changes at
// special terms. Across a wave boundary the last lane's prediction after its
// last term and the next wave's first prediction are the same f32 value,
// s + the waves' totals added in wave order by every wave alike.)
// A term that is negative or not finite, and a sum outside [2^-100, 2^127),
// fail the pass.
//
// The waves exchange their f32 totals, then their integer totals and special
// counts, through work; the lanes holding special terms write each one's
// integer prefix, predicted binade after it and value to its place in term
// order, and every wave then resolves the special terms alike: only their f32
// adds run one at a time, every check runs on all of them at once afterwards.
// work: kWgChainWork words of LDS that nothing else touches during the pass.
constexpr int kWgMaxSpecial = 48;  // past this many, the plain chain is cheaper
constexpr int kWgChainWork = 64 + 3 * kWgMaxSpecial;
template <int NW, int RL>
__device__ __forceinline__ bool wg_chain_pass(const float* __restrict__ a, int m, float& s, uint32_t* __restrict__ work) {
  static_assert(RL % 4 == 0, "whole 16-byte reads per lane");
  static_assert(NW >= 1 && NW <= 16, "the exchange holds up to sixteen waves");
  const uint32_t sb = __builtin_amdgcn_readfirstlane(__float_as_uint(s));
  if (sb - 0x0d800000u >= 0x7f000000u - 0x0d800000u) return false;  // positive, biased exponent 27 .. 253
  const float s_in = __uint_as_float(sb);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int base = RL * (64 * wave + lane);
  uint32_t* xf = work;        // [wave]: the wave's f32 total; [16 + wave]: it holds a non-finite term
  uint32_t* xr = work + 32;   // [wave]: the wave's integer total; [16 + wave]: its special count
  uint32_t* spb = work + 64;  // special term k: the integer prefix before it,
  uint32_t* spa = spb + kWgMaxSpecial;  // the binade predicted after it,
  uint32_t* spt = spa + kWgMaxSpecial;  // the term
  // a wave past the last term (its lanes would hold only zeros) skips the
  // per-term work and takes part in the exchanges with zero totals
  const bool busy = RL * 64 * wave < m;
  float av[RL];
  float inclW = 0.0f;
  bool nonfinite = false;
  if (busy) {
    const float4* a4 = (const float4*)a;
    const int last4 = (m >> 2) - 1;
#pragma unroll
    for (int k = 0; k < RL / 4; k++) {
      const float4 v = a4[min(base / 4 + k, last4)];
      av[4 * k] = v.x;
      av[4 * k + 1] = v.y;
      av[4 * k + 2] = v.z;
      av[4 * k + 3] = v.w;
    }
    uint32_t mx = 0u;
    float tot = 0.0f;
#pragma unroll
    for (int j = 0; j < RL; j++) {
      av[j] = base + j < m ? av[j] : 0.0f;
      mx = max(mx, __float_as_uint(av[j]));
      tot = tot + av[j];
    }
    nonfinite = __ballot(mx >= 0x7f800000u) != 0;  // every term a finite float >= +0
    inclW = wave_incl_scan_f32(tot);
  } else {
#pragma unroll
    for (int j = 0; j < RL; j++) av[j] = 0.0f;
  }
  if (lane == 63) {
    xf[wave] = __float_as_uint(inclW);
    xf[16 + wave] = nonfinite ? 1u : 0u;
  }
  __syncthreads();
  // the waves' totals before this wave and through it, added in wave order
  float offW = 0.0f, offN = 0.0f;
  bool bad_term = false;
#pragma unroll
  for (int i = 0; i < NW; i++) {
    const float t = __uint_as_float(xf[i]);
    bad_term |= xf[16 + i] != 0u;
    if (i < wave) offW = offW + t;
    if (i <= wave) offN = offN + t;
  }
  if (bad_term) {
    __syncthreads();  // every wave has read xf before a next pass may write it again
    return false;
  }
  uint32_t ef[RL + 1];  // exponent field of the predicted sum before term j
  uint32_t cum[RL], special = 0u, racc = 0u, incl = 0u, cnt = 0u, cincl = 0u;  // cum[j]: the lane's roundings before term j
  if (busy) {
    const float exclW = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(inclW), 0x138, 0xf, 0xf, false));  // wave_shr:1
    const float p0 = s_in + (offW + exclW);  // predicted sum before the lane's first term
    float p = p0;
#pragma unroll
    for (int j = 0; j < RL; j++) {
      ef[j] = __float_as_uint(p) & 0x7f800000u;
      p = p + av[j];
    }
    // after the lane's last term: the next lane's first prediction (wave_shl:1);
    // the last lane's is the next wave's first, s + offN (s + the total after the last wave)
    ef[RL] = (uint32_t)__builtin_amdgcn_update_dpp(__float_as_int(s_in + offN), __float_as_int(p0), 0x130, 0xf, 0xf, false) &
             0x7f800000u;
#pragma unroll
    for (int j = 0; j < RL; j++) {
      const float q = av[j] * __uint_as_float(0x8a800000u - ef[j]);  // a / u: a power-of-two scaling
      const uint32_t r = (uint32_t)__builtin_rintf(q);
      // only real terms are special: the zeros past m add nothing, and a zero in a
      // lane's last slot may sit between two predictions made in different orders
      const bool sp = base + j < m && (ef[j] != ef[j + 1] || __builtin_amdgcn_fractf(q) == 0.5f);
      cum[j] = racc;
      racc += sp ? 0u : r;  // r <= 2^24, so the lane's sum stays below 2^28
      special |= (sp ? 1u : 0u) << j;
    }
    incl = wave_incl_scan_u32(racc);  // wraps harmlessly: only run differences are used
    cnt = (uint32_t)__builtin_popcount(special);
    cincl = wave_incl_scan_u32(cnt);
  } else {
#pragma unroll
    for (int j = 0; j < RL; j++) {
      ef[j] = 0u;
      cum[j] = 0u;
    }
    ef[RL] = 0u;
  }
  if (lane == 63) {
    xr[wave] = incl;
    xr[16 + wave] = cincl;
  }
  __syncthreads();
  uint32_t offR = 0u, total = 0u, offC = 0u, K = 0u;
#pragma unroll
  for (int i = 0; i < NW; i++) {
    const uint32_t r = xr[i], c = xr[16 + i];
    if (i < wave) {
      offR += r;
      offC += c;
    }
    total += r;
    K += c;
  }
  const uint32_t excl = offR + incl - racc;
  uint32_t Ef = sb & 0x7f800000u;  // exponent field of the exact running sum
  uint32_t bstart = 0u;            // the integer prefix where the current run starts
  uint32_t S = (sb & 0x7fffffu) | 0x800000u;
  if (K != 0u) {
    if (K > (uint32_t)kWgMaxSpecial) return false;
    // the lane's special terms, in order, to their places in term order
    uint32_t rem = special, slot = offC + cincl - cnt;
    while (rem != 0u) {
      const int j = __builtin_ctz(rem);
      uint32_t b = 0u, af = 0u, tb = 0u;
#pragma unroll
      for (int jj = 0; jj < RL; jj++) {  // selects, not an indexed register read
        b = jj == j ? cum[jj] : b;
        af = jj == j ? ef[jj + 1] : af;
        tb = jj == j ? __float_as_uint(av[jj]) : tb;
      }
      spb[slot] = excl + b;
      spa[slot] = af;
      spt[slot] = tb;
      slot++;
      rem &= rem - 1u;
    }
    __syncthreads();
    const uint32_t g_before = lane < (int)K ? spb[lane] : 0u;
    const uint32_t g_after = lane < (int)K ? spa[lane] : 0u;
    const float g_term = lane < (int)K ? __uint_as_float(spt[lane]) : 0.0f;
    // the previous special term's prefix and binade after (the pass start's in lane 0)
    uint32_t p_before = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)g_before, 0x138, 0xf, 0xf, false);
    const uint32_t p_after = (uint32_t)__builtin_amdgcn_update_dpp((int)Ef, (int)g_after, 0x138, 0xf, 0xf, false);
    // kept out of the subtraction: folded into it, as v_subrev_u32_dpp, the
    // shift gave the difference with the opposite sign on gfx950
    asm volatile("" : "+v"(p_before));
    const uint32_t pre = g_before - p_before;                   // the run before the special term
    const float unit = __uint_as_float(p_after - (23u << 23));  // that run's unit
    // S in a vector register: the chain below stays on the vector unit
    uint32_t Sv = S, nbv = 0u;
    asm volatile("" : "+v"(Sv));
    for (int k = 0; k < (int)K; k++) {
      const uint32_t X = Sv + (uint32_t)__builtin_amdgcn_readlane((int)pre, k);
      const float se = (float)X * __int_as_float(__builtin_amdgcn_readlane(__float_as_int(unit), k));  // exact when X < 2^24
      const uint32_t nb = __float_as_uint(se + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(g_term), k)));
      Sv = (nb & 0x7fffffu) | 0x800000u;
      nbv = lane == k ? nb : nbv;
    }
    // lane k: the sum after special term k (nbv) and before it (S of the previous one, plus the run)
    const uint32_t p_nb = (uint32_t)__builtin_amdgcn_update_dpp((int)sb, (int)nbv, 0x138, 0xf, 0xf, false);
    const uint32_t X = ((p_nb & 0x7fffffu) | 0x800000u) + pre;
    const bool bad = lane < (int)K && ((pre >= (1u << 24)) | (X >= (1u << 24)) |
                                       (nbv - 0x0d800000u >= 0x7f000000u - 0x0d800000u) | ((nbv & 0x7f800000u) != g_after));
    if (__ballot(bad) != 0) return false;
    S = __builtin_amdgcn_readfirstlane(Sv);
    Ef = (uint32_t)__builtin_amdgcn_readlane((int)g_after, K - 1);
    bstart = (uint32_t)__builtin_amdgcn_readlane((int)g_before, K - 1);
  }
  const uint32_t pre = total - bstart;
  if (pre > (1u << 24) || S + pre > (1u << 24)) return false;  // exactly 2^(E+1) is exact too
  s = (float)(S + pre) * __uint_as_float(Ef - (23u << 23));
  return true;
}

__device__ __forceinline__ float wave_lane0_f32(float v) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}

// s + a[0] + a[1] + a[2] + ... + a[15] in index order (a 16-byte aligned),
// the same value in every lane
__device__ __forceinline__ float chain_head16(const float* __restrict__ a, float s) {
  const float4* a4 = (const float4*)a;
  const float4 v0 = a4[0], v1 = a4[1], v2 = a4[2], v3 = a4[3];
  const float4 v[4] = {v0, v1, v2, v3};
#pragma unroll
  for (int k = 0; k < 4; k++) {
    s = s + v[k].x;
    s = s + v[k].y;
    s = s + v[k].z;
    s = s + v[k].w;
  }
  return s;
}

// wave_chain_from's result, bit for bit, for terms that are finite and
// nonnegative (squares, exps), computed by all NW waves of a workgroup together
// and returned in every lane of every wave: the first 16 terms take the plain
// chain in every lane alike (the pass needs a positive running sum to start
// from), then passes of up to 64 * NW * MAXRL terms (wg_chain_pass, 4 or 8
// terms per lane when that covers them) each fall back to the plain chain when
// they cannot vouch for their result; a last run of fewer than 512 terms is
// cheaper on the plain chain. Every thread of the workgroup calls it with the
// same arguments (a in LDS, 16-byte aligned, n a multiple of 4); work is
// kWgChainWork words of LDS that nothing else touches meanwhile. Every wave has
// finished reading a when any wave returns, so a may be written right after
// the call.
template <int NW, int MAXRL = 16>
__device__ __forceinline__ float wg_chain_nonneg(const float* __restrict__ a, int n, float s, uint32_t* __restrict__ work) {
  static_assert(MAXRL == 4 || MAXRL == 8 || MAXRL == 16, "4, 8 or 16 terms per lane");
  // a plain chain read a after the last barrier of a successful pass (the
  // decisions below are the same in every wave, so the barrier is reached by all)
  bool plain_after = true;
  if (n < 16 + 512) {
    s = wave_lane0_f32(wave_chain_from(a, n, s));
  } else {
    s = chain_head16(a, s);
    int i = 16;
    while (n - i >= 512) {
      const int m = min(n - i, 64 * NW * MAXRL);
      bool ok;
      if (MAXRL == 4 || m <= 64 * NW * 4) ok = wg_chain_pass<NW, 4>(a + i, m, s, work);
      else if (MAXRL == 8 || m <= 64 * NW * 8) ok = wg_chain_pass<NW, 8>(a + i, m, s, work);
      else ok = wg_chain_pass<NW, 16>(a + i, m, s, work);
      if (!ok) s = wave_lane0_f32(wave_chain_from(a + i, m, s));
      plain_after = !ok;
      i += m;
    }
    if (n > i) {
      s = wave_lane0_f32(wave_chain_from(a + i, n - i, s));
      plain_after = true;
    }
  }
  if (plain_after) __syncthreads();
  return s;
}

// musl scalbnf
__device__ __forceinline__ float dev_scalbnf(float x, int n) {
  float y = x;
  if (n > 127) {
    y *= __uint_as_float(0x7f000000u);
    n -= 127;
    if (n > 127) {
      y *= __uint_as_float(0x7f000000u);
      n -= 127;
      if (n > 127) n = 127;
    }
  } else if (n < -126) {
    y *= __uint_as_float(0x00800000u) * __uint_as_float(0x4b800000u);
    n += 126 - 24;
    if (n < -126) {
      y *= __uint_as_float(0x00800000u) * __uint_as_float(0x4b800000u);
      n += 126 - 24;
      if (n < -126) n = -126;
    }
  }
  return y * __uint_as_float((uint32_t)(0x7f + n) << 23);
}

// musl expf (FreeBSD e_expf.c algorithm): x = k ln2 + r, exp(r) from the
// two-term Remez form, scaled by 2^k.
__device__ inline float dev_expf(float x) {
  const float ln2hi = 6.9314575195e-01f, ln2lo = 1.4286067653e-06f, invln2 = 1.4426950216e+00f;
  const float P1 = 1.6666625440e-1f, P2 = -2.7667332906e-3f;
  uint32_t hx = __float_as_uint(x);
  const int sign = (int)(hx >> 31);
  hx &= 0x7fffffffu;
  if (hx >= 0x42aeac50u) {
    if (hx > 0x7f800000u) return x;
    if (hx >= 0x42b17218u && !sign) return x * __uint_as_float(0x7f000000u);
    if (sign && hx >= 0x42cff1b5u) return 0.0f;
  }
  int k;
  float hi, lo;
  if (hx > 0x3eb17218u) {
    if (hx > 0x3f851592u)
      k = (int)(invln2 * x + (sign ? -0.5f : 0.5f));
    else
      k = 1 - sign - sign;
    const float kf = (float)k;
    hi = x - kf * ln2hi;
    lo = kf * ln2lo;
    x = hi - lo;
  } else if (hx > 0x39000000u) {
    k = 0;
    hi = x;
    lo = 0.0f;
  } else {
    return 1.0f + x;
  }
  const float xx = x * x;
  const float c = x - xx * (P1 + xx * P2);
  const float y = 1.0f + (x * c / (2.0f - c) - lo + hi);
  return k == 0 ? y : dev_scalbnf(y, k);
}

}  // namespace nrq
