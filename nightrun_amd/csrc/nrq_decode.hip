// Decode matvec, scalar f32 order, weights streamed straight from HBM into
// registers. Bit-identical to the reference's scalar kernels:
//   dot_q8_scalar  (crates/nr-tensor/src/kernels.rs:72-82)
//   dot_q4k_scalar (crates/nr-tensor/src/kquant.rs:192-218)
//   dot_q6k_scalar (crates/nr-tensor/src/kquant.rs:220-250)
// inside the row loops of matvec_q8 (kernels.rs:36-70) and kquant_matvec!
// (kquant.rs:536-564).
//
// Mapping. A small group of lanes owns one row and walks its blocks in
// order, so the reference's `sumf += contribution` chain is a register in
// lane 0 of the group:
//   Q4_K : a quad per row; lane c holds qs chunk c of the block (sub-blocks
//          2c and 2c+1); the 8 integer sub-dots reach every lane of the quad
//          through quad_perm DPP broadcasts and are summed in j order.
//   Q6_K : a quad per row; lane c = (half h, group parity u) holds the 16
//          quants of groups 8h+2n+u (n = 0..3); 16 group sums, broadcast by
//          DPP, summed in g order.
//   Q8_0 : an octet per row; lane j holds blocks 8t+j, and lane 0 adds the
//          octet's 8 contributions in block order (row_shl DPP).
// Each lane issues the loads of D blocks ahead (double-buffered), and the
// activation is staged once per workgroup in LDS with a padded layout that
// keeps the quads' simultaneous reads on distinct banks.
#include "nrq_device.h"
#include "nrq_launch.h"

namespace nrq {

// ---- cross-lane helpers ---------------------------------------------------------

template <int K>
__device__ __forceinline__ int quad_bcast(int v) {  // lane K of this quad
  return __builtin_amdgcn_mov_dpp(v, K * 0x55, 0xF, 0xF, false);
}

template <int N>
__device__ __forceinline__ float row_shl(float v) {  // value of lane (this + N) in the 16-lane row
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 + N, 0xF, 0xF, false));
}

__device__ __forceinline__ int quad_sum(int v) {
  v += __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);  // quad_perm(1,0,3,2)
  v += __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);  // quad_perm(2,3,0,1)
  return v;
}

// Dwords [a, a + N) of global memory, a 4-byte aligned.
template <int N>
__device__ __forceinline__ void gload(const uint8_t* __restrict__ p, uint32_t v[N]) {
  const uint32_t* q = (const uint32_t*)p;
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int i = 0; i < N / 4; i++) {
      u32x4 t = *((const u32x4*)(q + 4 * i));
      v[4 * i] = t.x;
      v[4 * i + 1] = t.y;
      v[4 * i + 2] = t.z;
      v[4 * i + 3] = t.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = *(q + i);
  }
}

// ---- activation staging ------------------------------------------------------------

// Padded LDS layouts (dwords per activation block):
//   Q8_0 : [qs 8][d 1][pad 3]                                     12
//   Q4_K : per chunk c: [qs 16][bsums pair 2c][bsums pair 2c+1][pad 2] x4, [d] [pad 3]   84
//   Q6_K : per half h: [qs 32][pad 8] x2, [group corr 16], [d] [pad 3]                    100
constexpr int kXs80 = 12;
constexpr int kXs4K = 84;
constexpr int kXs6K = 100;

template <int FMT>
__host__ __device__ constexpr int xs_dwords() {
  return FMT == kQ8_0 ? kXs80 : (FMT == kQ4K ? kXs4K : kXs6K);
}

// Cooperative copy of the bpr activation blocks at X (standard layout) into
// the padded LDS layout. `raw` is LDS scratch of x_raw bytes.
template <int FMT, int NT>
__device__ void stage_x_padded(const uint8_t* __restrict__ X, int bpr, uint32_t* xl, uint32_t* raw) {
  const int tid = threadIdx.x;
  const uintptr_t xa = (uintptr_t)X;
  const uint32_t xskew = (uint32_t)(xa & 3u);
  const uint32_t* src = (const uint32_t*)(xa - xskew);
  const int nx = (int)((xskew + (size_t)bpr * (FMT == kQ8_0 ? kQ8_0Bytes : kQ8KBytes) + 3) >> 2);
  constexpr int U = 8;
  for (int i0 = 0; i0 < nx; i0 += U * NT) {
    uint32_t v[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      int i = i0 + tid + u * NT;
      if (i < nx) v[u] = src[i];
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      int i = i0 + tid + u * NT;
      if (i < nx) raw[i] = v[u];
    }
  }
  __syncthreads();
  if constexpr (FMT == kQ8_0) {
    const uint8_t* rb = (const uint8_t*)raw;
    for (int i = tid; i < bpr * 9; i += NT) {
      int b = i / 9, t = i - b * 9;
      uint32_t o = xskew + (uint32_t)b * kQ8_0Bytes;
      uint32_t* dst = xl + b * kXs80;
      if (t < 8) dst[t] = lds_u32_even(raw, o + 2 + 4 * t);
      else dst[8] = __float_as_uint(f16_bits_to_f32(lds_u16(rb, o)));
    }
  } else {
    // Q8_K block = 73 dwords: d @0, qs @1..64, bsums @65..72.
    for (int i = tid; i < bpr * 64; i += NT) {
      int b = i >> 6, t = i & 63;
      uint32_t v = raw[b * 73 + 1 + t];
      if constexpr (FMT == kQ4K) xl[b * kXs4K + (t >> 4) * 20 + (t & 15)] = v;
      else xl[b * kXs6K + (t >> 5) * 40 + (t & 31)] = v;
    }
    for (int i = tid; i < bpr * 16; i += NT) {
      int b = i >> 4, g = i & 15;
      if constexpr (FMT == kQ4K) {
        if (g < 8) {  // bsums[2g] + bsums[2g+1] for sub-block g, beside chunk g/2
          uint32_t v = raw[b * 73 + 65 + g];
          int s = (int)(int16_t)(v & 0xffffu) + (int)(int16_t)(v >> 16);
          xl[b * kXs4K + (g >> 1) * 20 + 16 + (g & 1)] = (uint32_t)s;
        } else if (g == 8) {
          xl[b * kXs4K + 80] = raw[b * 73];
        }
      } else {
        // -32 * (sum of the group's 16 quants): the (q - 32) term of the scalar dot
        int s = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) s = sdot4(raw[b * 73 + 1 + 4 * g + k], 0xe0e0e0e0u, s);
        xl[b * kXs6K + 80 + g] = (uint32_t)s;
        if (g == 0) xl[b * kXs6K + 96] = raw[b * 73];
      }
    }
  }
  __syncthreads();
}

// ---- Q4_K: quad per row --------------------------------------------------------------

struct Q4KLane {
  uint32_t h[4];  // d|dmin, scales[0..4), scales[4..8), scales[8..12)
  uint32_t q[8];  // qs chunk c (32 bytes)
};

__device__ __forceinline__ void q4k_load(const uint8_t* __restrict__ blk, int c, Q4KLane& L) {
  gload<4>(blk, L.h);
  gload<8>(blk + 16 + 32 * c, L.q);
}

// One block's contribution d_all*sum_q - dmin_all*f32(sum_m) (kquant.rs:195-215),
// identical in every lane of the quad.
__device__ __forceinline__ float q4k_block(const Q4KLane& L, int c, const uint32_t* xb) {
  const uint32_t* xc = xb + 20 * c;
  int lo = 0, hi = 0;
#pragma unroll
  for (int t = 0; t < 8; t++) {
    lo = sdot4(L.q[t] & 0x0f0f0f0fu, xc[t], lo);
    hi = sdot4((L.q[t] >> 4) & 0x0f0f0f0fu, xc[8 + t], hi);
  }
  int sc[8], mn[8];
  q4k_unpack_scales(L.h[1], L.h[2], L.h[3], sc, mn);
  // this lane's sub-blocks are j = 2c, 2c+1
  int sl = c == 0 ? sc[0] : c == 1 ? sc[2] : c == 2 ? sc[4] : sc[6];
  int sh = c == 0 ? sc[1] : c == 1 ? sc[3] : c == 2 ? sc[5] : sc[7];
  int ml = c == 0 ? mn[0] : c == 1 ? mn[2] : c == 2 ? mn[4] : mn[6];
  int mh = c == 0 ? mn[1] : c == 1 ? mn[3] : c == 2 ? mn[5] : mn[7];
  const int tl = sl * lo, th = sh * hi;  // f32(sc)*f32(sub) == f32(sc*sub): |sc*sub| < 2^24
  const int sum_m = quad_sum(ml * (int)xc[16] + mh * (int)xc[17]);
  const int T[8] = {quad_bcast<0>(tl), quad_bcast<0>(th), quad_bcast<1>(tl), quad_bcast<1>(th),
                    quad_bcast<2>(tl), quad_bcast<2>(th), quad_bcast<3>(tl), quad_bcast<3>(th)};
  float sum_q = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; j++) sum_q = sum_q + (float)T[j];
  const float xd = __uint_as_float(xb[80]);
  const float d_all = f16_bits_to_f32(L.h[0] & 0xffffu) * xd;
  const float dmin_all = f16_bits_to_f32(L.h[0] >> 16) * xd;
  const float a = d_all * sum_q;
  const float m = dmin_all * (float)sum_m;
  return a - m;
}

// ---- Q6_K: quad per row ------------------------------------------------------------------

struct Q6KLane {
  uint32_t a[5], b[5], h[5];  // ql[64h+16u..], ql[64h+32+16u..], qh[32h+16u..] (+1 dword for realign)
  uint32_t s[3];              // scales[8h .. 8h+8) (+1 dword)
  uint32_t d;                 // dword holding d
};

__device__ __forceinline__ void q6k_load(const uint8_t* __restrict__ W, size_t boff, int hh, int u, Q6KLane& L) {
  const uint8_t* base = W + (boff & ~(size_t)3);
  const int o = (int)(boff & 3);  // 0 or 2
  gload<5>(base + 64 * hh + 16 * u, L.a);
  gload<5>(base + 64 * hh + 32 + 16 * u, L.b);
  gload<5>(base + 128 + 32 * hh + 16 * u, L.h);
  gload<3>(base + 192 + 8 * hh, L.s);
  (void)o;
  // bytes 208..211 past `base`: d sits in the low half (o = 0) or high half (o = 2)
  L.d = *((const uint32_t*)(base + 208));
}

// One block's contribution d_all * sum (kquant.rs:223-247), identical in every
// lane of the quad. `o` is the block's byte offset mod 4.
__device__ __forceinline__ float q6k_block(const Q6KLane& L, int hh, int u, uint32_t o, const uint32_t* xb) {
  const uint32_t* xh = xb + 40 * hh;
  int gs[4];
#pragma unroll
  for (int n = 0; n < 4; n++) gs[n] = (int)xb[80 + 8 * hh + 2 * n + u];
#pragma unroll
  for (int t = 0; t < 4; t++) {
    uint32_t q6[4];
    q6k_planes(__builtin_amdgcn_alignbyte(L.a[t + 1], L.a[t], o), __builtin_amdgcn_alignbyte(L.b[t + 1], L.b[t], o),
               __builtin_amdgcn_alignbyte(L.h[t + 1], L.h[t], o), q6);
#pragma unroll
    for (int n = 0; n < 4; n++) gs[n] = sdot4(q6[n], xh[8 * n + 4 * u + t], gs[n]);
  }
  const uint32_t s0 = __builtin_amdgcn_alignbyte(L.s[1], L.s[0], o);  // scales[8h .. 8h+4)
  const uint32_t s1 = __builtin_amdgcn_alignbyte(L.s[2], L.s[1], o);  // scales[8h+4 .. 8h+8)
  int T[4];
  T[0] = (int)(int8_t)((s0 >> (8 * u)) & 0xffu) * gs[0];        // sc[8h + u]
  T[1] = (int)(int8_t)((s0 >> (8 * u + 16)) & 0xffu) * gs[1];   // sc[8h + 2 + u]
  T[2] = (int)(int8_t)((s1 >> (8 * u)) & 0xffu) * gs[2];        // sc[8h + 4 + u]
  T[3] = (int)(int8_t)((s1 >> (8 * u + 16)) & 0xffu) * gs[3];   // sc[8h + 6 + u]
  // g = 8h + 2n + u lives in lane 2h + u, slot n. f32(sc)*f32(gs) == f32(sc*gs): |sc*gs| < 2^24.
  float sum = 0.0f;
#pragma unroll
  for (int hq = 0; hq < 2; hq++) {
#pragma unroll
    for (int n = 0; n < 4; n++) {
      int v0 = hq == 0 ? quad_bcast<0>(T[n]) : quad_bcast<2>(T[n]);
      int v1 = hq == 0 ? quad_bcast<1>(T[n]) : quad_bcast<3>(T[n]);
      sum = sum + (float)v0;
      sum = sum + (float)v1;
    }
  }
  const uint32_t dbits = o ? (L.d >> 16) : (L.d & 0xffffu);
  const float d_all = f16_bits_to_f32(dbits) * __uint_as_float(xb[96]);
  return d_all * sum;
}

// ---- Q8_0: octet per row -------------------------------------------------------------------

struct Q80Lane {
  uint32_t w[9];  // the 9 dwords from floor4(boff): the block's 34 bytes start at byte boff & 3
};

// The window [floor4(boff), +36) never starts before the block and ends at
// most 2 bytes past it, inside the dword holding the block's last bytes.
__device__ __forceinline__ void q80_load(const uint8_t* __restrict__ W, size_t boff, Q80Lane& L) {
  const uint8_t* p = W + (boff & ~(size_t)3);
  gload<8>(p, L.w);
  L.w[8] = *((const uint32_t*)(p + 32));
}

// contribution (f32(acc) * dw) * dx (kernels.rs:75-79)
__device__ __forceinline__ float q80_block(const Q80Lane& L, size_t boff, const uint32_t* xb) {
  const bool o2 = (boff & 2) != 0;  // block starts 2 bytes into its first dword
  int acc = 0;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    // qs dword i: bytes 2+4i.. of the block = window bytes o+2+4i..
    const uint32_t q = o2 ? L.w[i + 1] : __builtin_amdgcn_alignbyte(L.w[i + 1], L.w[i], 2);
    acc = sdot4(q, xb[i], acc);
  }
  const uint32_t dbits = o2 ? (L.w[0] >> 16) : (L.w[0] & 0xffffu);
  const float t = (float)acc * f16_bits_to_f32(dbits);
  return t * __uint_as_float(xb[8]);
}

// ---- kernels ----------------------------------------------------------------------------

constexpr int kDecodeD = 4;  // blocks per lane in flight per buffer

template <int NW>
__global__ __launch_bounds__(64 * NW) void q4k_decode(const uint8_t* __restrict__ W, const uint8_t* __restrict__ X,
                                                      float* __restrict__ Y, int rows, int bpr) {
  extern __shared__ __align__(16) uint32_t lds[];
  const int lane = threadIdx.x & 63;
  const int c = lane & 3;
  const int row = (blockIdx.x * NW + (threadIdx.x >> 6)) * 16 + (lane >> 2);
  const int rr = row < rows ? row : rows - 1;
  const uint8_t* wrow = W + (size_t)rr * bpr * kQ4KBytes;
  constexpr int D = kDecodeD;
  Q4KLane buf[2][D];
#pragma unroll
  for (int i = 0; i < D; i++)
    if (i < bpr) q4k_load(wrow + (size_t)i * kQ4KBytes, c, buf[0][i]);
  uint32_t* xl = lds;
  stage_x_padded<kQ4K, 64 * NW>(X, bpr, xl, lds + bpr * kXs4K);
  float s = 0.0f;
  for (int b0 = 0; b0 < bpr; b0 += 2 * D) {
#pragma unroll
    for (int i = 0; i < D; i++)
      if (b0 + D + i < bpr) q4k_load(wrow + (size_t)(b0 + D + i) * kQ4KBytes, c, buf[1][i]);
#pragma unroll
    for (int i = 0; i < D; i++)
      if (b0 + i < bpr) s = s + q4k_block(buf[0][i], c, xl + (b0 + i) * kXs4K);
#pragma unroll
    for (int i = 0; i < D; i++)
      if (b0 + 2 * D + i < bpr) q4k_load(wrow + (size_t)(b0 + 2 * D + i) * kQ4KBytes, c, buf[0][i]);
#pragma unroll
    for (int i = 0; i < D; i++)
      if (b0 + D + i < bpr) s = s + q4k_block(buf[1][i], c, xl + (b0 + D + i) * kXs4K);
  }
  if (c == 0 && row < rows) Y[row] = s;
}

template <int NW>
__global__ __launch_bounds__(64 * NW) void q6k_decode(const uint8_t* __restrict__ W, const uint8_t* __restrict__ X,
                                                      float* __restrict__ Y, int rows, int bpr) {
  extern __shared__ __align__(16) uint32_t lds[];
  const int lane = threadIdx.x & 63;
  const int c = lane & 3, hh = c >> 1, u = c & 1;
  const int row = (blockIdx.x * NW + (threadIdx.x >> 6)) * 16 + (lane >> 2);
  const int rr = row < rows ? row : rows - 1;
  const size_t roff = (size_t)rr * bpr * kQ6KBytes;
  constexpr int D = kDecodeD;
  Q6KLane buf[2][D];
#pragma unroll
  for (int i = 0; i < D; i++)
    if (i < bpr) q6k_load(W, roff + (size_t)i * kQ6KBytes, hh, u, buf[0][i]);
  uint32_t* xl = lds;
  stage_x_padded<kQ6K, 64 * NW>(X, bpr, xl, lds + bpr * kXs6K);
  float s = 0.0f;
  for (int b0 = 0; b0 < bpr; b0 += 2 * D) {
#pragma unroll
    for (int i = 0; i < D; i++)
      if (b0 + D + i < bpr) q6k_load(W, roff + (size_t)(b0 + D + i) * kQ6KBytes, hh, u, buf[1][i]);
#pragma unroll
    for (int i = 0; i < D; i++)
      if (b0 + i < bpr)
        s = s + q6k_block(buf[0][i], hh, u, (uint32_t)((roff + (size_t)(b0 + i) * kQ6KBytes) & 3),
                          xl + (b0 + i) * kXs6K);
#pragma unroll
    for (int i = 0; i < D; i++)
      if (b0 + 2 * D + i < bpr) q6k_load(W, roff + (size_t)(b0 + 2 * D + i) * kQ6KBytes, hh, u, buf[0][i]);
#pragma unroll
    for (int i = 0; i < D; i++)
      if (b0 + D + i < bpr)
        s = s + q6k_block(buf[1][i], hh, u, (uint32_t)((roff + (size_t)(b0 + D + i) * kQ6KBytes) & 3),
                          xl + (b0 + D + i) * kXs6K);
  }
  if (c == 0 && row < rows) Y[row] = s;
}

// Adds the octet's 8 contributions (lanes j = 0..7 hold blocks 8t+j) to the
// running sum of lane 0, in block order; `n` of them are real.
__device__ __forceinline__ float octet_chain(float s, float u, int n) {
  const float v1 = row_shl<1>(u), v2 = row_shl<2>(u), v3 = row_shl<3>(u), v4 = row_shl<4>(u);
  const float v5 = row_shl<5>(u), v6 = row_shl<6>(u), v7 = row_shl<7>(u);
  s = s + u;
  if (n > 1) s = s + v1;
  if (n > 2) s = s + v2;
  if (n > 3) s = s + v3;
  if (n > 4) s = s + v4;
  if (n > 5) s = s + v5;
  if (n > 6) s = s + v6;
  if (n > 7) s = s + v7;
  return s;
}

template <int NW>
__global__ __launch_bounds__(64 * NW) void q80_decode(const uint8_t* __restrict__ W, const uint8_t* __restrict__ X,
                                                      float* __restrict__ Y, int rows, int bpr) {
  extern __shared__ __align__(16) uint32_t lds[];
  const int lane = threadIdx.x & 63;
  const int j = lane & 7;
  const int row = (blockIdx.x * NW + (threadIdx.x >> 6)) * 8 + (lane >> 3);
  const int rr = row < rows ? row : rows - 1;
  const size_t roff = (size_t)rr * bpr * kQ8_0Bytes;
  const int steps = (bpr + 7) >> 3;
  constexpr int D = 2 * kDecodeD;
  Q80Lane buf[2][D];
  // lane j's t-th block is 8t+j; lanes past the row end load block bpr-1 and
  // are dropped from the chain
#define Q80_BOFF(t) (roff + (size_t)min(8 * (t) + j, bpr - 1) * kQ8_0Bytes)
#pragma unroll
  for (int i = 0; i < D; i++)
    if (i < steps) q80_load(W, Q80_BOFF(i), buf[0][i]);
  uint32_t* xl = lds;
  stage_x_padded<kQ8_0, 64 * NW>(X, bpr, xl, lds + bpr * kXs80);
  float s = 0.0f;
  for (int t0 = 0; t0 < steps; t0 += 2 * D) {
#pragma unroll
    for (int i = 0; i < D; i++)
      if (t0 + D + i < steps) q80_load(W, Q80_BOFF(t0 + D + i), buf[1][i]);
#pragma unroll
    for (int i = 0; i < D; i++)
      if (t0 + i < steps) {
        const int t = t0 + i;
        const int b = min(8 * t + j, bpr - 1);
        float uc = q80_block(buf[0][i], Q80_BOFF(t), xl + b * kXs80);
        s = octet_chain(s, uc, bpr - 8 * t);
      }
#pragma unroll
    for (int i = 0; i < D; i++)
      if (t0 + 2 * D + i < steps) q80_load(W, Q80_BOFF(t0 + 2 * D + i), buf[0][i]);
#pragma unroll
    for (int i = 0; i < D; i++)
      if (t0 + D + i < steps) {
        const int t = t0 + D + i;
        const int b = min(8 * t + j, bpr - 1);
        float uc = q80_block(buf[1][i], Q80_BOFF(t), xl + b * kXs80);
        s = octet_chain(s, uc, bpr - 8 * t);
      }
  }
#undef Q80_BOFF
  if (j == 0 && row < rows) Y[row] = s;
}

// ---- launch ---------------------------------------------------------------------------------

template <int FMT>
static size_t decode_lds_bytes(int bpr) {
  const size_t xl = (size_t)bpr * xs_dwords<FMT>() * 4;
  const size_t raw = (size_t)bpr * (FMT == kQ8_0 ? kQ8_0Bytes : kQ8KBytes) + 16;
  return xl + raw;
}

int launch_decode_scalar(int dtype, const MatvecLaunch& L) {
  if (L.rows <= 0 || L.bpr <= 0) return 0;
  const int rows_per_wave = dtype == kQ8_0 ? 8 : 16;
  const int waves = (L.rows + rows_per_wave - 1) / rows_per_wave;
  // four waves per workgroup share one activation copy when there are
  // enough rows to keep every CU busy; one wave otherwise
  const bool wide = waves >= 4 * 256 * 2;
  const int nw = wide ? 4 : 1;
  const int grid = (waves + nw - 1) / nw;
  size_t lds;
  if (dtype == kQ8_0) lds = decode_lds_bytes<kQ8_0>(L.bpr);
  else if (dtype == kQ4K) lds = decode_lds_bytes<kQ4K>(L.bpr);
  else lds = decode_lds_bytes<kQ6K>(L.bpr);
  if (lds > 160 * 1024) return NRQ_LAUNCH_TOO_WIDE;
  hipStream_t st = (hipStream_t)L.stream;
  const uint8_t* w = (const uint8_t*)L.w;
  const uint8_t* x = (const uint8_t*)L.x;
  if (dtype == kQ8_0) {
    if (wide) hipLaunchKernelGGL(q80_decode<4>, dim3(grid), dim3(256), lds, st, w, x, L.y, L.rows, L.bpr);
    else hipLaunchKernelGGL(q80_decode<1>, dim3(grid), dim3(64), lds, st, w, x, L.y, L.rows, L.bpr);
  } else if (dtype == kQ4K) {
    if (wide) hipLaunchKernelGGL(q4k_decode<4>, dim3(grid), dim3(256), lds, st, w, x, L.y, L.rows, L.bpr);
    else hipLaunchKernelGGL(q4k_decode<1>, dim3(grid), dim3(64), lds, st, w, x, L.y, L.rows, L.bpr);
  } else if (dtype == kQ6K) {
    if (wide) hipLaunchKernelGGL(q6k_decode<4>, dim3(grid), dim3(256), lds, st, w, x, L.y, L.rows, L.bpr);
    else hipLaunchKernelGGL(q6k_decode<1>, dim3(grid), dim3(64), lds, st, w, x, L.y, L.rows, L.bpr);
  } else {
    return NRQ_LAUNCH_BAD_ARG;
  }
  return hipGetLastError() == hipSuccess ? 0 : NRQ_LAUNCH_FAILED;
}

}  // namespace nrq
