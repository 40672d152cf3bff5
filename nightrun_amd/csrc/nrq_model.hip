// Llama-family decode on one GPU, every tensor resident in HBM: the forward
// pass of crates/nr-model/src/infer.rs (InferCtx::forward, infer.rs:510-595)
// with greedy sampling (sample.rs:32-35), bit-identical to the reference's
// scalar kernels. The quantized matvecs are libnrq's decode kernels; this file
// holds the f32 steps between them, each written in the reference's order:
//   rmsnorm   (crates/nr-tensor/src/vec.rs:4-14): sequential sum of squares
//   rope      (crates/nr-tensor/src/rope.rs:49-65): adjacent pairs, sincosf
//   KV append (infer.rs:547-551): f32 -> f16 softfloat (f16.rs:25-56)
//   attention (infer.rs:553-572): dot_f16 / softmax / axpy_f16 in position order
//   swiglu    (vec.rs:45-52), residual saxpy (vec.rs:63-67), argmax (vec.rs:80-90)
// expf and sincosf restate the published musl single-precision algorithms that
// the reference's libm crate (0.2.16) ports.
//
// The step is device-driven: the current token and position live in device
// memory, the embedding kernel reads the token and the argmax kernel writes
// the next one and advances the position, so a whole greedy step is one fixed
// kernel sequence (replayed as a HIP graph by nrq_model_generate).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "../../include/nrq.h"
#include "nrq_device.h"
#include "nrq_launch.h"

namespace nrq {

// ---- libm restatements (device) -------------------------------------------------

namespace {

// __sindf / __cosdf: double polynomials on [-pi/4, pi/4]
__device__ __forceinline__ float dev_sindf(double x) {
  const double S1 = -0x15555554cbac77.0p-55, S2 = 0x111110896efbb2.0p-59;
  const double S3 = -0x1a00f9e2cae774.0p-65, S4 = 0x16cd878c3b46a7.0p-71;
  const double z = x * x, w = z * z, r = S3 + z * S4, s = z * x;
  return (float)((x + s * (S1 + z * S2)) + s * w * r);
}
__device__ __forceinline__ float dev_cosdf(double x) {
  const double C0 = -0x1ffffffd0c5e81.0p-54, C1 = 0x155553e1053a42.0p-57;
  const double C2 = -0x16c087e80f1e27.0p-62, C3 = 0x199342e0ee5069.0p-68;
  const double z = x * x, w = z * z, r = C2 + z * C3;
  return (float)(((1.0 + z * C0) + w * C1) + (w * z) * r);
}

// __rem_pio2f, medium path (|x| < 2^28 pi/2; rope angles stay far below)
__device__ __forceinline__ int dev_rem_pio2f(float x, double* y) {
  const double toint = 1.5 / 2.220446049250313e-16, pio4 = 0x1.921fb6p-1;
  const double invpio2 = 6.36619772367581382433e-01, pio2_1 = 1.57079631090164184570e+00;
  const double pio2_1t = 1.58932547735281966916e-08;
  if ((__float_as_uint(x) & 0x7fffffffu) < 0x4dc90fdbu) {
    double fn = (double)x * invpio2 + toint - toint;
    int n = (int)fn;
    *y = x - fn * pio2_1 - fn * pio2_1t;
    if (*y < -pio4) {
      n--;
      fn--;
      *y = x - fn * pio2_1 - fn * pio2_1t;
    } else if (*y > pio4) {
      n++;
      fn++;
      *y = x - fn * pio2_1 - fn * pio2_1t;
    }
    return n;
  }
  *y = __builtin_nan("");
  return 0;
}

// musl sincosf
__device__ void dev_sincosf(float x, float* sn, float* cs) {
  const double s1pio2 = 1 * 1.57079632679489661923, s2pio2 = 2 * 1.57079632679489661923;
  const double s3pio2 = 3 * 1.57079632679489661923, s4pio2 = 4 * 1.57079632679489661923;
  uint32_t ix = __float_as_uint(x);
  const unsigned sign = ix >> 31;
  ix &= 0x7fffffffu;
  if (ix <= 0x3f490fdau) {
    if (ix < 0x39800000u) {
      *sn = x;
      *cs = 1.0f;
      return;
    }
    *sn = dev_sindf(x);
    *cs = dev_cosdf(x);
    return;
  }
  if (ix <= 0x407b53d1u) {
    if (ix <= 0x4016cbe3u) {
      if (sign) {
        *sn = -dev_cosdf(x + s1pio2);
        *cs = dev_sindf(x + s1pio2);
      } else {
        *sn = dev_cosdf(s1pio2 - x);
        *cs = dev_sindf(s1pio2 - x);
      }
      return;
    }
    *sn = -dev_sindf(sign ? x + s2pio2 : x - s2pio2);
    *cs = -dev_cosdf(sign ? x + s2pio2 : x - s2pio2);
    return;
  }
  if (ix <= 0x40e231d5u) {
    if (ix <= 0x40afeddfu) {
      if (sign) {
        *sn = dev_cosdf(x + s3pio2);
        *cs = -dev_sindf(x + s3pio2);
      } else {
        *sn = -dev_cosdf(x - s3pio2);
        *cs = dev_sindf(x - s3pio2);
      }
      return;
    }
    *sn = dev_sindf(sign ? x + s4pio2 : x - s4pio2);
    *cs = dev_cosdf(sign ? x + s4pio2 : x - s4pio2);
    return;
  }
  if (ix >= 0x7f800000u) {
    *sn = *cs = x - x;
    return;
  }
  double y;
  const unsigned n = (unsigned)dev_rem_pio2f(x, &y);
  const float s = dev_sindf(y), c = dev_cosdf(y);
  switch (n & 3) {
    case 0: *sn = s; *cs = c; break;
    case 1: *sn = c; *cs = -s; break;
    case 2: *sn = -s; *cs = -c; break;
    default: *sn = -c; *cs = s; break;
  }
}


// One 32-value Q8_0 block held one value per lane of a 32-lane group, written
// to blk in the BlockQ8_0 layout.
__device__ __forceinline__ void quant_q8_0_lane(float v, int lane32, uint8_t* __restrict__ blk) {
  uint32_t d_bits;
  const int q = q8_0_lane(v, &d_bits);
  blk[2 + lane32] = (uint8_t)(int8_t)q;
  if (lane32 == 0) {
    blk[0] = (uint8_t)(d_bits & 0xff);
    blk[1] = (uint8_t)(d_bits >> 8);
  }
}

// Control words in device memory.
enum { CTL_TOKEN = 0, CTL_POS = 1, CTL_STEP = 2, CTL_WORDS = 4 };

// ---- kernels ------------------------------------------------------------------------

// ctl[i0] = v0 and, when i1 >= 0, ctl[i1] = v1. Host values reach the control
// words as kernel arguments, so no host buffer has to outlive the enqueueing call.
__global__ void ctl_set_kernel(int* __restrict__ ctl, int i0, int v0, int i1, int v1) {
  if (threadIdx.x == 0) {
    ctl[i0] = v0;
    if (i1 >= 0) ctl[i1] = v1;
  }
}

// QMat::dequant_row (infer.rs:36-56), element i of row `row` (cols values):
//  Q8_0 (q8.rs:47-55): f32(q) * d;
//  Q4_K (kquant.rs:95-116): element 64c + k takes the low nibble of qs[32c + k]
//    with scale/min pair 2c when k < 32, else the high nibble of qs[32c + k - 32]
//    with pair 2c + 1: (d * sc) * q - dmin * m;
//  Q6_K (kquant.rs:118-142): in half h, element 32p + l takes plane p of
//    (ql, qh) at l: (d * sc[8h + l/16 + 2p]) * (q - 32).
__device__ inline float dequant_elem(const uint8_t* __restrict__ E, int dt, size_t row, int cols, int i) {
  if (dt == NRQ_Q4_K || dt == NRQ_Q6_K) {
    const size_t b = row * (size_t)(cols / 256) + (size_t)(i >> 8);
    const int e = i & 255;
    if (dt == NRQ_Q4_K) {
      const uint8_t* blk = E + b * 144;
      const float d = f16_bits_to_f32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
      const float dmin = f16_bits_to_f32((uint32_t)blk[2] | ((uint32_t)blk[3] << 8));
      const uint8_t* sc = blk + 4;
      const int c = e >> 6, k = e & 63, j = 2 * c + (k >> 5);
      uint32_t s, m;
      if (j < 4) {
        s = sc[j] & 63;
        m = sc[j + 4] & 63;
      } else {
        s = (sc[j + 4] & 0x0F) | ((sc[j - 4] >> 6) << 4);
        m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
      }
      const uint32_t qq = blk[16 + 32 * c + (k & 31)];
      const uint32_t q = k < 32 ? (qq & 0x0F) : (qq >> 4);
      const float d1 = d * (float)s, min1 = dmin * (float)m;
      return d1 * (float)q - min1;
    }
    const uint8_t* blk = E + b * 210;
    const int h = e >> 7, r = e & 127, p = r >> 5, l = r & 31;
    const uint8_t* ql = blk + 64 * h;
    const uint32_t qh = blk[128 + 32 * h + l];
    const uint32_t lo = (p & 1) ? ql[l + 32] : ql[l];
    const int q = (int)(((p & 2) ? (lo >> 4) : (lo & 0x0F)) | (((qh >> (2 * p)) & 3) << 4)) - 32;
    const float d = f16_bits_to_f32((uint32_t)blk[208] | ((uint32_t)blk[209] << 8));
    const float sc = (float)(int8_t)blk[192 + 8 * h + (l >> 4) + 2 * p];
    return d * sc * (float)q;
  }
  const uint8_t* blk = E + (row * (size_t)(cols / 32) + (size_t)(i >> 5)) * kQ8_0Bytes;
  const float d = f16_bits_to_f32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
  return (float)(int8_t)blk[2 + (i & 31)] * d;
}

// QMat::dequant_row for Q8_0 (infer.rs:37-42, q8.rs:47-55): x[i] = f32(q) * d
// Workgroup 0 also writes (cos, sin) of pos * freqs[i] for the step: rope::apply
// takes sincosf(pos * freq_i) for every head and layer alike (rope.rs:49-65).
__global__ void embed_kernel(const uint8_t* __restrict__ E, int dt, const int* __restrict__ ctl, int dim,
                                  float* __restrict__ x, const float* __restrict__ freqs, int half,
                                  float* __restrict__ rope_cs, float escale) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (blockIdx.x == 0 && (int)threadIdx.x < half) {
    float sn, cs;
    dev_sincosf((float)ctl[CTL_POS] * freqs[threadIdx.x], &sn, &cs);
    rope_cs[2 * threadIdx.x] = cs;
    rope_cs[2 * threadIdx.x + 1] = sn;
  }
  if (i >= dim) return;
  const float v = dequant_elem(E, dt, (size_t)(uint32_t)ctl[CTL_TOKEN], dim, i);
  x[i] = escale != 1.0f ? v * escale : v;  // muP embedding scale (infer.rs:519-521)
}

// Prefill: the embedding rows of B tokens (x[i][:]) and each token's (cos, sin)
// table at position base + i (base = ctl[CTL_POS]); grid (dim / 256, B).
__global__ void embed_rows_kernel(const uint8_t* __restrict__ E, int dt, const int* __restrict__ tokens,
                                       const int* __restrict__ ctl, int dim, float* __restrict__ x,
                                       const float* __restrict__ freqs, int half, float* __restrict__ rope_cs,
                                       float escale) {
  const int row = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (blockIdx.x == 0 && (int)threadIdx.x < half) {
    float sn, cs;
    dev_sincosf((float)(ctl[CTL_POS] + row) * freqs[threadIdx.x], &sn, &cs);
    rope_cs[(size_t)row * 2 * half + 2 * threadIdx.x] = cs;
    rope_cs[(size_t)row * 2 * half + 2 * threadIdx.x + 1] = sn;
  }
  if (i >= dim) return;
  const float v = dequant_elem(E, dt, (size_t)(uint32_t)tokens[row], dim, i);
  x[(size_t)row * dim + i] = escale != 1.0f ? v * escale : v;  // muP embedding scale (infer.rs:608-615)
}

constexpr int kNormNT = 512;
constexpr int kNormMax = 8192;
constexpr int kNormPT = kNormMax / kNormNT;  // values per thread

// Optional residual x += rs * add (saxpy, vec.rs:68-72; rs is residual_scale), then
// rmsnorm (vec.rs:4-14): ss += v*v in element order, scale = 1/sqrtf(ss/n + eps),
// out = x * scale * w. Writes out (f32) and, when xq != null, its Q8_0 blocks
// (q8.rs:27-44), when xqk != null its Q8_K blocks (kquant.rs:157-187). One
// workgroup of kNormNT threads; n <= kNormMax, a multiple of 256. Thread t owns
// the 8-value runs t + kNormNT k (four consecutive runs, an aligned lane quad,
// make one Q8_0 block; 32, an aligned half-wave, one Q8_K block), loaded once,
// all loads issued before the first use; all waves run the ordered sum of
// squares together. Workgroup r
// takes row r of [rows][n] x, add, out, xq and xqk (one row per workgroup in a
// prefill chunk).
__global__ __launch_bounds__(kNormNT) void norm_kernel(float* __restrict__ x, const float* __restrict__ add,
                                                       const float* __restrict__ w, int n, float eps, float rs,
                                                       float* __restrict__ out, uint8_t* __restrict__ xq,
                                                       uint8_t* __restrict__ xqk) {
  __shared__ __align__(16) float sq[kNormMax];
  __shared__ __align__(16) uint32_t chain_work[kWgChainWork];
  {
    const size_t r = blockIdx.x;
    x += r * n;
    if (add) add += r * n;
    out += r * n;
    if (xq) xq += r * (size_t)(n / 32) * kQ8_0Bytes;
    if (xqk) xqk += r * (size_t)(n / 256) * kQ8KBytes;
  }
  const int tid = threadIdx.x;
  const int nrun = n >> 3;
  constexpr int RK = kNormPT / 8;  // runs per thread
  float4 v[2 * RK], a[2 * RK], wv[2 * RK];
#pragma unroll
  for (int k = 0; k < RK; k++) {
    const int j = tid + kNormNT * k;
    if (j < nrun) {
      v[2 * k] = ((const float4*)x)[2 * j];
      v[2 * k + 1] = ((const float4*)x)[2 * j + 1];
      wv[2 * k] = ((const float4*)w)[2 * j];
      wv[2 * k + 1] = ((const float4*)w)[2 * j + 1];
      if (add) {
        a[2 * k] = ((const float4*)add)[2 * j];
        a[2 * k + 1] = ((const float4*)add)[2 * j + 1];
      }
    }
  }
#pragma unroll
  for (int k = 0; k < RK; k++) {
    const int j = tid + kNormNT * k;
    if (j < nrun) {
#pragma unroll
      for (int h = 0; h < 2; h++) {
        float4& p = v[2 * k + h];
        if (add) {
          const float4 q = a[2 * k + h];
          p.x = p.x + rs * q.x;
          p.y = p.y + rs * q.y;
          p.z = p.z + rs * q.z;
          p.w = p.w + rs * q.w;
          ((float4*)x)[2 * j + h] = p;
        }
        ((float4*)sq)[2 * j + h] = make_float4(p.x * p.x, p.y * p.y, p.z * p.z, p.w * p.w);
      }
    }
  }
  __syncthreads();
  const float ss = wg_chain_nonneg<kNormNT / 64>(sq, n, 0.0f, chain_work);  // every wave, the same result
  const float scale = 1.0f / sqrtf(ss / (float)n + eps);
#pragma unroll
  for (int k = 0; k < RK; k++) {
    const int j = tid + kNormNT * k;
    if (j < nrun) {
      const float4 p0 = v[2 * k], p1 = v[2 * k + 1], w0 = wv[2 * k], w1 = wv[2 * k + 1];
      float o[8] = {p0.x * scale * w0.x, p0.y * scale * w0.y, p0.z * scale * w0.z, p0.w * scale * w0.w,
                    p1.x * scale * w1.x, p1.y * scale * w1.y, p1.z * scale * w1.z, p1.w * scale * w1.w};
      ((float4*)out)[2 * j] = make_float4(o[0], o[1], o[2], o[3]);
      ((float4*)out)[2 * j + 1] = make_float4(o[4], o[5], o[6], o[7]);
      if (xq) {
        uint32_t lo, hi, d_bits;
        q8_0_quad8(o, &lo, &hi, &d_bits);
        uint8_t* blk = xq + (size_t)(j >> 2) * kQ8_0Bytes;
        uint16_t* qs = (uint16_t*)(blk + 2 + 8 * (j & 3));  // 2-byte aligned
        qs[0] = (uint16_t)lo;
        qs[1] = (uint16_t)(lo >> 16);
        qs[2] = (uint16_t)hi;
        qs[3] = (uint16_t)(hi >> 16);
        if ((j & 3) == 0) *(uint16_t*)blk = (uint16_t)d_bits;
      }
      if (xqk) {  // n is a multiple of 256: whole half-waves take this branch
        uint32_t lo, hi, d_bits;
        int ps;
        q8k_half_lanes(o, j & 31, &lo, &hi, &ps, &d_bits);
        q8k_half_store(xqk + (size_t)(j >> 5) * kQ8KBytes, j & 31, lo, hi, ps, d_bits);
      }
    }
  }
}

// Prefill: rope::apply (rope.rs:49-65) on every query and key head of token i
// = blockIdx.x at position base + i, queries in place, and the f16 KV append of
// its key and value rows (infer.rs:642-651). A chunk appends all its rows
// before any of its tokens attends, as prefill_chunk does. One wave per head,
// four heads per workgroup: blockIdx.y * 4 + wave indexes the query heads, then
// the key heads (whose waves also append the value row). With qn/kn (Qwen3),
// the head is first RMS-normalized (vec.rs:17-28, infer.rs:643-650): its
// squares are summed in element order by the wave (wave_chain_from), and
// x * (scale * w) is applied as the pair is rotated. Pair j of a head is
// (2j, 2j+1), or (j, j + hd/2) with neox. head_dim <= 128, a multiple of 32.
__global__ __launch_bounds__(256) void rope_append_kernel(float* __restrict__ q, const float* __restrict__ k,
                                                          const float* __restrict__ v,
                                                          const float* __restrict__ rope_cs,
                                                          const int* __restrict__ ctl, int n_heads, int n_kv_heads,
                                                          int hd, int ctx, int layer, uint16_t* __restrict__ kc,
                                                          uint16_t* __restrict__ vc, const float* __restrict__ qn,
                                                          const float* __restrict__ kn, float eps, int neox) {
  __shared__ __align__(16) float raw[4][128];
  __shared__ __align__(16) float sqs[4][128];
  const int i = blockIdx.x, w = threadIdx.x >> 6, lane = threadIdx.x & 63, half = hd / 2;
  const int h = (int)blockIdx.y * 4 + w;  // the wave's head: queries, then keys
  const bool live = h < n_heads + n_kv_heads, isq = h < n_heads;
  const int hh = isq ? h : h - n_heads;
  const int pos = ctl[CTL_POS] + i;
  float* qi = q + ((size_t)i * n_heads + hh) * hd;
  const float* src = isq ? (const float*)qi : k + ((size_t)i * n_kv_heads + hh) * hd;
  float* rw = raw[w];
  float* sq = sqs[w];
  if (live)
    for (int d = lane; d < hd; d += 64) {
      const float x = src[d];
      rw[d] = x;
      sq[d] = x * x;
    }
  __syncthreads();
  if (!live) return;
  float scale = 0.0f;
  if (qn) scale = 1.0f / sqrtf(wave_lane0_f32(wave_chain_from(sq, hd, 0.0f)) / (float)hd + eps);
  const float* cst = rope_cs + (size_t)i * hd;
  const float* nw = isq ? qn : kn;
  const size_t ctx8 = (size_t)ctx * 8;
  auto kvi = [&](int d) {
    return ((size_t)layer * n_kv_heads + hh) * hd * ctx + (size_t)(d >> 3) * ctx8 + (size_t)pos * 8 + (d & 7);
  };
  for (int j = lane; j < half; j += 64) {
    const int ia = neox ? j : 2 * j, ib = neox ? j + half : 2 * j + 1;
    const float cs = cst[2 * j], sn = cst[2 * j + 1];
    float a = rw[ia], b = rw[ib];
    if (qn) {
      a = a * (scale * nw[ia]);
      b = b * (scale * nw[ib]);
    }
    const float ra = a * cs - b * sn, rb = a * sn + b * cs;
    if (isq) {
      qi[ia] = ra;
      qi[ib] = rb;
    } else {
      kc[kvi(ia)] = (uint16_t)f32_to_f16_bits(ra);
      kc[kvi(ib)] = (uint16_t)f32_to_f16_bits(rb);
    }
  }
  if (!isq) {
    const float* vi = v + ((size_t)i * n_kv_heads + hh) * hd;
    for (int d = lane; d < hd; d += 64) vc[kvi(d)] = (uint16_t)f32_to_f16_bits(vi[d]);
  }
}

constexpr int kAttNT = 1024;
// Threads of attention_kernel: 1024, or 768 for 96- and 128-wide heads, whose
// key rows (16 pieces of 16 bytes per position) need the 168 registers per
// lane that twelve waves leave (sixteen waves leave 128, and spill)
__host__ __device__ constexpr int att_threads(int hd) { return hd >= 96 ? 768 : kAttNT; }
constexpr int kAttMaxCtx = 8192;
constexpr int kAttProd = 8704;  // floats per product stage (head_dim x (chunk + 4) <= 8704)
constexpr int kAttRing = 3 * 1024 * 16;  // bytes of the value ring: three chunks of at most 1024 pieces

// One workgroup per query head: the attention block of infer.rs:540-572.
//  1. Loads first (every key/value row but the current one is already in the
//     cache): the key rows of this thread's positions (two rounds of kAttNT
//     positions when they fit in registers) and, from the producer waves, DMA
//     requests of the first three chunks' value rows into an LDS ring. Then
//     rope::apply (rope.rs:49-65)
//     on the head's q and its KV head's k with the step's (cos, sin) table, and
//     the KV append as f16 (infer.rs:547-551) by the first query head of each
//     KV group. The fresh key/value are used from LDS, so the other heads of
//     the group never read the row being written.
//  2. scores: dot_f16(k_t, q) * scale (kernels.rs:146-160, dimension order).
//  3. softmax (vec.rs:30-42): max, exp, the exp-sum in position order (one
//     lane), inv, a_t = e_t * inv.
//  4. out[i] += a_t * v_t[i] in position order (kernels.rs:163-173). Chunks of
//     C positions: the producer waves form the products a_t * v_t[i] of the
//     next chunk in LDS, dimension-major (row stride C + 4 floats), from value
//     rows their DMA requests brought into the ring two chunks earlier; the
//     chain lanes (one per dimension) add the current chunk, four positions
//     per 16-byte LDS read.
//  5. out (f32) and, when out_q8 != null, its Q8_0 blocks for the output
//     projection.
// With PF (prefill), workgroup (h, i) serves token i of a chunk at position
// base + i: its query was roped by rope_append_kernel and every key and
// value row, its own included, is read from the cache (the chunk's rows were
// all appended before this launch); out and out_q8 are row i of [B][...].
// With DS > 1 (decode), DS workgroups serve one head: each runs steps 1-3
// for the whole head and step 4 for its HD / DS dimensions (the chain and the
// products of the other dimensions run on other CUs, whose LDS bandwidth the
// product stage and value ring would otherwise share). Workgroup b serves
// head 8 * (q / DS) + b % 8, dimension group q % DS (q = b / 8): the DS
// workgroups of a head share XCD b % 8 and its L2 (needs n_heads % 8 == 0).
// LDS: att[ctx] | prod[2][kAttProd] | q[hd] | kcur[hd] | vcur[hd] | red[32]
template <int HD, bool PF = false, int NT = att_threads(HD), int DS = 1>
__global__ __launch_bounds__(NT) void attention_kernel(
    const float* __restrict__ q_in, const float* __restrict__ k_in, const float* __restrict__ v_in,
    const float* __restrict__ rope_cs, const int* __restrict__ ctl, int n_heads, int n_kv_heads, int ctx, int layer,
    float scale, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, float* __restrict__ out,
    uint8_t* __restrict__ out_q8, const float* __restrict__ qn, const float* __restrict__ kn, float eps, int neox) {
  constexpr int hd = HD, half = HD / 2, g8 = HD / 8;
  static_assert(DS == 1 || (!PF && HD % (8 * DS) == 0 && (HD / DS == 32 || HD / DS == 16)),
                "dimension groups of 32, or 16 without the Q8_0 output");
  constexpr int DW = HD / DS;   // dimensions of this workgroup's value chains
  constexpr int g8w = DW / 8;   // their 16-byte pieces per position
  constexpr int C = DS > 1 ? 256 : (8192 / HD) & ~63 ? (8192 / HD) & ~63 : 64;  // positions per product chunk
  constexpr int CP = C + 4;
  static_assert(DW * CP <= kAttProd, "product chunk exceeds its LDS stage");
  constexpr int cw = (DW + 63) / 64;  // chain waves
  constexpr int nprod = NT - 64 * cw;
  constexpr int npc = C * g8w;  // 16-byte value pieces per chunk
  static_assert(npc <= 2 * nprod, "two pieces per producer thread");
  static_assert(npc % 64 == 0 && 3 * npc * 16 <= kAttRing, "whole-wave DMAs within the value ring");
  constexpr bool kTwoRounds = HD <= 64;  // second round of key rows held in registers
  extern __shared__ __align__(16) float sm[];
  const int bq = (int)blockIdx.x >> 3;
  const int h = DS > 1 ? 8 * (bq / DS) + ((int)blockIdx.x & 7) : (int)blockIdx.x, tid = threadIdx.x;
  const int dim0 = DS > 1 ? (bq % DS) * DW : 0;  // this workgroup's first value dimension
  const int tok = PF ? (int)(gridDim.y - 1 - blockIdx.y) : 0;  // prefill: the longest rows first
  const int pos = ctl[CTL_POS] + tok, n = pos + 1;
  const int self = PF ? -1 : pos;  // the position served from LDS rather than the cache
  if (PF) {
    q_in += (size_t)tok * n_heads * hd;
    out += (size_t)tok * n_heads * hd;
    if (out_q8) out_q8 += (size_t)tok * (n_heads * hd / 32) * kQ8_0Bytes;
  }
  const int gqa = n_heads / n_kv_heads, g = h / gqa;
  const bool writer = (h % gqa) == 0 && dim0 == 0;
  float* att = sm;
  float* prod = sm + ((ctx + 127) & ~127);
  float* qs = prod + 2 * kAttProd;
  float* kcur = qs + hd;
  float* vcur = kcur + hd;
  float* red = vcur + hd;
  // value pieces of three chunks, [3][npc] x 16 bytes, written by DMA
  uint4* vring = (uint4*)(red + 32);
  // KV cache, per layer and KV head, piece-major: [hd / 8][ctx][8 dims] f16, so
  // that lanes taking consecutive positions read consecutive 16-byte pieces
  const size_t base = ((size_t)layer * n_kv_heads + g) * hd * ctx;
  const size_t ctx8 = (size_t)ctx * 8;
  auto kvi = [&](int t, int d) { return base + (size_t)(d >> 3) * ctx8 + (size_t)t * 8 + (d & 7); };
  const int ptid = tid - 64 * cw;
  const bool producer = ptid >= 0;
  const int nchunks = (n + C - 1) / C;

  uint4 kr[g8], kr2[kTwoRounds ? g8 : 1];
  auto load_key = [&](int t, uint4* r) {
    if (t < n && t != self) {
      const uint4* src = (const uint4*)(kc + base + (size_t)t * 8);
#pragma unroll
      for (int j = 0; j < g8; j++) r[j] = src[(size_t)j * ctx];
    }
  };
  // Chunk c's value pieces go to ring slot c % 3 by DMA (global_load_lds_dwordx4,
  // no registers held): piece idx = position idx % C (consecutive lanes,
  // consecutive positions), dimensions 8 (idx / C) .. + 8. Producer wave p moves
  // pieces 64p + lane and nprod + 64p + lane, those below npc; positions past
  // the last are clamped to it (valid memory, never used) and the current
  // position's row is taken from LDS instead. Chunk c is requested two steps
  // before its products are formed, into the slot whose chunk was consumed
  // before the last barrier.
  const int pw = ptid >> 6;  // producer wave index (uniform)
  const int vdma = (64 * pw < npc ? 1 : 0) + (nprod + 64 * pw < npc ? 1 : 0);  // this wave's DMAs per chunk
  auto vload = [&](int c) {
    const int slot = c % 3;
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int wbase = 64 * pw + nprod * j;  // the wave's first piece
      if (wbase >= npc) break;
      const int idx = wbase + (tid & 63);
      const int tl = idx % C, i0 = dim0 + 8 * (idx / C);
      const int t = min(c * C + tl, n - 1);
      const uint32_t dst = __builtin_amdgcn_readfirstlane(
          (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint4*)(vring + (size_t)slot * npc + wbase));
      asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" : : "s"(dst), "v"(vc + kvi(t, i0)) : "memory");
    }
  };
  // this wave's DMAs for the older of its two outstanding chunks are done
  auto vwait = [&]() {
    asm volatile("" ::: "memory");
    if (vdma == 2) __builtin_amdgcn_s_waitcnt(2 | (7 << 4) | (15 << 8));
    else if (vdma == 1) __builtin_amdgcn_s_waitcnt(1 | (7 << 4) | (15 << 8));
    asm volatile("" ::: "memory");
  };
  // the first wait, with chunks 1 and 2 still outstanding
  auto vwait2 = [&]() {
    asm volatile("" ::: "memory");
    if (vdma == 2) __builtin_amdgcn_s_waitcnt(4 | (7 << 4) | (15 << 8));
    else if (vdma == 1) __builtin_amdgcn_s_waitcnt(2 | (7 << 4) | (15 << 8));
    asm volatile("" ::: "memory");
  };
  // With the q/k norm (Qwen3), the step's own q, k, v, the norm weights and
  // the rope table go to LDS before the cache rows are requested: the stores
  // wait for these loads only, and the norms and rope below run while the
  // cache rows arrive. (A load issued after the cache rows would wait for all
  // of them: vmcnt counts in issue order.) stg sits in the product stages,
  // free until the value loop.
  float* stg = prod + 2 * hd;  // qn | kn | (cos, sin) pairs | v, hd floats each
  const bool early = !PF && qn;
  if (early) {
    if (tid < hd) {
      qs[tid] = q_in[(size_t)h * hd + tid];
      kcur[tid] = k_in[(size_t)g * hd + tid];
      stg[tid] = qn[tid];
      stg[hd + tid] = kn[tid];
      stg[2 * hd + tid] = rope_cs[tid];
      stg[3 * hd + tid] = v_in[(size_t)g * hd + tid];
    }
    asm volatile("" ::: "memory");
  }
  load_key(tid, kr);
  if constexpr (kTwoRounds) load_key(tid + NT, kr2);
  if (producer) {
    vload(0);
    vload(1);
    vload(2);
  }
  if (PF) {
    for (int i = tid; i < hd; i += NT) qs[i] = q_in[(size_t)h * hd + i];
  } else if (qn || neox) {
    // Qwen3: the head's q and its KV head's k RMS-normalized (vec.rs:17-28,
    // infer.rs:533-541; squares in the product stage, free until the scores),
    // then rope with pair j = (j, j + hd/2) when neox; in LDS, in place.
    if (!early) {
      for (int i = tid; i < hd; i += NT) {
        qs[i] = q_in[(size_t)h * hd + i];
        kcur[i] = k_in[(size_t)g * hd + i];
      }
    }
    __syncthreads();
    if (qn) {
      float* sqq = prod;
      float* sqk = prod + hd;
      for (int i = tid; i < hd; i += NT) {
        sqq[i] = qs[i] * qs[i];
        sqk[i] = kcur[i] * kcur[i];
      }
      __syncthreads();
      if (tid == 0) red[0] = 1.0f / sqrtf(chain_sum(sqq, hd) / (float)hd + eps);
      if (tid == 64) red[1] = 1.0f / sqrtf(chain_sum(sqk, hd) / (float)hd + eps);
      __syncthreads();
      const float sq_ = red[0], sk_ = red[1];
      for (int i = tid; i < hd; i += NT) {  // qn set: the weights are staged
        qs[i] = qs[i] * (sq_ * stg[i]);
        kcur[i] = kcur[i] * (sk_ * stg[hd + i]);
      }
      __syncthreads();
    }
    for (int i = tid; i < half; i += NT) {
      const int ia = neox ? i : 2 * i, ib = neox ? i + half : 2 * i + 1;
      const float cs = early ? stg[2 * hd + 2 * i] : rope_cs[2 * i];
      const float sn = early ? stg[2 * hd + 2 * i + 1] : rope_cs[2 * i + 1];
      const float qa = qs[ia], qb = qs[ib];
      qs[ia] = qa * cs - qb * sn;
      qs[ib] = qa * sn + qb * cs;
      const float ka = kcur[ia], kb = kcur[ib];
      const uint32_t k0 = f32_to_f16_bits(ka * cs - kb * sn), k1 = f32_to_f16_bits(ka * sn + kb * cs);
      kcur[ia] = f16_bits_to_f32(k0);
      kcur[ib] = f16_bits_to_f32(k1);
      if (writer) {
        kc[kvi(pos, ia)] = (uint16_t)k0;
        kc[kvi(pos, ib)] = (uint16_t)k1;
      }
    }
    for (int i = tid; i < hd; i += NT) {
      const uint32_t vb = f32_to_f16_bits(early ? stg[3 * hd + i] : v_in[(size_t)g * hd + i]);
      vcur[i] = f16_bits_to_f32(vb);
      if (writer) vc[kvi(pos, i)] = (uint16_t)vb;
    }
  } else {
  for (int i = tid; i < half; i += NT) {
    const float cs = rope_cs[2 * i], sn = rope_cs[2 * i + 1];
    const float qa = q_in[(size_t)h * hd + 2 * i], qb = q_in[(size_t)h * hd + 2 * i + 1];
    qs[2 * i] = qa * cs - qb * sn;
    qs[2 * i + 1] = qa * sn + qb * cs;
    const float ka = k_in[(size_t)g * hd + 2 * i], kb = k_in[(size_t)g * hd + 2 * i + 1];
    const uint32_t k0 = f32_to_f16_bits(ka * cs - kb * sn), k1 = f32_to_f16_bits(ka * sn + kb * cs);
    kcur[2 * i] = f16_bits_to_f32(k0);
    kcur[2 * i + 1] = f16_bits_to_f32(k1);
    if (writer) {
      kc[kvi(pos, 2 * i)] = (uint16_t)k0;
      kc[kvi(pos, 2 * i + 1)] = (uint16_t)k1;
    }
  }
  for (int i = tid; i < hd; i += NT) {
    const uint32_t vb = f32_to_f16_bits(v_in[(size_t)g * hd + i]);
    vcur[i] = f16_bits_to_f32(vb);
    if (writer) vc[kvi(pos, i)] = (uint16_t)vb;
  }
  }
  __syncthreads();
  // Scores: thread tid takes positions tid, tid + NT, ...
  float mx = -INFINITY;
  auto score = [&](int t, const uint4* r) {
    float s = 0.0f;
    if (t == self) {
      for (int i = 0; i < hd; i++) s = s + kcur[i] * qs[i];
    } else {
#pragma unroll
      for (int p8 = 0; p8 < g8; p8++) {
        const uint32_t kw[4] = {r[p8].x, r[p8].y, r[p8].z, r[p8].w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
          s = s + f16_bits_to_f32(kw[j] & 0xffffu) * qs[8 * p8 + 2 * j];
          s = s + f16_bits_to_f32(kw[j] >> 16) * qs[8 * p8 + 2 * j + 1];
        }
      }
    }
    const float a = s * scale;
    att[t] = a;
    mx = fmaxf(mx, a);
  };
  if (tid < n) score(tid, kr);
  int t1 = tid + NT;
  if constexpr (kTwoRounds) {
    if (t1 < n) score(t1, kr2);
    t1 += NT;
  }
  for (; t1 < n; t1 += NT) {
    load_key(t1, kr);
    score(t1, kr);
  }
  // the max is order-independent, and the sign of a zero maximum cannot change
  // any exp(v - max)
  mx = wave_max(mx);
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  mx = red[0];
  for (int w = 1; w < NT / 64; w++) mx = fmaxf(mx, red[w]);
  // exps, then zeros up to a multiple of 128: adding +0 leaves the
  // (non-negative) sum unchanged, and the whole sum takes the DPP path
  const int n128 = (n + 127) & ~127;
  for (int t = tid; t < n128; t += NT) att[t] = t < n ? dev_expf(att[t] - mx) : 0.0f;
  __syncthreads();
  if (tid < 64) {
    const float tot = wave_chain_from(att, n128, 0.0f);
    if (tid == 0) red[16] = 1.0f / tot;
  }
  __syncthreads();
  const float inv = red[16];
  for (int t = tid; t < n; t += NT) att[t] = att[t] * inv;
  auto vprod = [&](int c) {
    float* pb = prod + (c & 1) * kAttProd;
    const uint4* r = vring + (size_t)(c % 3) * npc;
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int idx = ptid + nprod * j;
      const int tl = idx % C, i0 = 8 * (idx / C);
      const int t = c * C + tl;
      if (idx >= npc || t >= n) continue;
      const float a = att[t];
      float vv[8];
      if (t == self) {
#pragma unroll
        for (int q = 0; q < 8; q++) vv[q] = vcur[dim0 + i0 + q];
      } else {
        const uint4 rv = r[idx];
        const uint32_t vw[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
          vv[2 * q] = f16_bits_to_f32(vw[q] & 0xffffu);
          vv[2 * q + 1] = f16_bits_to_f32(vw[q] >> 16);
        }
      }
#pragma unroll
      for (int q = 0; q < 8; q++) pb[(i0 + q) * CP + tl] = a * vv[q];
    }
  };
  if (producer) vwait2();  // chunk 0
  __syncthreads();  // att[] normalized, chunk 0's values in the ring
  if (producer) {
    vprod(0);
    vwait();  // chunk 1 (chunk 2 outstanding)
  }
  __syncthreads();
  float o = 0.0f;
  // chunk cc: the chain lanes add it while the producers fill chunk cc + 1 (from
  // slot (cc + 1) % 3) and request chunk cc + 3 into the slot of chunk cc
  auto step = [&](int cc) {
    if (producer) {
      if (cc + 1 < nchunks) {
        vprod(cc + 1);
        vload(cc + 3);  // into the slot of chunk cc, consumed before the last barrier
        vwait();        // chunk cc + 2 (chunk cc + 3 outstanding), read after the barrier
      }
    } else if (tid < DW) {
      o = chain_from(prod + (cc & 1) * kAttProd + tid * CP, min(C, n - cc * C), o);
    }
    __syncthreads();
  };
  for (int c = 0; c < nchunks; c++) step(c);
  // requests past the last chunk land in unread slots; none may still be
  // writing to LDS when the workgroup ends
  if (producer) __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));
  if (tid < DW) {
    out[(size_t)h * hd + dim0 + tid] = o;
    if constexpr (DW >= 32) {  // a Q8_0 block is 32 dimensions of one workgroup
      if (out_q8) quant_q8_0_lane(o, tid & 31, out_q8 + (size_t)((h * hd + dim0 + tid) >> 5) * kQ8_0Bytes);
    }
  }
}

// Prefill attention for GH query heads of one KV head: workgroup (b, i) of NT
// threads serves token i of a chunk (position base + i) for heads b*GH ..
// b*GH+GH-1 (all of a KV group's heads, or a part of them), whose KV head is
// b*GH / (n_heads / n_kv_heads). Each key row is loaded once for the GH scores
// and each value piece once for the GH heads' products, so a launch reads the
// cached keys and values GH times less than one workgroup per head would. Per head, everything else is
// attention_kernel's, in the same order: dot_f16 in dimension order times the
// scale, the max, expf, the exp-sum in position order (one wave per head),
// a = e * inv, and out[d] += a_t * v_t[d] in position order (one chain lane
// per head and dimension, fed by producer waves in chunks of C positions).
// LDS: att[GH][ctx128] | prod[2][GH * HD * CP] | q[GH * HD] | red[64]
constexpr int kGrpProd = 9216;  // floats per product stage

template <int HD, int GH, int NT = kAttNT, int PROD = kGrpProd>
struct AttGroup {
  // positions per chunk: the product stage's, at most one value piece per producer thread
  static constexpr int C0 = (PROD / (GH * HD) - 4) & ~3;
  static constexpr int C1 = ((NT - GH * HD) / (HD / 8)) & ~3;
  static constexpr int C = C0 < C1 ? C0 : C1;
  static constexpr int CP = C + 4;
  static constexpr int stage = GH * HD * CP;
  static constexpr int cw = GH * HD / 64;  // chain waves
  static constexpr int nprod = NT - 64 * cw;
  static constexpr int npc = C * (HD / 8);  // 16-byte value pieces per chunk
  static size_t lds_bytes(int ctx) {
    return ((size_t)GH * ((ctx + 127) & ~127) + 2 * (size_t)stage + (size_t)GH * HD + 64) * 4;
  }
};

template <int HD, int GH, int NT = kAttNT, int PROD = kGrpProd>
__global__ __launch_bounds__(NT, NT <= 512 ? 4 : 1) void attention_group_kernel(
    const float* __restrict__ q_in, const int* __restrict__ ctl, int n_heads, int n_kv_heads, int ctx, int layer,
    float scale, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc, float* __restrict__ out,
    uint8_t* __restrict__ out_q8, uint8_t* __restrict__ out_q8k) {
  using A = AttGroup<HD, GH, NT, PROD>;
  constexpr int hd = HD, g8 = HD / 8, C = A::C, CP = A::CP, cw = A::cw, nprod = A::nprod, npc = A::npc;
  static_assert(C >= 4, "product chunk too small");
  static_assert(npc <= nprod, "one value piece per producer thread");
  static_assert(GH <= NT / 64 && NT / 64 <= 16, "one wave per head for the exp-sum, 16 waves at most");
  extern __shared__ __align__(16) float sm[];
  // the chunk's last tokens (the most positions) are dispatched first
  const int h0 = (int)blockIdx.x * GH, tok = (int)(gridDim.y - 1 - blockIdx.y), tid = threadIdx.x;
  const int g = h0 / (n_heads / n_kv_heads);  // the KV head
  const int pos = ctl[CTL_POS] + tok, n = pos + 1;
  const int n128 = (n + 127) & ~127;
  const int ctx128 = (ctx + 127) & ~127;
  float* att = sm;  // [GH][ctx128]
  float* prod = sm + (size_t)GH * ctx128;
  float* qs = prod + 2 * A::stage;  // [GH][hd]
  float* red = qs + GH * hd;         // [64]
  q_in += (size_t)tok * n_heads * hd + (size_t)h0 * hd;
  out += (size_t)tok * n_heads * hd + (size_t)h0 * hd;
  if (out_q8) out_q8 += ((size_t)tok * n_heads * hd + (size_t)h0 * hd) / 32 * kQ8_0Bytes;
  const size_t base = ((size_t)layer * n_kv_heads + g) * hd * ctx;
  const size_t ctx8 = (size_t)ctx * 8;
  for (int i = tid; i < GH * hd; i += NT) qs[i] = q_in[i];
  __syncthreads();
  // scores: thread tid takes positions tid, tid + NT, ...
  float mx[GH];
#pragma unroll
  for (int j = 0; j < GH; j++) mx[j] = -INFINITY;
  for (int t = tid; t < n; t += NT) {
    const uint4* src = (const uint4*)(kc + base + (size_t)t * 8);
    if constexpr (NT <= 512) {
      // the key row in halves of g8 / 2 pieces (registers for four waves per SIMD);
      // each head's dot runs on over the halves, in dimension order
      constexpr int hp = g8 / 2;
      float sc[GH];
#pragma unroll
      for (int j = 0; j < GH; j++) sc[j] = 0.0f;
#pragma unroll
      for (int hf = 0; hf < 2; hf++) {
        uint4 kr[hp];
#pragma unroll
        for (int p = 0; p < hp; p++) kr[p] = src[(size_t)(hp * hf + p) * ctx];
#pragma unroll
        for (int j = 0; j < GH; j++) {
          const float* q = qs + j * hd + 8 * hp * hf;
#pragma unroll
          for (int p = 0; p < hp; p++) {
            const uint32_t kw[4] = {kr[p].x, kr[p].y, kr[p].z, kr[p].w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
              sc[j] = sc[j] + f16_bits_to_f32(kw[e] & 0xffffu) * q[8 * p + 2 * e];
              sc[j] = sc[j] + f16_bits_to_f32(kw[e] >> 16) * q[8 * p + 2 * e + 1];
            }
          }
        }
      }
#pragma unroll
      for (int j = 0; j < GH; j++) att[(size_t)j * ctx128 + t] = sc[j] * scale;
    } else {
      uint4 kr[g8];
#pragma unroll
      for (int p8 = 0; p8 < g8; p8++) kr[p8] = src[(size_t)p8 * ctx];
#pragma unroll 1
      for (int j = 0; j < GH; j++) {  // one head at a time beside the packed key
        const float* q = qs + j * hd;
        float sc = 0.0f;
#pragma unroll
        for (int p8 = 0; p8 < g8; p8++) {
          const uint32_t kw[4] = {kr[p8].x, kr[p8].y, kr[p8].z, kr[p8].w};
#pragma unroll
          for (int e = 0; e < 4; e++) {
            sc = sc + f16_bits_to_f32(kw[e] & 0xffffu) * q[8 * p8 + 2 * e];
            sc = sc + f16_bits_to_f32(kw[e] >> 16) * q[8 * p8 + 2 * e + 1];
          }
        }
        const float a = sc * scale;
        att[(size_t)j * ctx128 + t] = a;
      }
    }
  }
  // each thread's maximum per head over the scores it wrote
  for (int t = tid; t < n; t += NT) {
#pragma unroll
    for (int j = 0; j < GH; j++) mx[j] = fmaxf(mx[j], att[(size_t)j * ctx128 + t]);
  }
#pragma unroll
  for (int j = 0; j < GH; j++) {
    const float m = wave_max(mx[j]);
    if ((tid & 63) == 0) red[j * 16 + (tid >> 6)] = m;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < GH; j++) {
    float m = red[j * 16];
    for (int w = 1; w < NT / 64; w++) m = fmaxf(m, red[j * 16 + w]);
    mx[j] = m;
  }
  __syncthreads();  // red is reused below
  for (int t = tid; t < n128; t += NT) {
#pragma unroll
    for (int j = 0; j < GH; j++)
      att[(size_t)j * ctx128 + t] = t < n ? dev_expf(att[(size_t)j * ctx128 + t] - mx[j]) : 0.0f;
  }
  __syncthreads();
  {
    const int w = tid >> 6;  // wave w < GH sums head w's exps in position order
    if (w < GH) {
      const float tot = wave_chain_from(att + (size_t)w * ctx128, n128, 0.0f);
      if ((tid & 63) == 0) red[w] = 1.0f / tot;
    }
  }
  __syncthreads();
  for (int t = tid; t < n; t += NT) {
#pragma unroll
    for (int j = 0; j < GH; j++) att[(size_t)j * ctx128 + t] = att[(size_t)j * ctx128 + t] * red[j];
  }
  // chunked axpy: producers form a_j(t) * v_t[d] for every head, chain lanes add
  const int ptid = tid - 64 * cw;
  const bool producer = ptid >= 0;
  const int nchunks = (n + C - 1) / C;
  auto vload = [&](int c, uint4& r) {
    const int tl = ptid % C, i0 = 8 * (ptid / C);
    const int t = c * C + tl;
    if (ptid < npc && t < n) r = *(const uint4*)(vc + base + (size_t)(i0 >> 3) * ctx8 + (size_t)t * 8);
  };
  auto vprod = [&](int c, const uint4& r) {
    const int tl = ptid % C, i0 = 8 * (ptid / C);
    const int t = c * C + tl;
    if (ptid >= npc || t >= n) return;
    float* pb = prod + (c & 1) * A::stage;
    float vv[8];
    const uint32_t vw[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int q = 0; q < 4; q++) {
      vv[2 * q] = f16_bits_to_f32(vw[q] & 0xffffu);
      vv[2 * q + 1] = f16_bits_to_f32(vw[q] >> 16);
    }
#pragma unroll
    for (int j = 0; j < GH; j++) {
      const float a = att[(size_t)j * ctx128 + t];
#pragma unroll
      for (int q = 0; q < 8; q++) pb[(j * hd + i0 + q) * CP + tl] = a * vv[q];
    }
  };
  uint4 s0 = make_uint4(0, 0, 0, 0), s1 = s0, s2 = s0;  // value pieces of chunks k with k % 3 == 0, 1, 2
  if (producer) {
    vload(0, s0);
    vload(1, s1);
    vload(2, s2);
  }
  __syncthreads();  // att[] normalized
  if (producer) {
    vprod(0, s0);
    vload(3, s0);
  }
  __syncthreads();
  float o = 0.0f;
  auto step = [&](int cc, uint4& slot) {
    if (producer) {
      if (cc + 1 < nchunks) {
        vprod(cc + 1, slot);
        vload(cc + 4, slot);
      }
    } else {
      o = chain_from(prod + (cc & 1) * A::stage + tid * CP, min(C, n - cc * C), o);
    }
    __syncthreads();
  };
  for (int c = 0; c < nchunks; c += 3) {
    step(c, s1);
    if (c + 1 < nchunks) step(c + 1, s2);
    if (c + 2 < nchunks) step(c + 2, s0);
  }
  if (tid < GH * hd) {
    out[tid] = o;
    if (out_q8) quant_q8_0_lane(o, tid & 31, out_q8 + (size_t)(tid >> 5) * kQ8_0Bytes);
  }
  if constexpr (GH * HD == 256) {
    // the output's Q8_K block (kquant.rs:157-187) for a K-quant o projection:
    // the workgroup's heads are one block; the product stages are free
    if (out_q8k) {
      float* ob = prod;
      if (tid < 256) ob[tid] = o;
      __syncthreads();
      if (tid < 64) {  // both half-waves form the block; the first stores it
        const int r = tid & 31;
        const float4 v0 = ((const float4*)ob)[2 * r], v1 = ((const float4*)ob)[2 * r + 1];
        const float v8[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        uint32_t lo, hi, d_bits;
        int ps;
        q8k_half_lanes(v8, r, &lo, &hi, &ps, &d_bits);
        if (tid < 32)
          q8k_half_store(out_q8k + ((size_t)tok * n_heads * hd + (size_t)h0 * hd) / 256 * kQ8KBytes, r, lo, hi, ps,
                         d_bits);
      }
    }
  }
}

// vec.rs:45-52: gate = gate / (1 + expf(-gate)) * up; with xq != null also its
// Q8_0 blocks (n is a multiple of 256).
__global__ __launch_bounds__(256) void swiglu_kernel(float* __restrict__ gate, const float* __restrict__ up, int n,
                                                     uint8_t* __restrict__ xq) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float g = gate[i];
  const float silu = g / (1.0f + dev_expf(-g));
  const float v = silu * up[i];
  gate[i] = v;
  if (xq) quant_q8_0_lane(v, threadIdx.x & 31, xq + (size_t)(i >> 5) * kQ8_0Bytes);
}

// scale_inplace (vec.rs:61-65): x[i] *= s
__global__ void scale_kernel(float* __restrict__ x, int n, float s) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) x[i] = x[i] * s;
}

constexpr int kArgNT = 1024;

// vec.rs:80-90 (first index of the largest value; NaN never wins), then the
// step's bookkeeping: next token, output slot, position + 1 (without ctl, only
// out_tokens[0]).
__global__ __launch_bounds__(kArgNT) void argmax_kernel(const float* __restrict__ x, int n, int* __restrict__ ctl,
                                                        uint32_t* __restrict__ out_tokens, int max_out) {
  __shared__ float sv[kArgNT / 64];
  __shared__ int si[kArgNT / 64];
  const int tid = threadIdx.x;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  // each thread scans its indices in increasing order (strict >), 4 at a time
  const int n4 = n >> 2;
  const float4* x4 = (const float4*)x;
  int j = tid;
  for (; j + 3 * kArgNT < n4; j += 4 * kArgNT) {
    float4 v[4];
#pragma unroll
    for (int u = 0; u < 4; u++) v[u] = x4[j + u * kArgNT];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int b = 4 * (j + u * kArgNT);
      if (v[u].x > bv) { bv = v[u].x; bi = b; }
      if (v[u].y > bv) { bv = v[u].y; bi = b + 1; }
      if (v[u].z > bv) { bv = v[u].z; bi = b + 2; }
      if (v[u].w > bv) { bv = v[u].w; bi = b + 3; }
    }
  }
  for (; j < n4; j += kArgNT) {
    const float4 v = x4[j];
    const int b = 4 * j;
    if (v.x > bv) { bv = v.x; bi = b; }
    if (v.y > bv) { bv = v.y; bi = b + 1; }
    if (v.z > bv) { bv = v.z; bi = b + 2; }
    if (v.w > bv) { bv = v.w; bi = b + 3; }
  }
  for (int i = 4 * n4 + tid; i < n; i += kArgNT)
    if (x[i] > bv) {
      bv = x[i];
      bi = i;
    }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float ov = __shfl_xor(bv, m);
    const int oi = __shfl_xor(bi, m);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if ((tid & 63) == 0) {
    sv[tid >> 6] = bv;
    si[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int wv = 1; wv < kArgNT / 64; wv++)
      if (sv[wv] > bv || (sv[wv] == bv && si[wv] < bi)) {
        bv = sv[wv];
        bi = si[wv];
      }
    const int best = bi == 0x7fffffff ? 0 : bi;
    if (!ctl) {  // a lone draw (nrq_dev_sample): the id only
      out_tokens[0] = (uint32_t)best;
      return;
    }
    ctl[CTL_TOKEN] = best;
    const int step = ctl[CTL_STEP];
    if (out_tokens && step < max_out) out_tokens[step] = (uint32_t)best;
    ctl[CTL_STEP] = step + 1;
    ctl[CTL_POS] = ctl[CTL_POS] + 1;
  }
}

constexpr int kTopK = 64;                      // sample.rs:12
constexpr int kSelPartWaves = 4;               // waves per workgroup of the first kernel
constexpr int kSelPer = 8;                     // logits per lane in the first kernel
constexpr int kSelSlice = kSelPartWaves * 64 * kSelPer;  // logits per workgroup of the first kernel
constexpr int kSelWaves = 16;                  // waves of the second kernel
constexpr int kSelPart = 2 * kTopK;            // words per partial list (64 packed candidates)

// Sampler::next_f32 (sample.rs:23-30)
__device__ inline float sampler_next_f32(unsigned long long* rng) {
  unsigned long long x = *rng;
  x ^= x << 13;
  x ^= x >> 7;
  x ^= x << 17;
  *rng = x;
  return (float)(x >> 40) / (float)(1u << 24);
}

// Order-preserving key of a logit: larger logit, larger key; -0 and +0 share a
// key (they compare equal); NaN and -inf get 0, "no candidate" (the heap's
// strict > never admits them, sample.rs:41-49).
__device__ inline uint32_t logit_key(float v) {
  if (!(v > -INFINITY)) return 0u;
  uint32_t u = __float_as_uint(v);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// A candidate packed as key << 32 | ~id: a larger word is a larger logit, or an
// equal one with a lower id; 0 is an empty slot (below every candidate).
__device__ inline unsigned long long cand_pack(uint32_t key, uint32_t id) {
  return key ? ((unsigned long long)key << 32) | (uint32_t)~id : 0ull;
}

__device__ inline void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ inline int lanes_below(unsigned long long m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// The exact 64 largest of a wave's 64*E (key, id) pairs (ids distinct among
// present keys; key 0 = absent), returned sorted: lane l holds the l-th
// largest packed candidate. A bisection over the key bits, counting with
// ballots, finds the 64th largest key T; every key above T is taken, and of
// those equal to T the lowest ids, by a second bisection over the id bits when
// there are more than are needed. The set is packed into sc (this wave's 64
// words of LDS), then each candidate moves to its rank. Fewer than 64 present
// keys leave empty slots at the end.
template <int E>
__device__ inline unsigned long long wave_sorted64(const uint32_t (&k)[E], const uint32_t (&id)[E],
                                                   unsigned long long* sc) {
  const int lane = threadIdx.x & 63;
  uint32_t T = 0;
  for (int b = 31; b >= 0; b--) {
    const uint32_t c = T | (1u << b);
    int cnt = 0;
#pragma unroll
    for (int e = 0; e < E; e++) cnt += __popcll(__ballot(k[e] >= c));
    if (cnt >= kTopK) T = c;
  }
  uint32_t J = 0xffffffffu;  // of the keys equal to T, the ids up to J
  if (T != 0) {              // T is at most the key of +inf, so T + 1 does not wrap
    int gt = 0, eq = 0;
#pragma unroll
    for (int e = 0; e < E; e++) {
      gt += __popcll(__ballot(k[e] > T));
      eq += __popcll(__ballot(k[e] == T));
    }
    const int need = kTopK - gt;
    if (eq > need) {
      J = 0;
      for (int b = 31; b >= 0; b--) {
        const uint32_t c = J | (1u << b);
        int cnt = 0;
#pragma unroll
        for (int e = 0; e < E; e++) cnt += __popcll(__ballot(k[e] == T && id[e] < c));
        if (cnt < need) J = c;
      }
    }
  }
  int base = 0;
#pragma unroll
  for (int e = 0; e < E; e++) {
    const bool sel = T == 0 ? k[e] != 0 : (k[e] > T || (k[e] == T && id[e] <= J));
    const unsigned long long m = __ballot(sel);
    if (sel) sc[base + lanes_below(m)] = cand_pack(k[e], id[e]);
    base += __popcll(m);
  }
  if (lane >= base) sc[lane] = 0ull;
  wave_sync();
  const unsigned long long c = sc[lane];
  int r = 0;
  const ulonglong2* s2 = (const ulonglong2*)sc;
#pragma unroll
  for (int j = 0; j < kTopK / 2; j++) {
    const ulonglong2 t = s2[j];
    r += (t.x > c ? 1 : 0) + (t.y > c ? 1 : 0);
  }
  if (c == 0ull) r = lane;  // empty slots already follow the present ones
  wave_sync();
  sc[r] = c;
  wave_sync();
  return sc[lane];
}

// The value of lane l ^ J, by VALU cross-lane moves: DPP within a 16-lane row
// (quad_perm for J = 1, 2; row_shl / row_shr by 4 for J = 4; row_ror:8 for
// J = 8), v_permlane16_swap / v_permlane32_swap across rows (J = 16, 32).
template <int J>
__device__ inline uint32_t lane_xor(uint32_t v) {
  const int lane = threadIdx.x & 63;
  if constexpr (J == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return lane < 32 ? r[1] : r[0];
  } else if constexpr (J == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (lane & 16) ? r[0] : r[1];
  } else if constexpr (J == 8) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x128, 0xf, 0xf, false);  // row_ror:8
  } else if constexpr (J == 4) {
    const uint32_t up = (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x104, 0xf, 0xf, false);  // row_shl:4
    const uint32_t dn = (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x114, 0xf, 0xf, false);  // row_shr:4
    return (lane & 4) ? dn : up;
  } else if constexpr (J == 2) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x4e, 0xf, 0xf, false);  // quad_perm [2,3,0,1]
  } else {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0xb1, 0xf, 0xf, false);  // quad_perm [1,0,3,2]
  }
}

template <int J>
__device__ inline unsigned long long bitonic_stage(unsigned long long c) {
  const uint32_t lo = lane_xor<J>((uint32_t)c), hi = lane_xor<J>((uint32_t)(c >> 32));
  const unsigned long long o = ((unsigned long long)hi << 32) | lo;
  return ((threadIdx.x & J) == 0) ? (c > o ? c : o) : (c < o ? c : o);
}

// The 64 largest of two sorted lists, sorted: lane l holds a's l-th largest
// and b's (63-l)-th (b read in reverse lane order). max(a_l, b_{63-l}) is
// bitonic and holds the 64 largest of the union; a bitonic merge orders it.
__device__ inline unsigned long long merge64(unsigned long long a, unsigned long long b_rev) {
  unsigned long long c = a > b_rev ? a : b_rev;
  c = bitonic_stage<32>(c);
  c = bitonic_stage<16>(c);
  c = bitonic_stage<8>(c);
  c = bitonic_stage<4>(c);
  c = bitonic_stage<2>(c);
  return bitonic_stage<1>(c);
}

// First half of Sampler::sample (sample.rs:38-61) for temperature > 0: each
// workgroup takes kSelSlice logits, each wave selects the 64 largest of its
// 512, the four sorted lists merge in a tree, and the workgroup writes its
// sorted 64 as one partial list.
__global__ __launch_bounds__(kSelPartWaves * 64) void top64_part_kernel(const float* __restrict__ x, int n,
                                                                        unsigned long long* __restrict__ part) {
  __shared__ unsigned long long sc[kSelPartWaves][kTopK];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int base = blockIdx.x * kSelSlice + w * 64 * kSelPer;
  uint32_t k[kSelPer], id[kSelPer];
  float v[kSelPer];
#pragma unroll
  for (int e = 0; e < kSelPer; e++) v[e] = x[min(base + e * 64 + lane, n - 1)];  // all loads in flight
#pragma unroll
  for (int e = 0; e < kSelPer; e++) {
    const int i = base + e * 64 + lane;
    id[e] = (uint32_t)i;
    k[e] = i < n ? logit_key(v[e]) : 0u;
  }
  unsigned long long c = wave_sorted64<kSelPer>(k, id, sc[w]);
  __syncthreads();
#pragma unroll
  for (int h = kSelPartWaves / 2; h >= 1; h >>= 1) {
    if (w < h) {
      c = merge64(c, sc[w + h][63 - lane]);
      sc[w][lane] = c;
    }
    __syncthreads();
  }
  if (w == 0) part[(size_t)blockIdx.x * kTopK + lane] = c;
}

// Second half of Sampler::sample (sample.rs:38-96), one workgroup over the
// nparts sorted partial lists:
//  1. The 64 largest of the lists: wave w merges lists w, w + 16, ..., then the
//     16 waves' lists merge in a tree. The logits of the reference's heap are
//     thus found exactly, in descending order; exact ties are ordered by token
//     id, where the reference's unstable sort leaves their order open (matched
//     whenever the drawn logit is not tied). Fewer than 64 valid logits leave
//     (-inf, 0) slots, as the heap's initial entries do.
//  2. In the reference's order: p_k = expf((v_k - max) / T) (one per lane),
//     the running sums s_k = s_{k-1} + p_k (in order), the nucleus n = first k
//     with s_k >= top_p * s_63, r = next_f32() * s_{n-1}, and the first k < n
//     with r <= s_k (else the last of the nucleus).
// With ctl, the step's bookkeeping of argmax_kernel; else the id goes to *token.
__global__ __launch_bounds__(kSelWaves * 64) void top64_sample_kernel(
    const unsigned long long* __restrict__ part, int nparts, const float* __restrict__ x, float temperature,
    float top_p, unsigned long long* __restrict__ rng, int* __restrict__ ctl, uint32_t* __restrict__ out_tokens,
    int max_out, uint32_t* __restrict__ token) {
  __shared__ unsigned long long sc[kSelWaves][kTopK];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  // list q (lane order l, or reversed), or an empty one past the last
  // (clamped loads, four in flight)
  auto list = [&](int q, int l) {
    const unsigned long long c = part[(size_t)min(q, nparts - 1) * kTopK + l];
    return q < nparts ? c : 0ull;
  };
  unsigned long long c = list(w, lane);
  for (int q = w + kSelWaves; q < nparts; q += 3 * kSelWaves) {
    const int rl = 63 - lane;
    const unsigned long long l1 = list(q, rl), l2 = list(q + kSelWaves, rl), l3 = list(q + 2 * kSelWaves, rl);
    c = merge64(c, l1);
    if (q + kSelWaves < nparts) c = merge64(c, l2);
    if (q + 2 * kSelWaves < nparts) c = merge64(c, l3);
  }
  sc[w][lane] = c;
  __syncthreads();
#pragma unroll
  for (int h = kSelWaves / 2; h >= 1; h >>= 1) {
    if (w < h) {
      c = merge64(c, sc[w + h][63 - lane]);
      sc[w][lane] = c;
    }
    __syncthreads();
  }
  if (w != 0) return;
  const uint32_t cid = c ? ~(uint32_t)c : 0u;
  const float v = c ? x[cid] : -INFINITY;
  const float mx = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float p = dev_expf((v - mx) / temperature);
  // s_q = s_{q-1} + p_q in order, every lane running the chain; lane q keeps s_q
  float s = 0.0f, mine = 0.0f;
#pragma unroll
  for (int q = 0; q < kTopK; q++) {
    s = s + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), q));
    mine = lane == q ? s : mine;
  }
  const float cut = top_p * s;
  const unsigned long long inn = __ballot(mine >= cut);
  const int nn = inn ? __builtin_ctzll(inn) + 1 : kTopK;
  const float cum = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), nn - 1));
  unsigned long long st = *rng;
  const float rr = sampler_next_f32(&st) * cum;
  const unsigned long long hit = __ballot(lane < nn && rr <= mine);
  const uint32_t pick = (uint32_t)__builtin_amdgcn_readlane((int)cid, hit ? __builtin_ctzll(hit) : nn - 1);
  if (lane == 0) {
    *rng = st;
    if (ctl) {
      ctl[CTL_TOKEN] = (int)pick;
      const int step = ctl[CTL_STEP];
      if (out_tokens && step < max_out) out_tokens[step] = pick;
      ctl[CTL_STEP] = step + 1;
      ctl[CTL_POS] = ctl[CTL_POS] + 1;
    } else {
      *token = pick;
    }
  }
}

__global__ void mathf_kernel(int fn, const float* __restrict__ x, float* __restrict__ y, long long n) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  if (fn == 0) {
    y[i] = dev_expf(x[i]);
  } else {
    float s, c;
    dev_sincosf(x[i], &s, &c);
    y[i] = fn == 1 ? s : c;
  }
}

}  // namespace
}  // namespace nrq

// ---- the sampler's fixed scratch (nrq_dev_sample_noalloc) ------------------------------
// The partial top-64 lists of top64_part_kernel for callers that cannot
// allocate: one array per device, 128 KiB, held until the process ends. Every
// call on a device shares it and leaves its lists there; top64_sample_kernel
// reads only the lists the same call's top64_part_kernel wrote, so nothing
// needs clearing. In host code `scratch` is a host-side stand-in: only the
// per-device address from hipGetSymbolAddress is passed to kernels.
namespace nrq {
constexpr int kSampleMaxLogits = 1 << 19;
constexpr int kSampleScratchLists = kSampleMaxLogits / kSelSlice;
}  // namespace nrq
static __device__ __align__(256) unsigned long long scratch[nrq::kSampleScratchLists * nrq::kTopK];

namespace {
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kScratchDevices];  // address of `scratch` on each device, once looked up

// The address of this device's `scratch` (the device must be current).
int scratch_on_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kScratchDevices) {
    nrq::set_last_error("sampler scratch: no usable current device");
    return NRQ_ERR_DEVICE;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      nrq::set_last_error((std::string("sampler scratch: hipGetSymbolAddress: ") + hipGetErrorString(e)).c_str());
      return NRQ_ERR_DEVICE;
    }
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return NRQ_OK;
}
}  // namespace

namespace nrq {
int sample_scratch_setup() {
  void* p = nullptr;
  return scratch_on_current_device(&p);
}
}  // namespace nrq

// ---- host side -----------------------------------------------------------------------

namespace {

int mfail(int code, const char* msg) {
  nrq::set_last_error(msg);
  return code;
}

#define MHIP(expr)                                                                  \
  do {                                                                              \
    hipError_t e_ = (expr);                                                         \
    if (e_ != hipSuccess) {                                                         \
      nrq::set_last_error((std::string(#expr) + ": " + hipGetErrorString(e_)).c_str()); \
      return NRQ_ERR_DEVICE;                                                        \
    }                                                                               \
  } while (0)

struct Mat {
  const void* w = nullptr;
  int dt = 0;
};

struct Layer {
  Mat m[7];  // q, k, v, o, gate, up, down
  const float* attn_norm = nullptr;
  const float* ffn_norm = nullptr;
  const float* q_norm = nullptr;  // Qwen3 per-head RMSNorm weights, head_dim each
  const float* k_norm = nullptr;
};

size_t act_bytes(int dt, size_t n) { return dt == NRQ_Q8_0 ? n / 32 * 34 : n / 256 * 292; }
int qk_of(int dt) { return dt == NRQ_Q8_0 ? 32 : 256; }

}  // namespace

struct nrq_model {
  nrq_model_config cfg{};
  // HIP events recorded after each stage of a timed eager step (nrq_model_step_profile)
  std::vector<hipEvent_t> tev;
  std::vector<int> tstage;
  bool timing = false;
  int kv_dim = 0, att_dim = 0, maxd = 0;
  hipStream_t stream = nullptr;
  Mat embed, output;
  const float* out_norm = nullptr;
  std::vector<Layer> L;
  float* freqs = nullptr;
  float* rope_cs = nullptr;  // (cos, sin) of the step's position, head_dim floats
  uint16_t *kc = nullptr, *vc = nullptr;
  float *x = nullptr, *x2 = nullptr, *xb = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr;
  float *gate = nullptr, *up = nullptr, *xb2 = nullptr, *logits = nullptr;
  uint8_t *xq = nullptr, *xq2 = nullptr;
  int* ctl = nullptr;
  uint32_t* out_tokens = nullptr;
  int max_out = 0;
  hipGraphExec_t exec = nullptr;
  hipGraph_t graph = nullptr;
  int host_pos = 0;
  size_t att_lds = 0;
  void* owned = nullptr;  // the data section a loader uploaded; freed with the model
  // prefill scratch, [kMaxBatch][*], made at the first prefill
  float *bx = nullptr, *bxb = nullptr, *bxn = nullptr, *bq = nullptr, *bk = nullptr, *bv = nullptr;
  float *battn = nullptr, *bgate = nullptr, *bup = nullptr, *brope = nullptr;
  uint8_t *bxq = nullptr, *bxq2 = nullptr;
  int* btok = nullptr;
  // Sampler (sample.rs:5-21): temperature <= 0 is greedy
  float samp_t = 0.0f, samp_p = 1.0f;
  unsigned long long* rng = nullptr;  // device word, seed | 1
  unsigned long long* samp_part = nullptr;  // the sampler's partial top-64 lists
  // the recipe (infer.rs:447-461): Neox rope pairs, muP scalars
  int rope_neox = 0;
  float embed_scale = 1.0f, att_scale = 0.0f, res_scale = 1.0f, logit_recip = 1.0f;
};

namespace nrq {
void model_adopt_buffer(nrq_model* m, void* dev) { m->owned = dev; }
}  // namespace nrq

namespace {

// Quantize `src` (n floats) into the activation format of weight dtype dt.
int quantize_for(nrq_model* m, int dt, const float* src, int n, uint8_t* dst) {
  nrq::QuantLaunch Q{src, dst, (long long)n, m->stream};
  const int rc = dt == NRQ_Q8_0 ? nrq::launch_quantize_q8_0(Q) : nrq::launch_quantize_q8k(Q);
  return rc ? mfail(NRQ_ERR_DEVICE, "model: activation quantize launch failed") : NRQ_OK;
}

int matvec(nrq_model* m, const Mat& w, const uint8_t* xq, float* y, int rows, int cols) {
  nrq::MatvecLaunch L;
  L.w = w.w;
  L.x = xq;
  L.y = y;
  L.rows = rows;
  L.bpr = cols / qk_of(w.dt);
  L.tile_rows = 0;
  L.stream = m->stream;
  const int rc = nrq::launch_matvec(w.dt, nrq::kOrderScalar, L);
  return rc ? mfail(rc == nrq::NRQ_LAUNCH_TOO_WIDE ? NRQ_ERR_UNSUPPORTED : NRQ_ERR_DEVICE, "model: matvec launch failed")
            : NRQ_OK;
}

// Normalize the residual xr (after xr += add, in place), quantize for dtype dt.
int norm_quant(nrq_model* m, float* xr, const float* add, const float* w, int dt) {
  const auto& c = m->cfg;
  hipLaunchKernelGGL(nrq::norm_kernel, dim3(1), dim3(nrq::kNormNT), 0, m->stream, xr, add, w, c.dim, c.norm_eps,
                     m->res_scale, m->xb, dt == NRQ_Q8_0 ? m->xq : nullptr, dt != NRQ_Q8_0 ? m->xq : nullptr);
  if (hipGetLastError() != hipSuccess) return mfail(NRQ_ERR_DEVICE, "model: norm launch failed");
  return NRQ_OK;
}

// Matvecs sharing one input vector: the activation is quantized once per
// format (infer.rs:232-261); `xb` holds the f32 input, m->xq its blocks for
// the first matrix's format.
int matvec_group(nrq_model* m, const Mat* const* ws, float* const* ys, const int* rows, int n, int cols) {
  const int first = ws[0]->dt == NRQ_Q8_0 ? 0 : 1;
  bool other_ready = false;
  for (int i = 0; i < n;) {
    const int fmt = ws[i]->dt == NRQ_Q8_0 ? 0 : 1;
    const uint8_t* xq = m->xq;
    if (fmt != first) {
      if (!other_ready) {
        int rc = quantize_for(m, ws[i]->dt, m->xb, cols, m->xq2);
        if (rc) return rc;
        other_ready = true;
      }
      xq = m->xq2;
    }
    // a run of matrices of one dtype goes out as one launch (q|k, gate|up)
    int j = i + 1;
    while (j < n && ws[j]->dt == ws[i]->dt) j++;
    if (j - i > 1) {
      const void* w[3];
      float* y[3];
      int r[3];
      for (int t = i; t < j; t++) {
        w[t - i] = ws[t]->w;
        y[t - i] = ys[t];
        r[t - i] = rows[t];
      }
      const int g = nrq::launch_wstream_group(ws[i]->dt, w, y, r, j - i, xq, cols / qk_of(ws[i]->dt), m->stream);
      if (g == nrq::NRQ_LAUNCH_TOO_WIDE) {  // one launch per matrix, as the ungrouped step runs them
        for (int t = i; t < j; t++) {
          int rc = matvec(m, *ws[t], xq, ys[t], rows[t], cols);
          if (rc) return rc;
        }
      } else if (g) {
        return mfail(NRQ_ERR_DEVICE, "model: grouped matvec launch failed");
      }
    } else {
      int rc = matvec(m, *ws[i], xq, ys[i], rows[i], cols);
      if (rc) return rc;
    }
    i = j;
  }
  return NRQ_OK;
}

// Norm + Q8_0 matvecs of one input in a single launch when every matrix is
// Q8_0: the residual is read from *xr and, with a pending add, the sum goes to
// *xo and the two buffers swap. Returns 1 when the shapes do not allow it.
int fused_norm_group(nrq_model* m, float** xr, float** xo, const float* add, const float* normw,
                     const Mat* const* ws, float* const* ys, const int* rows, int n, uint8_t* swiglu_q8 = nullptr) {
  // Q8_0 groups, or K-quant groups (Q4_K / Q6_K, no swiglu epilogue): the
  // leading run of one dtype takes the fused launch, which for K-quants also
  // stores the Q8_K activation that the rest of the group reads
  const int dt = ws[0]->dt;
  const bool kq = dt != NRQ_Q8_0;
  for (int i = 0; i < n; i++)
    if ((ws[i]->dt == NRQ_Q8_0) == kq) return 1;
  if (kq && swiglu_q8) return 1;
  int j = 1;
  while (j < n && ws[j]->dt == dt) j++;
  nrq::NormMatvecLaunch L{};
  L.x = *xr;
  L.add = add;
  L.x_out = add ? *xo : nullptr;
  L.norm_w = normw;
  L.n = m->cfg.dim;
  L.eps = m->cfg.norm_eps;
  L.rscale = m->res_scale;
  L.nmat = j;
  for (int i = 0; i < j; i++) {
    L.w[i] = ws[i]->w;
    L.y[i] = ys[i];
    L.rows[i] = rows[i];
  }
  L.swiglu_q8 = swiglu_q8;
  L.xq_out = kq ? m->xq : nullptr;
  L.stream = m->stream;
  const int rc = nrq::launch_norm_matvec(dt, L);
  if (rc == nrq::NRQ_LAUNCH_TOO_WIDE) return 1;
  if (rc) return mfail(NRQ_ERR_DEVICE, "model: norm + matvec launch failed");
  if (add) std::swap(*xr, *xo);
  if (j < n) return matvec_group(m, ws + j, ys + j, rows + j, n - j, m->cfg.dim);
  return NRQ_OK;
}

int set_ctl(nrq_model* m, int i0, int v0, int i1 = -1, int v1 = 0) {
  hipLaunchKernelGGL(nrq::ctl_set_kernel, dim3(1), dim3(64), 0, m->stream, m->ctl, i0, v0, i1, v1);
  return hipGetLastError() == hipSuccess ? NRQ_OK : mfail(NRQ_ERR_DEVICE, "model: control word launch failed");
}

// muP logit scale (infer.rs:589-591): logits *= 1/logit_scale when it is not 1
int scale_logits(nrq_model* m) {
  if (m->logit_recip == 1.0f) return NRQ_OK;
  const int n = m->cfg.vocab;
  hipLaunchKernelGGL(nrq::scale_kernel, dim3((n + 255) / 256), dim3(256), 0, m->stream, m->logits, n, m->logit_recip);
  return hipGetLastError() == hipSuccess ? NRQ_OK : mfail(NRQ_ERR_DEVICE, "model: logit scale launch failed");
}

// Holds the stream for `ticks` of the 100 MHz real-time clock (one wave, a
// bounded wait), so that the host enqueues a whole timed step before the GPU
// reaches its first kernel.
__global__ void hold_kernel(long long ticks) {
  const long long t0 = wall_clock64();
  while (wall_clock64() - t0 < ticks) __builtin_amdgcn_s_sleep(8);
}

// Stages of a decode step, as nrq_model_step_profile reports them.
enum { kStEmbed, kStQkv, kStAttention, kStO, kStGateUp, kStDown, kStFinalNorm, kStHead, kStPick, kStCount };

// In a timed step: an event after the stage just enqueued.
static void step_mark(nrq_model* m, int stage) {
  if (!m->timing) return;
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return;
  hipEventRecord(e, m->stream);
  m->tev.push_back(e);
  m->tstage.push_back(stage);
}

// One decode step, enqueued on m->stream (infer.rs:510-595 + argmax).
int att_dim_split(const nrq_model_config& c);

int enqueue_step(nrq_model* m) {
  const auto& c = m->cfg;
  const int d = c.dim, kvd = m->kv_dim, att = m->att_dim, ffn = c.ffn_dim;
  hipLaunchKernelGGL(nrq::embed_kernel, dim3((d + 255) / 256), dim3(256), 0, m->stream,
                     (const uint8_t*)m->embed.w, m->embed.dt, m->ctl, d, m->x, m->freqs, c.head_dim / 2, m->rope_cs,
                     m->embed_scale);
  if (hipGetLastError() != hipSuccess) return mfail(NRQ_ERR_DEVICE, "model: embed launch failed");
  step_mark(m, kStEmbed);
  const float scale = m->att_scale;
  const float* pending = nullptr;  // residual not yet added into *xr
  float* xr = m->x;                // the residual stream
  float* xo = m->x2;               // where a fused norm writes xr + pending
  int rc;
  for (int l = 0; l < c.n_layers; l++) {
    const Layer& Ly = m->L[l];
    bool swiglu_done = false;
    {
      const Mat* ws[3] = {&Ly.m[0], &Ly.m[1], &Ly.m[2]};
      float* ys[3] = {m->q, m->k, m->v};
      const int rows[3] = {att, kvd, kvd};
      rc = fused_norm_group(m, &xr, &xo, pending, Ly.attn_norm, ws, ys, rows, 3);
      if (rc == 1) {
        if ((rc = norm_quant(m, xr, pending, Ly.attn_norm, Ly.m[0].dt))) return rc;
        rc = matvec_group(m, ws, ys, rows, 3, d);
      }
      if (rc) return rc;
      step_mark(m, kStQkv);
    }
    {
      const bool q8 = Ly.m[3].dt == NRQ_Q8_0;
      // a K-quant o projection quantizes the output itself: 128-wide heads
      // then split eight ways (16 value dimensions per workgroup)
      const int ds = att_dim_split(c) * (c.head_dim == 128 && !q8 && att_dim_split(c) == 4 ? 2 : 1);
      auto* kern = c.head_dim == 32   ? nrq::attention_kernel<32>
                   : c.head_dim == 64 ? (ds == 2 ? nrq::attention_kernel<64, false, nrq::kAttNT, 2>
                                                 : nrq::attention_kernel<64>)
                   : c.head_dim == 96 ? nrq::attention_kernel<96>
                                      : (ds == 8   ? nrq::attention_kernel<128, false, 768, 8>
                                         : ds == 4 ? nrq::attention_kernel<128, false, 768, 4>
                                                   : nrq::attention_kernel<128>);
      hipLaunchKernelGGL(kern, dim3(c.n_heads * ds), dim3(nrq::att_threads(c.head_dim)), m->att_lds, m->stream, m->q, m->k, m->v,
                         m->rope_cs, m->ctl, c.n_heads, c.n_kv_heads, c.ctx, l, scale, m->kc, m->vc, m->attn,
                         q8 ? m->xq : nullptr, Ly.q_norm, Ly.k_norm, c.norm_eps, m->rope_neox);
      if (hipGetLastError() != hipSuccess) return mfail(NRQ_ERR_DEVICE, "model: attention launch failed");
      step_mark(m, kStAttention);
      // a K-quant o projection quantizes the attention output in its prologue
      const int fq = q8 ? nrq::NRQ_LAUNCH_TOO_WIDE
                        : nrq::launch_quant_matvec(Ly.m[3].dt, m->attn, att, Ly.m[3].w, m->xb2, d, m->stream);
      if (fq && fq != nrq::NRQ_LAUNCH_TOO_WIDE) return mfail(NRQ_ERR_DEVICE, "model: quantize + matvec launch failed");
      if (fq) {
        if (!q8 && (rc = quantize_for(m, Ly.m[3].dt, m->attn, att, m->xq))) return rc;
        if ((rc = matvec(m, Ly.m[3], m->xq, m->xb2, d, att))) return rc;
      }
    }
    step_mark(m, kStO);
    {
      const Mat* ws[2] = {&Ly.m[4], &Ly.m[5]};
      float* ys[2] = {m->gate, m->up};
      const int rows[2] = {ffn, ffn};
      // with a Q8_0 down projection the same launch also applies swiglu and
      // quantizes its input
      const bool sw = Ly.m[6].dt == NRQ_Q8_0;
      rc = fused_norm_group(m, &xr, &xo, m->xb2, Ly.ffn_norm, ws, ys, rows, 2, sw ? m->xq : nullptr);
      if (rc == 1 && sw) rc = fused_norm_group(m, &xr, &xo, m->xb2, Ly.ffn_norm, ws, ys, rows, 2);
      else if (rc == 0 && sw) swiglu_done = true;
      if (rc == 1) {
        if ((rc = norm_quant(m, xr, m->xb2, Ly.ffn_norm, Ly.m[4].dt))) return rc;
        rc = matvec_group(m, ws, ys, rows, 2, d);
      }
      if (rc) return rc;
    }
    if (!swiglu_done) {
      const bool q8 = Ly.m[6].dt == NRQ_Q8_0;
      if (q8) {
        hipLaunchKernelGGL(nrq::swiglu_kernel, dim3((ffn + 255) / 256), dim3(256), 0, m->stream, m->gate, m->up, ffn,
                           m->xq);
        if (hipGetLastError() != hipSuccess) return mfail(NRQ_ERR_DEVICE, "model: swiglu launch failed");
      } else {  // swiglu inside the Q8_K quantizer, one launch
        nrq::QuantLaunch Q{m->gate, m->xq, (long long)ffn, m->stream};
        Q.up = m->up;
        if (nrq::launch_quantize_q8k(Q)) return mfail(NRQ_ERR_DEVICE, "model: swiglu + quantize launch failed");
      }
    }
    step_mark(m, kStGateUp);
    if ((rc = matvec(m, Ly.m[6], m->xq, m->xb2, d, ffn))) return rc;
    step_mark(m, kStDown);
    pending = m->xb2;
  }
  if ((rc = norm_quant(m, xr, pending, m->out_norm, m->output.dt))) return rc;
  step_mark(m, kStFinalNorm);
  if ((rc = matvec(m, m->output, m->xq, m->logits, c.vocab, d))) return rc;
  if ((rc = scale_logits(m))) return rc;
  step_mark(m, kStHead);
  if (m->samp_t > 0.0f) {
    const int np = (c.vocab + nrq::kSelSlice - 1) / nrq::kSelSlice;
    hipLaunchKernelGGL(nrq::top64_part_kernel, dim3(np), dim3(nrq::kSelPartWaves * 64), 0, m->stream, m->logits,
                       c.vocab, m->samp_part);
    hipLaunchKernelGGL(nrq::top64_sample_kernel, dim3(1), dim3(nrq::kSelWaves * 64), 0, m->stream, m->samp_part, np,
                       m->logits,
                       m->samp_t, m->samp_p, m->rng, m->ctl, m->out_tokens, m->max_out, nullptr);
    if (hipGetLastError() != hipSuccess) return mfail(NRQ_ERR_DEVICE, "model: sampler launch failed");
    step_mark(m, kStPick);
    return NRQ_OK;
  }
  hipLaunchKernelGGL(nrq::argmax_kernel, dim3(1), dim3(nrq::kArgNT), 0, m->stream, m->logits, c.vocab, m->ctl,
                     m->out_tokens, m->max_out);
  if (hipGetLastError() != hipSuccess) return mfail(NRQ_ERR_DEVICE, "model: argmax launch failed");
  step_mark(m, kStPick);
  return NRQ_OK;
}

constexpr int kMaxBatch = 512;  // tokens per prefill chunk (the reference's MAX_BATCH is 64, infer.rs:101)

using AttGroupFn = void (*)(const float*, const int*, int, int, int, int, float, const uint16_t*, const uint16_t*,
                            float*, uint8_t*, uint8_t*);

template <int HD, int NT = nrq::kAttNT, int PROD = nrq::kGrpProd>
AttGroupFn att_group_for(int gh, size_t* lds, int ctx) {
  switch (gh) {
    case 2: *lds = nrq::AttGroup<HD, 2, NT, PROD>::lds_bytes(ctx); return nrq::attention_group_kernel<HD, 2, NT, PROD>;
    case 3: *lds = nrq::AttGroup<HD, 3, NT, PROD>::lds_bytes(ctx); return nrq::attention_group_kernel<HD, 3, NT, PROD>;
    case 4: *lds = nrq::AttGroup<HD, 4, NT, PROD>::lds_bytes(ctx); return nrq::attention_group_kernel<HD, 4, NT, PROD>;
    default: *lds = 0; return nullptr;
  }
}

// Workgroups per head of the decode attention, 32 value dimensions each (all
// of a head's on one XCD) when the head count allows that mapping: two for
// 64-wide heads, four for 128-wide ones; NRQ_ATT_SPLIT=1 forces one.
int att_dim_split(const nrq_model_config& c) {
  const char* env = getenv("NRQ_ATT_SPLIT");
  if (env && env[0] == '1') return 1;
  if (c.n_heads % 8) return 1;
  return c.head_dim == 64 ? 2 : c.head_dim == 128 ? 4 : 1;
}

// The grouped prefill attention for this model's shape, or fn null (then one
// workgroup per query head); NRQ_ATT_GROUP=0 forces the latter. 64-wide heads:
// all of a KV group's heads in one 512-thread workgroup, 24-position chunks for
// four heads (two workgroups per CU at 1032 positions: Llama-3.2-1B prefill
// 20.7 K -> 21.8 K tok/s against one 1024-thread workgroup, 21.2 K with
// 16-position chunks). 128-wide heads: two heads per
// 512-thread workgroup, key rows read in halves and 16-position chunks, so
// that its 80 registers per lane and 46 KB of LDS (at 640 positions) let two
// or three workgroups share a CU (Qwen3-4B prefill 11.35 K -> 12.48 K tok/s
// against one 768-thread workgroup per CU with whole key rows in registers).
struct AttGroupCfg {
  AttGroupFn fn = nullptr;
  size_t lds = 0;
  int gh = 0, nt = 0;
};
AttGroupCfg att_group(const nrq_model_config& c) {
  AttGroupCfg g;
  const char* env = getenv("NRQ_ATT_GROUP");
  if (env && env[0] == '0') return g;
  const int gqa = c.n_heads / c.n_kv_heads;
  if (c.head_dim == 64) {
    g.fn = att_group_for<64, 512, 28 * 256>(gqa, &g.lds, c.ctx);  // 24 positions per chunk with four heads
    g.gh = gqa;
    g.nt = 512;
  } else if (c.head_dim == 128 && gqa % 2 == 0) {
    g.fn = nrq::attention_group_kernel<128, 2, 512>;
    g.lds = nrq::AttGroup<128, 2, 512>::lds_bytes(c.ctx);
    g.gh = 2;
    g.nt = 512;
  }
  if (!g.fn || g.lds > 160 * 1024) g = AttGroupCfg{};
  return g;
}

int prefill_alloc(nrq_model* m) {
  if (m->bx) return NRQ_OK;
  const auto& c = m->cfg;
  const size_t B = kMaxBatch, maxd = (size_t)m->maxd;
  struct {
    void** p;
    size_t bytes;
  } allocs[] = {
      {(void**)&m->bx, B * c.dim * 4},          {(void**)&m->bxb, B * c.dim * 4},
      {(void**)&m->bxn, B * maxd * 4},          {(void**)&m->bq, B * m->att_dim * 4},
      {(void**)&m->bk, B * m->kv_dim * 4},      {(void**)&m->bv, B * m->kv_dim * 4},
      {(void**)&m->battn, B * m->att_dim * 4},  {(void**)&m->bgate, B * c.ffn_dim * 4},
      {(void**)&m->bup, B * c.ffn_dim * 4},     {(void**)&m->brope, B * c.head_dim * 4},
      {(void**)&m->bxq, B * act_bytes(NRQ_Q8_0, maxd) + 64}, {(void**)&m->bxq2, B * act_bytes(NRQ_Q4_K, maxd) + 64},
      {(void**)&m->btok, B * 4},
  };
  for (auto& a : allocs) MHIP(hipMalloc(a.p, a.bytes));
  return NRQ_OK;
}

int matmul_rows(nrq_model* m, const Mat& w, const uint8_t* xs, float* y, int rows, int cols, int B) {
  nrq::MatmulLaunch L;
  L.w = w.w;
  L.xs = xs;
  L.y = y;
  L.rows = rows;
  L.bpr = cols / qk_of(w.dt);
  L.batch = B;
  L.stream = m->stream;
  const int rc = nrq::launch_matmul(w.dt, nrq::kOrderScalar, L);
  return rc ? mfail(rc == nrq::NRQ_LAUNCH_TOO_WIDE ? NRQ_ERR_UNSUPPORTED : NRQ_ERR_DEVICE, "model: matmul launch failed")
            : NRQ_OK;
}

// Matmuls of one [B][cols] input (Acts::matmul_group, infer.rs:180-228): the
// rows are quantized once per format; m->bxq holds the Q8_0 blocks when
// `have_q8` (written by the producing kernel), m->bxq2 the Q8_K ones.
int matmul_group_rows(nrq_model* m, const Mat* const* ws, float* const* ys, const int* rows, int n, const float* x,
                      int cols, int B, bool have_q8, bool have_q8k = false) {
  bool need_q8 = false, need_q8k = false;
  for (int i = 0; i < n; i++) (ws[i]->dt == NRQ_Q8_0 ? need_q8 : need_q8k) = true;
  int rc;
  if (need_q8 && !have_q8 && (rc = quantize_for(m, NRQ_Q8_0, x, B * cols, m->bxq))) return rc;
  if (need_q8k && !have_q8k && (rc = quantize_for(m, NRQ_Q4_K, x, B * cols, m->bxq2))) return rc;
  // two runs of different K-quant formats (Qwen3 Q4_K_M: q|k, then the Q6_K
  // v) in one launch where the prefill kernel takes the pair
  {
    int j = 1;
    while (j < n && ws[j]->dt == ws[0]->dt) j++;
    bool two = j < n && ws[0]->dt != NRQ_Q8_0 && ws[j]->dt != NRQ_Q8_0;
    for (int k = j + 1; k < n && two; k++) two = ws[k]->dt == ws[j]->dt;
    if (two) {
      nrq::MatmulGroupLaunch G[2]{};
      for (int gi = 0; gi < 2; gi++) {
        const int a = gi ? j : 0, b = gi ? n : j;
        for (int k = a; k < b; k++) {
          G[gi].w[k - a] = ws[k]->w;
          G[gi].y[k - a] = ys[k];
          G[gi].rows[k - a] = rows[k];
        }
        G[gi].nmat = b - a;
        G[gi].xs = m->bxq2;
        G[gi].bpr = cols / 256;
        G[gi].batch = B;
        G[gi].stream = m->stream;
      }
      const int lr = nrq::launch_mmt_group2(ws[0]->dt, G[0], ws[j]->dt, G[1]);
      if (lr == nrq::NRQ_LAUNCH_OK) return NRQ_OK;
      if (lr != nrq::NRQ_LAUNCH_BAD_ARG) return mfail(NRQ_ERR_DEVICE, "model: matmul group launch failed");
    }
  }
  // each run of neighbours of one format in one launch where the prefill
  // kernel takes it
  for (int i = 0; i < n;) {
    int j = i + 1;
    while (j < n && ws[j]->dt == ws[i]->dt) j++;
    bool done = false;
    if (j - i > 1) {
      nrq::MatmulGroupLaunch G{};
      for (int k = i; k < j; k++) {
        G.w[k - i] = ws[k]->w;
        G.y[k - i] = ys[k];
        G.rows[k - i] = rows[k];
      }
      G.nmat = j - i;
      G.xs = ws[i]->dt == NRQ_Q8_0 ? m->bxq : m->bxq2;
      G.bpr = cols / qk_of(ws[i]->dt);
      G.batch = B;
      G.stream = m->stream;
      const int lr = nrq::launch_mmt_group(ws[i]->dt, G);
      if (lr != nrq::NRQ_LAUNCH_OK && lr != nrq::NRQ_LAUNCH_BAD_ARG)
        return mfail(NRQ_ERR_DEVICE, "model: matmul group launch failed");
      done = lr == nrq::NRQ_LAUNCH_OK;
    }
    for (int k = i; k < j && !done; k++)
      if ((rc = matmul_rows(m, *ws[k], ws[k]->dt == NRQ_Q8_0 ? m->bxq : m->bxq2, ys[k], rows[k], cols, B))) return rc;
    i = j;
  }
  return NRQ_OK;
}

bool any_q8(const Mat* const* ws, int n) {
  for (int i = 0; i < n; i++)
    if (ws[i]->dt == NRQ_Q8_0) return true;
  return false;
}

bool any_kquant(const Mat* const* ws, int n) {
  for (int i = 0; i < n; i++)
    if (ws[i]->dt != NRQ_Q8_0) return true;
  return false;
}

// InferCtx::prefill_chunk (infer.rs:601-750) for B tokens at positions
// pos..pos+B-1 (ctl[CTL_POS] = pos): batched norms and matmuls, all the
// chunk's K/V appended, then causal attention for every (head, token); the
// last token's logits. Each kernel computes a row exactly as the decode step
// does, so the KV cache and logits equal B forward steps bit for bit.
int enqueue_prefill(nrq_model* m, int B) {
  const auto& c = m->cfg;
  const int d = c.dim, kvd = m->kv_dim, att = m->att_dim, ffn = c.ffn_dim;
  hipLaunchKernelGGL(nrq::embed_rows_kernel, dim3((d + 255) / 256, B), dim3(256), 0, m->stream,
                     (const uint8_t*)m->embed.w, m->embed.dt, m->btok, m->ctl, d, m->bx, m->freqs, c.head_dim / 2,
                     m->brope,
                     m->embed_scale);
  if (hipGetLastError() != hipSuccess) return mfail(NRQ_ERR_DEVICE, "model: embed launch failed");
  const float scale = m->att_scale;
  const float* pending = nullptr;
  int rc;
  for (int l = 0; l < c.n_layers; l++) {
    const Layer& Ly = m->L[l];
    {
      const Mat* ws[3] = {&Ly.m[0], &Ly.m[1], &Ly.m[2]};
      float* ys[3] = {m->bq, m->bk, m->bv};
      const int rows[3] = {att, kvd, kvd};
      const bool q8 = any_q8(ws, 3), q8k = any_kquant(ws, 3);
      hipLaunchKernelGGL(nrq::norm_kernel, dim3(B), dim3(nrq::kNormNT), 0, m->stream, m->bx, pending, Ly.attn_norm,
                         d, c.norm_eps, m->res_scale, m->bxn, q8 ? m->bxq : nullptr, q8k ? m->bxq2 : nullptr);
      if (hipGetLastError() != hipSuccess) return mfail(NRQ_ERR_DEVICE, "model: norm launch failed");
      if ((rc = matmul_group_rows(m, ws, ys, rows, 3, m->bxn, d, B, q8, q8k))) return rc;
    }
    hipLaunchKernelGGL(nrq::rope_append_kernel, dim3(B, (c.n_heads + c.n_kv_heads + 3) / 4), dim3(256), 0, m->stream,
                       m->bq, m->bk, m->bv, m->brope,
                       m->ctl, c.n_heads, c.n_kv_heads, c.head_dim, c.ctx, l, m->kc, m->vc, Ly.q_norm, Ly.k_norm,
                       c.norm_eps, m->rope_neox);
    if (hipGetLastError() != hipSuccess) return mfail(NRQ_ERR_DEVICE, "model: rope launch failed");
    {
      const bool q8 = Ly.m[3].dt == NRQ_Q8_0;
      const AttGroupCfg gk = att_group(c);
      // a K-quant o projection's Q8_K input, written by the attention when a
      // workgroup's heads are one 256-value block
      const bool q8k = !q8 && gk.fn && gk.gh * c.head_dim == 256;
      if (gk.fn) {
        hipLaunchKernelGGL(gk.fn, dim3(c.n_heads / gk.gh, B), dim3(gk.nt), gk.lds, m->stream, m->bq, m->ctl, c.n_heads,
                           c.n_kv_heads, c.ctx, l, scale, m->kc, m->vc, m->battn, q8 ? m->bxq : nullptr,
                           q8k ? m->bxq2 : nullptr);
      } else {
        auto* kern = c.head_dim == 32   ? nrq::attention_kernel<32, true>
                     : c.head_dim == 64 ? nrq::attention_kernel<64, true>
                     : c.head_dim == 96 ? nrq::attention_kernel<96, true>
                                        : nrq::attention_kernel<128, true>;
        hipLaunchKernelGGL(kern, dim3(c.n_heads, B), dim3(nrq::att_threads(c.head_dim)), m->att_lds, m->stream, m->bq,
                           m->bk, m->bv,
                           m->brope, m->ctl, c.n_heads, c.n_kv_heads, c.ctx, l, scale, m->kc, m->vc, m->battn,
                           q8 ? m->bxq : nullptr, nullptr, nullptr, 0.0f, 0);
      }
      if (hipGetLastError() != hipSuccess) return mfail(NRQ_ERR_DEVICE, "model: attention launch failed");
      const Mat* ws[1] = {&Ly.m[3]};
      float* ys[1] = {m->bxb};
      const int rows[1] = {d};
      if ((rc = matmul_group_rows(m, ws, ys, rows, 1, m->battn, att, B, q8, q8k))) return rc;
    }
    {
      const Mat* ws[2] = {&Ly.m[4], &Ly.m[5]};
      float* ys[2] = {m->bgate, m->bup};
      const int rows[2] = {ffn, ffn};
      const bool q8 = any_q8(ws, 2), q8k = any_kquant(ws, 2);
      hipLaunchKernelGGL(nrq::norm_kernel, dim3(B), dim3(nrq::kNormNT), 0, m->stream, m->bx, m->bxb, Ly.ffn_norm, d,
                         c.norm_eps, m->res_scale, m->bxn, q8 ? m->bxq : nullptr, q8k ? m->bxq2 : nullptr);
      if (hipGetLastError() != hipSuccess) return mfail(NRQ_ERR_DEVICE, "model: norm launch failed");
      if ((rc = matmul_group_rows(m, ws, ys, rows, 2, m->bxn, d, B, q8, q8k))) return rc;
    }
    {
      const bool q8 = Ly.m[6].dt == NRQ_Q8_0;
      const long long n = (long long)B * ffn;
      if (q8) {
        hipLaunchKernelGGL(nrq::swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, m->stream, m->bgate,
                           m->bup, (int)n, m->bxq);
        if (hipGetLastError() != hipSuccess) return mfail(NRQ_ERR_DEVICE, "model: swiglu launch failed");
      } else {
        // swiglu inside the Q8_K quantizer, as in the decode step (vec.rs:45-52)
        nrq::QuantLaunch Q{m->bgate, m->bxq2, n, m->stream, m->bup};
        if (nrq::launch_quantize_q8k(Q)) return mfail(NRQ_ERR_DEVICE, "model: swiglu quantize launch failed");
      }
      const Mat* ws[1] = {&Ly.m[6]};
      float* ys[1] = {m->bxb};
      const int rows[1] = {d};
      if ((rc = matmul_group_rows(m, ws, ys, rows, 1, m->bgate, ffn, B, q8, !q8))) return rc;
    }
    pending = m->bxb;
  }
  // only the last token's logits (infer.rs:738-745); the other rows' final
  // residual add is never read
  const size_t last = (size_t)(B - 1) * d;
  if ((rc = norm_quant(m, m->bx + last, pending + last, m->out_norm, m->output.dt))) return rc;
  if ((rc = matvec(m, m->output, m->xq, m->logits, c.vocab, d))) return rc;
  return scale_logits(m);
}

int check_ready(nrq_model* m, const char* name) {
  if (!m) return mfail(NRQ_ERR_ARG, "model: null handle");
  if (!m->embed.w || !m->out_norm || !m->output.w) return mfail(NRQ_ERR_ARG, "model: embedding/output tensors not set");
  for (int l = 0; l < m->cfg.n_layers; l++) {
    const Layer& Ly = m->L[l];
    for (int i = 0; i < 7; i++)
      if (!Ly.m[i].w) return mfail(NRQ_ERR_ARG, "model: a layer matrix is not set");
    if (!Ly.attn_norm || !Ly.ffn_norm) return mfail(NRQ_ERR_ARG, "model: a layer norm is not set");
    if (!Ly.q_norm != !Ly.k_norm) return mfail(NRQ_ERR_ARG, "model: attn_q_norm and attn_k_norm come as a pair");
  }
  // the prefill rope kernel holds every head's squares in LDS
  if (m->L[0].q_norm && (size_t)(m->cfg.n_heads + m->cfg.n_kv_heads) * (m->cfg.head_dim + 1) * 4 > 65536)
    return mfail(NRQ_ERR_UNSUPPORTED, "model: too many heads for the qk-norm prefill kernel");
  (void)name;
  return NRQ_OK;
}

}  // namespace

extern "C" {

int nrq_model_create(const nrq_model_config* cfg, nrq_model** out) {
  if (!cfg || !out) return mfail(NRQ_ERR_ARG, "nrq_model_create: null argument");
  const nrq_model_config& c = *cfg;
  if (c.dim <= 0 || c.n_layers <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 || c.head_dim <= 0 || c.ffn_dim <= 0 ||
      c.vocab <= 0 || c.ctx <= 0)
    return mfail(NRQ_ERR_SHAPE, "nrq_model_create: non-positive dimension");
  // products in 64 bits: the buffers below are indexed with int
  if ((long long)c.n_heads * c.head_dim > INT_MAX || (long long)c.n_kv_heads * c.head_dim > INT_MAX)
    return mfail(NRQ_ERR_UNSUPPORTED, "nrq_model_create: attention width does not fit an int");
  if (c.n_heads % c.n_kv_heads || c.head_dim % 32 || c.head_dim > 128 || c.dim % 256 || c.ffn_dim % 256 ||
      ((long long)c.n_heads * c.head_dim) % 256)
    return mfail(NRQ_ERR_UNSUPPORTED, "nrq_model_create: head or width layout not supported");
  if (c.dim > nrq::kNormMax || c.ctx > nrq::kAttMaxCtx)
    return mfail(NRQ_ERR_UNSUPPORTED, "nrq_model_create: dim or context larger than the kernels' LDS buffers");
  nrq_model* m = new nrq_model();
  m->cfg = c;
  m->att_scale = 1.0f / sqrtf((float)c.head_dim);  // infer.rs:455-459 without attn_scale
  m->kv_dim = c.n_kv_heads * c.head_dim;
  m->att_dim = c.n_heads * c.head_dim;
  m->maxd = std::max(std::max(c.dim, m->att_dim), c.ffn_dim);
  m->L.resize(c.n_layers);
  m->att_lds = ((size_t)((c.ctx + 127) & ~127) + 2 * nrq::kAttProd + 3 * (size_t)c.head_dim + 32) * 4 +
               nrq::kAttRing;
  auto bail = [&](hipError_t e, const char* what) {
    nrq::set_last_error((std::string(what) + ": " + hipGetErrorString(e)).c_str());
    nrq_model_destroy(m);
    return NRQ_ERR_DEVICE;
  };
  hipError_t e;
  if ((e = hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking)) != hipSuccess) return bail(e, "stream");
  const size_t kvn = (size_t)c.n_layers * c.ctx * m->kv_dim;
  struct {
    void** p;
    size_t bytes;
  } allocs[] = {
      {(void**)&m->freqs, (size_t)c.head_dim / 2 * 4}, {(void**)&m->rope_cs, (size_t)c.head_dim * 4},
      {(void**)&m->kc, kvn * 2}, {(void**)&m->vc, kvn * 2},
      {(void**)&m->x, (size_t)c.dim * 4}, {(void**)&m->x2, (size_t)c.dim * 4}, {(void**)&m->xb, (size_t)m->maxd * 4},
      {(void**)&m->q, (size_t)m->att_dim * 4}, {(void**)&m->k, (size_t)m->kv_dim * 4},
      {(void**)&m->v, (size_t)m->kv_dim * 4}, {(void**)&m->attn, (size_t)m->att_dim * 4},
      {(void**)&m->gate, (size_t)c.ffn_dim * 4}, {(void**)&m->up, (size_t)c.ffn_dim * 4},
      {(void**)&m->xb2, (size_t)c.dim * 4}, {(void**)&m->logits, (size_t)c.vocab * 4},
      {(void**)&m->xq, act_bytes(NRQ_Q8_0, m->maxd) + act_bytes(NRQ_Q4_K, m->maxd) + 64},
      {(void**)&m->xq2, act_bytes(NRQ_Q8_0, m->maxd) + act_bytes(NRQ_Q4_K, m->maxd) + 64},
      {(void**)&m->ctl, nrq::CTL_WORDS * 4},
      {(void**)&m->rng, 8},
      {(void**)&m->samp_part, (size_t)(c.vocab + nrq::kSelSlice - 1) / nrq::kSelSlice * nrq::kSelPart * 4},
  };
  for (auto& a : allocs) {
    if ((e = hipMalloc(a.p, a.bytes)) != hipSuccess) return bail(e, "hipMalloc");
    if ((e = hipMemset(*a.p, 0, a.bytes)) != hipSuccess) return bail(e, "hipMemset");
  }
  // rope_freqs (rope.rs:14-34, no scaling): theta^(-2i/head_dim), on the host
  std::vector<float> f(c.head_dim / 2);
  for (int i = 0; i < c.head_dim / 2; i++) {
    const float exponent = -2.0f * (float)i / (float)c.head_dim;
    f[i] = powf(c.rope_theta, exponent);
  }
  if ((e = hipMemcpy(m->freqs, f.data(), f.size() * 4, hipMemcpyHostToDevice)) != hipSuccess) return bail(e, "freqs");
  *out = m;
  return NRQ_OK;
}

int nrq_model_set_tensor(nrq_model* m, int kind, int layer, int dtype, const void* dev_ptr) {
  if (!m || !dev_ptr) return mfail(NRQ_ERR_ARG, "nrq_model_set_tensor: null argument");
  const bool is_norm = kind == NRQ_TENSOR_ATTN_NORM || kind == NRQ_TENSOR_FFN_NORM || kind == NRQ_TENSOR_OUTPUT_NORM ||
                       kind == NRQ_TENSOR_ATTN_Q_NORM || kind == NRQ_TENSOR_ATTN_K_NORM;
  if (is_norm) {
    if (dtype != NRQ_F32) return mfail(NRQ_ERR_ARG, "nrq_model_set_tensor: norms are f32");
    if (((uintptr_t)dev_ptr & 15) != 0) return mfail(NRQ_ERR_ARG, "nrq_model_set_tensor: norm not 16-byte aligned");
  } else {
    if (dtype != NRQ_Q8_0 && dtype != NRQ_Q4_K && dtype != NRQ_Q6_K)
      return mfail(NRQ_ERR_ARG, "nrq_model_set_tensor: unknown matrix dtype");
    if (((uintptr_t)dev_ptr & 15) != 0) return mfail(NRQ_ERR_ARG, "nrq_model_set_tensor: matrix not 16-byte aligned");
  }
  const bool layered = kind >= NRQ_TENSOR_ATTN_NORM && kind <= NRQ_TENSOR_ATTN_K_NORM;
  if (layered && (layer < 0 || layer >= m->cfg.n_layers))
    return mfail(NRQ_ERR_ARG, "nrq_model_set_tensor: layer out of range");
  const Mat mat{dev_ptr, dtype};
  switch (kind) {
    case NRQ_TENSOR_TOK_EMBED:
      if (dtype != NRQ_Q8_0 && m->cfg.dim % 256)
        return mfail(NRQ_ERR_SHAPE, "nrq_model_set_tensor: a K-quant embedding needs dim % 256 == 0");
      m->embed = mat;
      if (!m->output.w) m->output = mat;  // tied head until an output tensor is set
      break;
    case NRQ_TENSOR_OUTPUT: m->output = mat; break;
    case NRQ_TENSOR_OUTPUT_NORM: m->out_norm = (const float*)dev_ptr; break;
    case NRQ_TENSOR_ATTN_NORM: m->L[layer].attn_norm = (const float*)dev_ptr; break;
    case NRQ_TENSOR_FFN_NORM: m->L[layer].ffn_norm = (const float*)dev_ptr; break;
    case NRQ_TENSOR_ATTN_Q: m->L[layer].m[0] = mat; break;
    case NRQ_TENSOR_ATTN_K: m->L[layer].m[1] = mat; break;
    case NRQ_TENSOR_ATTN_V: m->L[layer].m[2] = mat; break;
    case NRQ_TENSOR_ATTN_O: m->L[layer].m[3] = mat; break;
    case NRQ_TENSOR_FFN_GATE: m->L[layer].m[4] = mat; break;
    case NRQ_TENSOR_FFN_UP: m->L[layer].m[5] = mat; break;
    case NRQ_TENSOR_FFN_DOWN: m->L[layer].m[6] = mat; break;
    case NRQ_TENSOR_ATTN_Q_NORM: m->L[layer].q_norm = (const float*)dev_ptr; break;
    case NRQ_TENSOR_ATTN_K_NORM: m->L[layer].k_norm = (const float*)dev_ptr; break;
    default: return mfail(NRQ_ERR_ARG, "nrq_model_set_tensor: unknown tensor kind");
  }
  if (m->exec) {  // tensors changed: the captured step is stale
    hipGraphExecDestroy(m->exec);
    hipGraphDestroy(m->graph);
    m->exec = nullptr;
    m->graph = nullptr;
  }
  return NRQ_OK;
}

int nrq_model_set_recipe(nrq_model* m, int rope_style, float embed_scale, float attn_scale, float residual_scale,
                         float logit_scale) {
  if (!m) return mfail(NRQ_ERR_ARG, "nrq_model_set_recipe: null handle");
  if (rope_style != NRQ_ROPE_ADJACENT && rope_style != NRQ_ROPE_NEOX)
    return mfail(NRQ_ERR_ARG, "nrq_model_set_recipe: unknown rope style");
  // the ranges Model::parse accepts for the muP scalars
  if (!std::isfinite(embed_scale) || !std::isfinite(attn_scale) || attn_scale < 0.0f ||
      !std::isfinite(residual_scale) || residual_scale <= 0.0f || !std::isfinite(logit_scale) || logit_scale <= 0.0f)
    return mfail(NRQ_ERR_ARG, "nrq_model_set_recipe: muP scale out of range");
  MHIP(hipStreamSynchronize(m->stream));
  m->rope_neox = rope_style == NRQ_ROPE_NEOX;
  m->embed_scale = embed_scale;
  m->att_scale = attn_scale != 0.0f ? attn_scale : 1.0f / sqrtf((float)m->cfg.head_dim);
  m->res_scale = residual_scale;
  m->logit_recip = 1.0f / logit_scale;
  if (m->exec) {  // the captured step holds the old scalars
    hipGraphExecDestroy(m->exec);
    hipGraphDestroy(m->graph);
    m->exec = nullptr;
    m->graph = nullptr;
  }
  return NRQ_OK;
}

int nrq_model_set_rope_freqs(nrq_model* m, const float* freqs, int n) {
  if (!m || !freqs) return mfail(NRQ_ERR_ARG, "nrq_model_set_rope_freqs: null argument");
  if (n != m->cfg.head_dim / 2) return mfail(NRQ_ERR_SHAPE, "nrq_model_set_rope_freqs: need head_dim / 2 values");
  MHIP(hipStreamSynchronize(m->stream));
  MHIP(hipMemcpy(m->freqs, freqs, (size_t)n * 4, hipMemcpyHostToDevice));
  return NRQ_OK;
}

int nrq_model_set_sampler(nrq_model* m, float temperature, float top_p, uint64_t seed) {
  if (!m) return mfail(NRQ_ERR_ARG, "nrq_model_set_sampler: null handle");
  MHIP(hipStreamSynchronize(m->stream));
  const unsigned long long st = (unsigned long long)(seed | 1u);  // sample.rs:19
  MHIP(hipMemcpy(m->rng, &st, 8, hipMemcpyHostToDevice));
  const bool was = m->samp_t > 0.0f, now = temperature > 0.0f;
  m->samp_t = temperature;
  m->samp_p = top_p;
  if (m->exec && (was || now)) {  // the captured step's last kernel (or its arguments) changes
    hipGraphExecDestroy(m->exec);
    hipGraphDestroy(m->graph);
    m->exec = nullptr;
    m->graph = nullptr;
  }
  return NRQ_OK;
}

int nrq_model_sampler_state(nrq_model* m, uint64_t* state) {
  if (!m || !state) return mfail(NRQ_ERR_ARG, "nrq_model_sampler_state: null argument");
  MHIP(hipStreamSynchronize(m->stream));
  unsigned long long st = 0;
  MHIP(hipMemcpy(&st, m->rng, 8, hipMemcpyDeviceToHost));
  *state = st;
  return NRQ_OK;
}

int nrq_dev_sample(const float* logits, int n, float temperature, float top_p, uint64_t* rng, uint32_t* token,
                   void* stream) {
  if (!logits || !token || (temperature > 0.0f && !rng)) return mfail(NRQ_ERR_ARG, "nrq_dev_sample: null pointer");
  if (n <= 0) return mfail(NRQ_ERR_ARG, "nrq_dev_sample: empty logits");
  if (temperature > 0.0f) {
    // the partial lists live in stream-ordered memory, so calls on different
    // streams do not share them
    hipStream_t s = (hipStream_t)stream;
    const int np = (n + nrq::kSelSlice - 1) / nrq::kSelSlice;
    unsigned long long* part = nullptr;
    if (hipMallocAsync((void**)&part, (size_t)np * nrq::kSelPart * 4, s) != hipSuccess)
      return mfail(NRQ_ERR_DEVICE, "nrq_dev_sample: hipMallocAsync failed");
    hipLaunchKernelGGL(nrq::top64_part_kernel, dim3(np), dim3(nrq::kSelPartWaves * 64), 0, s, logits, n, part);
    hipLaunchKernelGGL(nrq::top64_sample_kernel, dim3(1), dim3(nrq::kSelWaves * 64), 0, s, part, np, logits,
                       temperature,
                       top_p, (unsigned long long*)rng, nullptr, nullptr, 0, token);
    const hipError_t le = hipGetLastError();
    if (hipFreeAsync(part, s) != hipSuccess || le != hipSuccess)
      return mfail(NRQ_ERR_DEVICE, "nrq_dev_sample: launch failed");
    return NRQ_OK;
  } else {
    hipLaunchKernelGGL(nrq::argmax_kernel, dim3(1), dim3(nrq::kArgNT), 0, (hipStream_t)stream, logits, n, nullptr,
                       token, 1);
  }
  return hipGetLastError() == hipSuccess ? NRQ_OK : mfail(NRQ_ERR_DEVICE, "nrq_dev_sample: launch failed");
}

int nrq_dev_sample_noalloc(const float* logits, int n, float temperature, float top_p, uint64_t* rng,
                           uint32_t* token, void* stream) {
  if (!logits || !token || (temperature > 0.0f && !rng))
    return mfail(NRQ_ERR_ARG, "nrq_dev_sample_noalloc: null pointer");
  if (n <= 0) return mfail(NRQ_ERR_ARG, "nrq_dev_sample_noalloc: empty logits");
  if (n > nrq::kSampleMaxLogits)
    return mfail(NRQ_ERR_UNSUPPORTED, "nrq_dev_sample_noalloc: more than 524288 logits (its fixed scratch holds "
                                      "the partial lists of at most that many)");
  hipStream_t s = (hipStream_t)stream;
  if (temperature <= 0.0f) {  // argmax: no scratch
    hipLaunchKernelGGL(nrq::argmax_kernel, dim3(1), dim3(nrq::kArgNT), 0, s, logits, n, nullptr, token, 1);
    return hipGetLastError() == hipSuccess ? NRQ_OK : mfail(NRQ_ERR_DEVICE, "nrq_dev_sample_noalloc: launch failed");
  }
  if (s) {  // the scratch used is the current device's: the stream must be on it
    int sdev = -1, cur = -1;
    if (hipStreamGetDevice(s, &sdev) != hipSuccess || hipGetDevice(&cur) != hipSuccess || sdev != cur)
      return mfail(NRQ_ERR_ARG, "nrq_dev_sample_noalloc: the stream is not on the current device");
  }
  void* part = nullptr;
  int rc = scratch_on_current_device(&part);
  if (rc) return rc;
  const int np = (n + nrq::kSelSlice - 1) / nrq::kSelSlice;
  hipLaunchKernelGGL(nrq::top64_part_kernel, dim3(np), dim3(nrq::kSelPartWaves * 64), 0, s, logits, n,
                     (unsigned long long*)part);
  hipLaunchKernelGGL(nrq::top64_sample_kernel, dim3(1), dim3(nrq::kSelWaves * 64), 0, s,
                     (const unsigned long long*)part, np, logits, temperature, top_p, (unsigned long long*)rng, nullptr,
                     nullptr, 0, token);
  return hipGetLastError() == hipSuccess ? NRQ_OK : mfail(NRQ_ERR_DEVICE, "nrq_dev_sample_noalloc: launch failed");
}

int nrq_model_reset(nrq_model* m) {
  if (!m) return mfail(NRQ_ERR_ARG, "nrq_model_reset: null handle");
  MHIP(hipStreamSynchronize(m->stream));
  MHIP(hipMemset(m->ctl, 0, nrq::CTL_WORDS * 4));
  m->host_pos = 0;
  return NRQ_OK;
}

int nrq_model_pos(const nrq_model* m) { return m ? m->host_pos : -1; }

int nrq_model_forward(nrq_model* m, uint32_t token, float* logits_host) {
  int rc = check_ready(m, "nrq_model_forward");
  if (rc) return rc;
  // infer.rs:513: assert!(pos < d.ctx, "context window exhausted")
  if (m->host_pos >= m->cfg.ctx) return mfail(NRQ_ERR_SHAPE, "assertion failed: pos < d.ctx: context window exhausted");
  if (token >= (uint32_t)m->cfg.vocab) return mfail(NRQ_ERR_ARG, "nrq_model_forward: token out of vocabulary");
  if ((rc = set_ctl(m, nrq::CTL_TOKEN, (int)token))) return rc;
  uint32_t* keep = m->out_tokens;
  m->out_tokens = nullptr;
  rc = enqueue_step(m);
  m->out_tokens = keep;
  if (rc) return rc;
  if (logits_host)
    MHIP(hipMemcpyAsync(logits_host, m->logits, (size_t)m->cfg.vocab * 4, hipMemcpyDeviceToHost, m->stream));
  MHIP(hipStreamSynchronize(m->stream));
  m->host_pos += 1;
  return NRQ_OK;
}

int nrq_model_step_profile(nrq_model* m, uint32_t token, float* stage_us, int n_stages) {
  int rc = check_ready(m, "nrq_model_step_profile");
  if (rc) return rc;
  if (!stage_us || n_stages < kStCount) return mfail(NRQ_ERR_ARG, "nrq_model_step_profile: needs 9 stage slots");
  if (m->host_pos >= m->cfg.ctx) return mfail(NRQ_ERR_SHAPE, "assertion failed: pos < d.ctx: context window exhausted");
  if (token >= (uint32_t)m->cfg.vocab) return mfail(NRQ_ERR_ARG, "nrq_model_step_profile: token out of vocabulary");
  if ((rc = set_ctl(m, nrq::CTL_TOKEN, (int)token))) return rc;
  MHIP(hipStreamSynchronize(m->stream));
  hipEvent_t e0 = nullptr;
  MHIP(hipEventCreate(&e0));
  // 3 ms of hold (the host enqueues a step in well under that), then the step
  hipLaunchKernelGGL(hold_kernel, dim3(1), dim3(64), 0, m->stream, 300000LL);
  hipEventRecord(e0, m->stream);
  uint32_t* keep = m->out_tokens;
  m->out_tokens = nullptr;
  m->timing = true;
  rc = enqueue_step(m);
  m->timing = false;
  m->out_tokens = keep;
  const hipError_t es = hipStreamSynchronize(m->stream);
  for (int i = 0; i < n_stages; i++) stage_us[i] = 0.0f;
  hipEvent_t prev = e0;
  for (size_t i = 0; i < m->tev.size() && es == hipSuccess && rc == 0; i++) {
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, prev, m->tev[i]) == hipSuccess) stage_us[m->tstage[i]] += ms * 1e3f;
    prev = m->tev[i];
  }
  for (hipEvent_t e : m->tev) hipEventDestroy(e);
  m->tev.clear();
  m->tstage.clear();
  hipEventDestroy(e0);
  if (rc) return rc;
  MHIP(es);
  m->host_pos += 1;
  return NRQ_OK;
}

int nrq_model_prefill(nrq_model* m, const uint32_t* tokens, int n, float* logits_host) {
  int rc = check_ready(m, "nrq_model_prefill");
  if (rc) return rc;
  // infer.rs:754: assert!(!tokens.is_empty())
  if (n <= 0) return mfail(NRQ_ERR_SHAPE, "assertion failed: !tokens.is_empty()");
  if (!tokens) return mfail(NRQ_ERR_ARG, "nrq_model_prefill: null tokens");
  for (int i = 0; i < n; i++)
    if (tokens[i] >= (uint32_t)m->cfg.vocab) return mfail(NRQ_ERR_ARG, "nrq_model_prefill: token out of vocabulary");
  // infer.rs:605 (checked per chunk there; the chunks are consecutive)
  if (m->host_pos + n > m->cfg.ctx)
    return mfail(NRQ_ERR_SHAPE, "assertion failed: self.pos + b <= d.ctx: context window exhausted");
  if ((rc = prefill_alloc(m))) return rc;
  for (int i0 = 0; i0 < n; i0 += kMaxBatch) {
    const int B = std::min(kMaxBatch, n - i0);
    const int base = m->host_pos;
    MHIP(hipMemcpyAsync(m->btok, tokens + i0, (size_t)B * 4, hipMemcpyHostToDevice, m->stream));
    if ((rc = set_ctl(m, nrq::CTL_POS, base)) || (rc = enqueue_prefill(m, B)) ||
        (rc = set_ctl(m, nrq::CTL_POS, base + B))) {
      hipStreamSynchronize(m->stream);  // the token copy reads the caller's array
      return rc;
    }
    MHIP(hipStreamSynchronize(m->stream));
    m->host_pos = base + B;
  }
  if (logits_host)
    MHIP(hipMemcpyAsync(logits_host, m->logits, (size_t)m->cfg.vocab * 4, hipMemcpyDeviceToHost, m->stream));
  MHIP(hipStreamSynchronize(m->stream));
  return NRQ_OK;
}

int nrq_model_generate(nrq_model* m, uint32_t token, int n, uint32_t* out_tokens, float* last_logits) {
  int rc = check_ready(m, "nrq_model_generate");
  if (rc) return rc;
  if (n <= 0) return NRQ_OK;
  if (!out_tokens) return mfail(NRQ_ERR_ARG, "nrq_model_generate: null output");
  if (m->host_pos + n > m->cfg.ctx) return mfail(NRQ_ERR_SHAPE, "assertion failed: pos < d.ctx: context window exhausted");
  if (token >= (uint32_t)m->cfg.vocab) return mfail(NRQ_ERR_ARG, "nrq_model_generate: token out of vocabulary");
  if (n > m->max_out) {
    if (m->out_tokens) hipFree(m->out_tokens);
    m->out_tokens = nullptr;
    m->max_out = 0;
    MHIP(hipMalloc(&m->out_tokens, (size_t)n * 4));
    m->max_out = n;
    if (m->exec) {  // the captured step points at the old buffer
      hipGraphExecDestroy(m->exec);
      hipGraphDestroy(m->graph);
      m->exec = nullptr;
      m->graph = nullptr;
    }
  }
  if ((rc = set_ctl(m, nrq::CTL_TOKEN, (int)token, nrq::CTL_STEP, 0))) return rc;
  if (!m->exec) {
    MHIP(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
    rc = enqueue_step(m);
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(m->stream, &g);
    if (rc) {
      if (g) hipGraphDestroy(g);
      return rc;
    }
    if (e != hipSuccess) return mfail(NRQ_ERR_DEVICE, "nrq_model_generate: graph capture failed");
    hipGraphExec_t x = nullptr;
    if (hipGraphInstantiate(&x, g, nullptr, nullptr, 0) != hipSuccess) {
      hipGraphDestroy(g);
      return mfail(NRQ_ERR_DEVICE, "nrq_model_generate: graph instantiate failed");
    }
    m->graph = g;
    m->exec = x;
  }
  // every copy into the caller's buffers completes before this returns, on error too
  hipError_t e = hipSuccess;
  for (int i = 0; i < n && e == hipSuccess; i++) e = hipGraphLaunch(m->exec, m->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(out_tokens, m->out_tokens, (size_t)n * 4, hipMemcpyDeviceToHost, m->stream);
  if (e == hipSuccess && last_logits)
    e = hipMemcpyAsync(last_logits, m->logits, (size_t)m->cfg.vocab * 4, hipMemcpyDeviceToHost, m->stream);
  const hipError_t es = hipStreamSynchronize(m->stream);
  MHIP(e);
  MHIP(es);
  m->host_pos += n;
  return NRQ_OK;
}

int nrq_model_kv_cache(nrq_model* m, void* k_host, void* v_host, size_t bytes) {
  if (!m) return mfail(NRQ_ERR_ARG, "nrq_model_kv_cache: null handle");
  const size_t kvb = (size_t)m->cfg.n_layers * m->cfg.ctx * m->kv_dim * 2;
  if (bytes != kvb) return mfail(NRQ_ERR_SHAPE, "nrq_model_kv_cache: size mismatch");
  MHIP(hipStreamSynchronize(m->stream));
  // the device cache is piece-major per (layer, KV head): [hd / 8][ctx][8]
  const int L = m->cfg.n_layers, ctx = m->cfg.ctx, nkv = m->cfg.n_kv_heads, hd = m->cfg.head_dim;
  std::vector<uint16_t> raw(kvb / 2);
  void* outs[2] = {k_host, v_host};
  const uint16_t* devs[2] = {m->kc, m->vc};
  for (int a = 0; a < 2; a++) {
    if (!outs[a]) continue;
    MHIP(hipMemcpy(raw.data(), devs[a], kvb, hipMemcpyDeviceToHost));
    uint16_t* o = (uint16_t*)outs[a];
    for (int l = 0; l < L; l++)
      for (int g = 0; g < nkv; g++) {
        const uint16_t* src = raw.data() + ((size_t)l * nkv + g) * hd * ctx;
        for (int j = 0; j < hd / 8; j++)
          for (int t = 0; t < ctx; t++)
            memcpy(o + ((size_t)l * ctx + t) * m->kv_dim + (size_t)g * hd + 8 * j, src + ((size_t)j * ctx + t) * 8, 16);
      }
  }
  return NRQ_OK;
}

int nrq_dev_rmsnorm(const float* x, const float* w, float* out, size_t rows, size_t n, float eps, void* stream) {
  if (rows == 0) return NRQ_OK;
  if (!x || !w || !out) return mfail(NRQ_ERR_ARG, "nrq_dev_rmsnorm: null pointer");
  if (n == 0 || n % 256 || n > (size_t)nrq::kNormMax) return mfail(NRQ_ERR_SHAPE, "nrq_dev_rmsnorm: n must be a multiple of 256, at most 8192");
  if (rows > (size_t)INT_MAX) return mfail(NRQ_ERR_SHAPE, "nrq_dev_rmsnorm: too many rows");
  // norm_kernel updates x in place only when it adds a residual; here it reads x
  hipLaunchKernelGGL(nrq::norm_kernel, dim3((unsigned)rows), dim3(nrq::kNormNT), 0, (hipStream_t)stream,
                     const_cast<float*>(x), nullptr, w, (int)n, eps, 1.0f, out, nullptr, nullptr);
  return hipGetLastError() == hipSuccess ? NRQ_OK : mfail(NRQ_ERR_DEVICE, "nrq_dev_rmsnorm: launch failed");
}

int nrq_dev_mathf(int fn, const float* x, float* y, size_t n, void* stream) {
  if (fn < 0 || fn > 2) return mfail(NRQ_ERR_ARG, "nrq_dev_mathf: unknown function");
  if (n == 0) return NRQ_OK;
  if (!x || !y) return mfail(NRQ_ERR_ARG, "nrq_dev_mathf: null pointer");
  hipLaunchKernelGGL(nrq::mathf_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, fn, x, y,
                     (long long)n);
  return hipGetLastError() == hipSuccess ? NRQ_OK : mfail(NRQ_ERR_DEVICE, "nrq_dev_mathf: launch failed");
}

int nrq_model_destroy(nrq_model* m) {
  if (!m) return NRQ_OK;
  if (m->stream) hipStreamSynchronize(m->stream);
  if (m->exec) hipGraphExecDestroy(m->exec);
  if (m->graph) hipGraphDestroy(m->graph);
  void* bufs[] = {m->freqs, m->rope_cs, m->kc, m->vc, m->x, m->x2, m->xb, m->q, m->k, m->v, m->attn, m->gate, m->up, m->xb2,
                  m->logits, m->xq, m->xq2, m->ctl, m->out_tokens, m->owned, m->bx, m->bxb, m->bxn, m->bq,
                  m->bk, m->bv, m->battn, m->bgate, m->bup, m->brope, m->bxq, m->bxq2, m->btok, m->rng, m->samp_part};
  for (void* p : bufs)
    if (p) hipFree(p);
  if (m->stream) hipStreamDestroy(m->stream);
  delete m;
  return NRQ_OK;
}

}  // extern "C"
