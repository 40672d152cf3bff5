// Activation quantizers on gfx950, bit-exact restatements of
//   q8::quantize        (crates/nr-tensor/src/q8.rs:27-44)      f32 -> Q8_0
//   kquant::quantize_q8k (crates/nr-tensor/src/kquant.rs:157-187) f32 -> Q8_K
// including the reference's softfloat f32 -> f16 (f16.rs:25-56), whose
// subnormal rounding is half-up rather than the hardware's nearest-even.
#include "nrq_device.h"
#include "nrq_launch.h"

namespace nrq {

// One wave per 64 consecutive Q8_0 blocks' worth of work: lane i of a
// 32-lane half handles element i of its block.
__global__ __launch_bounds__(256) void quantize_q8_0_kernel(const float* __restrict__ src, uint8_t* __restrict__ dst,
                                                            long long nblocks) {
  long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  long long b = gid >> 5;
  int i = (int)(gid & 31);
  if (b >= nblocks) return;
  float v = src[b * 32 + i];
  // amax over the block; max is order-independent, and fmaxf ignores NaN as
  // f32::max does.
  float amax = fabsf(v);
#pragma unroll
  for (int m = 16; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 32));
  amax = fmaxf(0.0f, amax);
  uint32_t d_bits = f32_to_f16_bits(amax / 127.0f);
  float d = f16_bits_to_f32(d_bits);
  float inv = d > 0.0f ? 1.0f / d : 0.0f;
  float x = v * inv;
  float r = x >= 0.0f ? x + 0.5f : x - 0.5f;
  int q = rust_f32_to_i32(r);
  q = q < -127 ? -127 : (q > 127 ? 127 : q);
  uint8_t* blk = dst + b * kQ8_0Bytes;
  blk[2 + i] = (uint8_t)(int8_t)q;
  if (i == 0) {
    blk[0] = (uint8_t)(d_bits & 0xff);
    blk[1] = (uint8_t)(d_bits >> 8);
  }
}

// One Q8_K block per 256-thread workgroup: thread t loads value t (and with
// `up` forms swiglu(src, up) = src / (1 + expf(-src)) * up, vec.rs:45-52,
// written back over src), then the first half-wave quantizes the block,
// lane r holding values 8r .. 8r+7 (q8k_half_lanes, nrq_device.h).
__global__ __launch_bounds__(256) void quantize_q8k_kernel(float* __restrict__ src, uint8_t* __restrict__ dst,
                                                           const float* __restrict__ up) {
  __shared__ __align__(16) float s_v[256];
  const long long b = blockIdx.x;
  const int t = threadIdx.x;
  float v = src[b * 256 + t];
  if (up) {
    v = v / (1.0f + dev_expf(-v)) * up[b * 256 + t];
    src[b * 256 + t] = v;
  }
  s_v[t] = v;
  __syncthreads();
  if (t < 32) {
    const float4 p0 = ((const float4*)s_v)[2 * t], p1 = ((const float4*)s_v)[2 * t + 1];
    const float o[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
    uint32_t lo, hi, d_bits;
    int ps;
    q8k_half_lanes(o, t, &lo, &hi, &ps, &d_bits);
    q8k_half_store(dst + b * kQ8KBytes, t, lo, hi, ps, d_bits);
  }
}

__global__ void fill_zero_kernel(float* __restrict__ y, long long n) {
  long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = 0.0f;
}

// A plain streaming read (16 bytes per lane, four loads in flight, grid-stride,
// xor-folded so that nothing is elided): the rate every matvec here is judged
// against on the same GPU. 1024 workgroups of 256 lanes.
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ p, long long n16,
                                                          uint32_t* __restrict__ out) {
  long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long stride = (long long)gridDim.x * 256;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u32x4 a = __builtin_nontemporal_load(p + i), b = __builtin_nontemporal_load(p + i + stride);
    const u32x4 c = __builtin_nontemporal_load(p + i + 2 * stride), d = __builtin_nontemporal_load(p + i + 3 * stride);
    acc ^= a ^ b ^ c ^ d;
  }
  for (; i < n16; i += stride) acc ^= p[i];
  const uint32_t v = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (v == 0x5eed5eedu) out[0] = v;  // practically never: keeps the loads live
}

int launch_stream_read(const void* p, long long bytes, uint32_t* out, void* stream) {
  if (bytes < 16) return 0;
  hipLaunchKernelGGL(stream_read_kernel, dim3(1024), dim3(256), 0, (hipStream_t)stream, (const u32x4*)p, bytes / 16,
                     out);
  return hipGetLastError() == hipSuccess ? 0 : NRQ_LAUNCH_FAILED;
}

int launch_fill_zero(float* y, long long n, void* stream) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, y, n);
  return hipGetLastError() == hipSuccess ? 0 : NRQ_LAUNCH_FAILED;
}

int launch_quantize_q8_0(const QuantLaunch& L) {
  if (L.n <= 0) return 0;
  if (L.n % 32) return NRQ_LAUNCH_BAD_ARG;
  long long nb = L.n / 32;
  long long threads = nb * 32;
  int grid = (int)((threads + 255) / 256);
  hipLaunchKernelGGL(quantize_q8_0_kernel, dim3(grid), dim3(256), 0, (hipStream_t)L.stream, L.src, (uint8_t*)L.dst,
                     nb);
  return hipGetLastError() == hipSuccess ? 0 : NRQ_LAUNCH_FAILED;
}

int launch_quantize_q8k(const QuantLaunch& L) {
  if (L.n <= 0) return 0;
  if (L.n % 256) return NRQ_LAUNCH_BAD_ARG;
  const long long nb = L.n / 256;
  hipLaunchKernelGGL(quantize_q8k_kernel, dim3((unsigned)nb), dim3(256), 0, (hipStream_t)L.stream,
                     const_cast<float*>(L.src), (uint8_t*)L.dst, L.up);
  return hipGetLastError() == hipSuccess ? 0 : NRQ_LAUNCH_FAILED;
}

}  // namespace nrq
