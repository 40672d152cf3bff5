// Batched prefill matmul on int8 MFMA, scalar f32 order, 16 x 16 tiles: the
// kernel for Q8_0 weights below 1024 rows (Q4_K / Q6_K and wider Q8_0 run the
// 32 x 32 tiles of nrq_mmt.hip):
//   y[t][r] = dot(W[r, :], xs[t])   for t < batch (the reference's MAX_BATCH is 64)
// bit-identical to per-token matvec, as the reference's matmul_q8 guarantees
// (crates/nr-tensor/src/kernels.rs:84-143), in the order of dot_q8_scalar
// (kernels.rs:72-82).
//
// Every block's integer sub-dot is one exact int32 output of
// v_mfma_i32_16x16x32_i8, taken for 16 tokens x 16 weight rows at once. The
// reference's per-block f32 steps then run per (token, row) element in its
// order.
//
// Tiling. A workgroup owns a 16-token x 16-row element tile. Its 4 waves split
// the row's blocks into 4 contiguous ranges and write each block's f32
// contribution to LDS; after a barrier, one lane per element adds the
// contributions in block order (the reference's `sumf +=` chain), in chunks
// of up to 32 blocks. MFMA orientation D[token][row]: lane l holds row
// r0 + l % 16 (per-row scales are lane-local) and tokens t0 + 4*(l / 16) + i.
// The A operand (activation) of lane l is token t0 + l % 16, k-group l / 16
// (8 bytes); the B operand (weights) is row r0 + l % 16, the same k-group.
//
// The workgroups of one row tile (one per 16-token tile) are numbered so that
// they land on the same XCD: its L2 serves the weights to all of them.
#include "nrq_device.h"
#include "nrq_launch.h"

namespace nrq {

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ i32x4 mfma16(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1) {
  const long a = (long)(((uint64_t)a1 << 32) | a0);
  const long b = (long)(((uint64_t)b1 << 32) | b0);
  const i32x4 z = {0, 0, 0, 0};
  return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, z, 0, 0, 0);
}

// Dwords [o, o+4n) of a byte array whose start is 2-byte aligned; reads
// whole aligned dwords and realigns.
template <int N>
__device__ __forceinline__ void load_even(const uint8_t* __restrict__ base, size_t o, uint32_t v[N]) {
  const uint32_t* p = (const uint32_t*)(base + (o & ~(size_t)3));
  const uint32_t sh = (uint32_t)(o & 3);
  uint32_t prev = p[0];
#pragma unroll
  for (int t = 0; t < N; t++) {
    const uint32_t next = p[t + 1];
    v[t] = __builtin_amdgcn_alignbyte(next, prev, sh);
    prev = next;
  }
}

// f32 contribution of block b for this lane's 4 elements (tokens t0 + 4g + i,
// row r), written exactly as the reference's scalar kernel forms it.
template <int FMT>
__device__ __forceinline__ void block_contrib(const uint8_t* __restrict__ W, const uint8_t* __restrict__ X, int rc,
                                              int bpr, int b, int t0, int tac, bool a_live, int batch, int g,
                                              float out[4]);

template <>
__device__ __forceinline__ void block_contrib<kQ8_0>(const uint8_t* __restrict__ W, const uint8_t* __restrict__ X,
                                                     int rc, int bpr, int b, int t0, int tac, bool a_live, int batch,
                                                     int g, float out[4]) {
  const size_t wo = ((size_t)rc * bpr + b) * kQ8_0Bytes;
  uint32_t wq[2], xq[2];
  load_even<2>(W, wo + 2 + 8 * g, wq);
  load_even<2>(X, ((size_t)tac * bpr + b) * kQ8_0Bytes + 2 + 8 * g, xq);
  if (!a_live) xq[0] = xq[1] = 0u;
  const i32x4 c = mfma16(xq[0], xq[1], wq[0], wq[1]);  // kernels.rs:75-78
  const float dw = f16_bits_to_f32(*(const uint16_t*)(W + wo));
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int t = min(t0 + 4 * g + i, batch - 1);
    const float dx = f16_bits_to_f32(*(const uint16_t*)(X + ((size_t)t * bpr + b) * kQ8_0Bytes));
    const float t1 = (float)c[i] * dw;  // kernels.rs:79: (f32(acc) * dw) * dx
    out[i] = t1 * dx;
  }
}

}  // namespace

constexpr int kMmqChunk = 32;  // blocks whose contributions one LDS pass holds (32 KiB)

template <int FMT>
__global__ __launch_bounds__(256) void mmq_kernel(const uint8_t* __restrict__ W, const uint8_t* __restrict__ X,
                                                  float* __restrict__ Y, int rows, int bpr, int batch, int ntt,
                                                  int nrt) {
  __shared__ float cont[kMmqChunk * 256];  // cont[b][i * 64 + lane]
  // XCD-aware numbering: workgroups i, i+8, i+16, ... share an XCD; the ntt
  // token tiles of one row tile take consecutive slots of one XCD.
  const int wg = blockIdx.x;
  const int xcd = wg & 7, slot = wg >> 3;
  const int tt = slot % ntt;
  const int rt = (slot / ntt) * 8 + xcd;
  if (rt >= nrt) return;  // padding workgroup (uniform: before any barrier)
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int n = lane & 15, g = lane >> 4;
  const int r = rt * 16 + n;
  const int rc = r < rows ? r : rows - 1;  // rows past the end: load row rows-1, store nothing
  const int t0 = tt * 16;
  const int ta = t0 + n;  // A-operand token of this lane
  const bool a_live = ta < batch;
  const int tac = a_live ? ta : batch - 1;
  // chain lane: element e = tid holds token t0 + 4*(e/16 % 4) + e/64 ... as laid out below
  const int ce_i = tid >> 6, ce_lane = tid & 63;
  const int ce_row = rt * 16 + (ce_lane & 15);
  const int ce_tok = t0 + 4 * (ce_lane >> 4) + ce_i;
  float chain = 0.0f;

  for (int c0 = 0; c0 < bpr; c0 += kMmqChunk) {
    const int nb = min(kMmqChunk, bpr - c0);
    const int per = (nb + 3) >> 2;
    const int b_lo = wave * per, b_hi = min(nb, b_lo + per);
    for (int bi = b_lo; bi < b_hi; bi++) {
      float o[4];
      block_contrib<FMT>(W, X, rc, bpr, c0 + bi, t0, tac, a_live, batch, g, o);
#pragma unroll
      for (int i = 0; i < 4; i++) cont[bi * 256 + i * 64 + lane] = o[i];
    }
    __syncthreads();
    // the reference's `sumf += contribution` chain, block order
    for (int bi = 0; bi < nb; bi++) chain = chain + cont[bi * 256 + tid];
    __syncthreads();
  }
  if (ce_row < rows && ce_tok < batch) Y[(size_t)ce_tok * rows + ce_row] = chain;
}

int launch_mmq(int dtype, const MatmulLaunch& L) {
  if (L.rows <= 0 || L.bpr <= 0 || L.batch <= 0) return 0;
  const int nrt = (L.rows + 15) / 16, ntt = (L.batch + 15) / 16;
  const long nwg = (long)((nrt + 7) / 8) * 8 * ntt;
  if (nwg > 0x7fffffffL) return NRQ_LAUNCH_BAD_ARG;
  const dim3 grid((unsigned)nwg);
  hipStream_t st = (hipStream_t)L.stream;
  const uint8_t* w = (const uint8_t*)L.w;
  const uint8_t* x = (const uint8_t*)L.xs;
  if (mmt_fits(dtype, L)) return launch_mmt(dtype, L);  // every Q4_K / Q6_K shape
  if (dtype != kQ8_0) return NRQ_LAUNCH_BAD_ARG;
  hipLaunchKernelGGL(mmq_kernel<kQ8_0>, grid, dim3(256), 0, st, w, x, L.y, L.rows, L.bpr, L.batch, ntt, nrt);
  return hipGetLastError() == hipSuccess ? 0 : NRQ_LAUNCH_FAILED;
}

}  // namespace nrq
