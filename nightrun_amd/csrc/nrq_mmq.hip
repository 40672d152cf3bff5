// Batched prefill matmul on int8 MFMA, scalar f32 order, 16 x 16 tiles: the
// kernel for Q8_0 weights, and an alternate for Q4_K / Q6_K (whose default is
// the 32 x 32 tile kernel of nrq_mmt.hip):
//   y[t][r] = dot(W[r, :], xs[t])   for t < batch (the reference's MAX_BATCH is 64)
// bit-identical to per-token matvec, as the reference's matmul_q8 /
// kquant_matmul! guarantee (crates/nr-tensor/src/kernels.rs:84-143,
// crates/nr-tensor/src/kquant.rs:566-639), in the order of the scalar dots
// dot_q8_scalar (kernels.rs:72-82), dot_q4k_scalar (kquant.rs:192-218) and
// dot_q6k_scalar (kquant.rs:220-250).
//
// Every integer sub-dot the scalar kernels form (a Q8_0 block, a Q4_K 32-wide
// sub-block, a Q6_K 16-wide group) is one exact int32 output of
// v_mfma_i32_16x16x32_i8, taken for 16 tokens x 16 weight rows at once (a Q6_K
// group fills half of K; the other half is zero). The reference's per-block
// f32 steps then run per (token, row) element in its order.
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

// (q - 32) for four 6-bit quants q = lo4 | hi2 << 4 held one per byte, as int8:
// bits 4-5 become the two's-complement high part (hi2 - 2), sign-extended.
__device__ __forceinline__ uint32_t q6_minus_32(uint32_t q6) {
  const uint32_t v = q6 ^ 0x20202020u;
  const uint32_t s = v & 0x20202020u;
  return v | (s << 1) | (s << 2);
}

// f32 contribution of block b for this lane's 4 elements (tokens t0 + 4g + i,
// row r), written exactly as the reference's scalar kernel forms it.
// sum + f32(s) * f32(p) is evaluated as fmaf(f32(s), f32(p), sum): the product
// of the two exact integers is below 2^24, so it is exact and the fused and
// unfused forms round the same sum once.
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

template <>
__device__ __forceinline__ void block_contrib<kQ4K>(const uint8_t* __restrict__ W, const uint8_t* __restrict__ X,
                                                    int rc, int bpr, int b, int t0, int tac, bool a_live, int batch,
                                                    int g, float out[4]) {
  const uint8_t* wb = W + ((size_t)rc * bpr + b) * kQ4KBytes;
  const u32x4 h = *(const u32x4*)wb;  // d | dmin, scales[12]
  uint32_t q[8];                      // qs[32c + 8g .. +8) for c = 0..3
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const uint2 v = *(const uint2*)(wb + 16 + 32 * c + 8 * g);
    q[2 * c] = v.x;
    q[2 * c + 1] = v.y;
  }
  const uint32_t* xw = (const uint32_t*)(X + ((size_t)tac * bpr + b) * kQ8KBytes + 4);  // qs dwords
  uint32_t xv[16];                                                                       // x[32j + 8g .. +8)
#pragma unroll
  for (int j = 0; j < 8; j++) {
    xv[2 * j] = a_live ? xw[8 * j + 2 * g] : 0u;
    xv[2 * j + 1] = a_live ? xw[8 * j + 2 * g + 1] : 0u;
  }
  // kquant.rs:83-92
  const uint32_t s0 = h.y, s1 = h.z, s2 = h.w;
  const uint32_t scA = s0 & 0x3f3f3f3fu, mnA = s1 & 0x3f3f3f3fu;
  const uint32_t scB = (s2 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u);
  const uint32_t mnB = ((s2 >> 4) & 0x0f0f0f0fu) | ((s1 >> 2) & 0x30303030u);
  float sum_q[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const int c = j >> 1;
    const uint32_t b0 = (j & 1) ? (q[2 * c] >> 4) & 0x0f0f0f0fu : q[2 * c] & 0x0f0f0f0fu;
    const uint32_t b1 = (j & 1) ? (q[2 * c + 1] >> 4) & 0x0f0f0f0fu : q[2 * c + 1] & 0x0f0f0f0fu;
    const i32x4 sub = mfma16(xv[2 * j], xv[2 * j + 1], b0, b1);  // kquant.rs:200-208
    const float sc = (float)(((j < 4 ? scA : scB) >> (8 * (j & 3))) & 0xffu);
    // kquant.rs:207: sum_q += f32(sc) * f32(sub); |sc * sub| <= 63 * 61440 < 2^24
#pragma unroll
    for (int i = 0; i < 4; i++) sum_q[i] = fmaf(sc, (float)sub[i], sum_q[i]);
  }
  uint32_t mm[8];  // m_j in both i16 halves
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t a = (mnA >> (8 * j)) & 0xffu, bq = (mnB >> (8 * j)) & 0xffu;
    mm[j] = a | (a << 16);
    mm[j + 4] = bq | (bq << 16);
  }
  const float dw = f16_bits_to_f32(h.x & 0xffffu), dmw = f16_bits_to_f32(h.x >> 16);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int t = min(t0 + 4 * g + i, batch - 1);
    const uint8_t* xb = X + ((size_t)t * bpr + b) * kQ8KBytes;
    const float xd = *(const float*)xb;
    const uint32_t* bs = (const uint32_t*)(xb + 260);  // bsums[2j] | bsums[2j+1] << 16
    // sum_m = sum_j m_j * (bsums[2j] + bsums[2j+1])  (kquant.rs:209-213)
    int sum_m = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) sum_m = sdot2(mm[j], bs[j], sum_m);
    const float d_all = dw * xd, dmin_all = dmw * xd;
    const float a = d_all * sum_q[i];
    const float m = dmin_all * (float)sum_m;
    out[i] = a - m;  // kquant.rs:215
  }
}

template <>
__device__ __forceinline__ void block_contrib<kQ6K>(const uint8_t* __restrict__ W, const uint8_t* __restrict__ X,
                                                    int rc, int bpr, int b, int t0, int tac, bool a_live, int batch,
                                                    int g, float out[4]) {
  const size_t bo = ((size_t)rc * bpr + b) * kQ6KBytes;  // even
  const bool kl = g < 2;                                  // k-groups 2, 3 carry the zero half of K
  const int gg = kl ? g : 0;
  uint32_t S[4];
  load_even<4>(W, bo + 192, S);  // scales[16]
  uint32_t dbits;
  {
    const uint32_t* p = (const uint32_t*)(W + ((bo + 208) & ~(size_t)3));
    dbits = ((bo + 208) & 2) ? (p[0] >> 16) : (p[0] & 0xffffu);
  }
  const float dw = f16_bits_to_f32(dbits);
  const uint32_t* xw = (const uint32_t*)(X + ((size_t)tac * bpr + b) * kQ8KBytes + 4);
  float sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int hh = 0; hh < 2; hh++) {
    // this lane's 8 quants of each group: l = 16u + 8g + i of the half's planes
    uint32_t LA[2][2], LB[2][2], QH[2][2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
      load_even<2>(W, bo + 64 * hh + 16 * u + 8 * gg, LA[u]);        // ql[l]
      load_even<2>(W, bo + 64 * hh + 32 + 16 * u + 8 * gg, LB[u]);   // ql[l + 32]
      load_even<2>(W, bo + 128 + 32 * hh + 16 * u + 8 * gg, QH[u]);  // qh[l]
    }
#pragma unroll
    for (int pn = 0; pn < 4; pn++) {
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const int G = 8 * hh + 2 * pn + u;  // kquant.rs:232-242 group order
        uint32_t bq[2];
#pragma unroll
        for (int k = 0; k < 2; k++) {
          uint32_t q6[4];
          q6k_planes(LA[u][k], LB[u][k], QH[u][k], q6);
          bq[k] = kl ? q6_minus_32(q6[pn]) : 0u;
        }
        // activation elements 128h + 32pn + 16u + 8g + i
        const int xo = 32 * hh + 8 * pn + 4 * u + 2 * gg;
        const uint32_t a0 = (a_live && kl) ? xw[xo] : 0u;
        const uint32_t a1 = (a_live && kl) ? xw[xo + 1] : 0u;
        const i32x4 gs = mfma16(a0, a1, bq[0], bq[1]);
        const float sc = (float)(int)(int8_t)((S[G >> 2] >> (8 * (G & 3))) & 0xffu);
        // kquant.rs:244: sum += f32(sc) * f32(gs); |sc * gs| <= 128 * 65536 < 2^24
#pragma unroll
        for (int i = 0; i < 4; i++) sum[i] = fmaf(sc, (float)gs[i], sum[i]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int t = min(t0 + 4 * g + i, batch - 1);
    const float xd = *(const float*)(X + ((size_t)t * bpr + b) * kQ8KBytes);
    const float d_all = dw * xd;
    out[i] = d_all * sum[i];  // kquant.rs:246-247
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
  if (L.variant == 0 && mmt_fits(dtype, L)) return launch_mmt(dtype, L);
  if (dtype == kQ8_0)
    hipLaunchKernelGGL(mmq_kernel<kQ8_0>, grid, dim3(256), 0, st, w, x, L.y, L.rows, L.bpr, L.batch, ntt, nrt);
  else if (dtype == kQ4K)
    hipLaunchKernelGGL(mmq_kernel<kQ4K>, grid, dim3(256), 0, st, w, x, L.y, L.rows, L.bpr, L.batch, ntt, nrt);
  else if (dtype == kQ6K)
    hipLaunchKernelGGL(mmq_kernel<kQ6K>, grid, dim3(256), 0, st, w, x, L.y, L.rows, L.bpr, L.batch, ntt, nrt);
  else
    return NRQ_LAUNCH_BAD_ARG;
  return hipGetLastError() == hipSuccess ? 0 : NRQ_LAUNCH_FAILED;
}

}  // namespace nrq
