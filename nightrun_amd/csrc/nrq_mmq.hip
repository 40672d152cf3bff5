// Batched prefill matmul on int8 MFMA, scalar f32 order:
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

// ---- LDS-staged kernel: Q4_K / Q6_K weights against Q8_K activations ---------------------
//
// A wave owns a 16-token x 16-row element tile and a contiguous range of the
// row's blocks (split s of S). Per block it moves, with LDS DMA
// (global_load_lds, no VGPRs), the 16 tokens' Q8_K blocks and the 16 rows'
// weight blocks into one of two wave-private stages, so the next block is in
// flight while this one is computed; a wave waits only on its own loads.
//
// Per block, each integer sub-dot is one v_mfma_i32_16x16x32_i8 output:
//   Q4_K: sub-block j (32 quants) is one MFMA; sum_m is four v_dot2 of the
//         rows' mins against the tokens' bsum pair sums.
//   Q6_K: group G (16 quants) fills k-groups 0-1 with raw 6-bit quants; k-groups
//         2-3 carry the same activation bytes against -32, so the MFMA returns
//         sum((q - 32) * q8) exactly (kquant.rs:232-242).
// Then the reference's f32 steps run per element in its order. The block
// contributions of a split stay in registers; after all splits, the
// reference's `sumf +=` chain runs split by split in block order, each split
// continuing from the previous split's partial sum (handed over in LDS).
//
// Workgroup: 4 waves = T token tiles x S splits (T * S = 4), one 16-row tile.
// Stage layout (dwords). Every DMA moves 16 bytes per lane from a 16-byte
// aligned address; a Q8_K token block (292 B, 4-byte aligned) lands in a
// 19-piece window and starts s4 dwords in; a Q6_K block (210 B, 2-byte
// aligned) lands in a 14-piece window and starts `skew` bytes in.
constexpr int kMqAct = 0;       // [16 tokens][76]: 5 DMAs of 64 pieces (+64 pieces of clamped lanes)
constexpr int kMqScal = 1280;   // [5][16]: tokens' bsum pair sums P0..P3, then d
constexpr int kMqWt = 1360;     // Q4_K [16 rows][36], 3 DMAs | Q6_K [16 rows][56], 4 DMAs
constexpr int kMqActInst = 5;
constexpr int kMqMaxPer = 16;   // blocks per split held in registers when S > 1

template <int FMT>
struct MQ;
template <>
struct MQ<kQ4K> {
  static constexpr int WI = 3, WROW = 36, STAGE = kMqWt + 3 * 256;
  static constexpr int NI = kMqActInst + WI;
};
template <>
struct MQ<kQ6K> {
  static constexpr int WI = 4, WROW = 56, STAGE = kMqWt + 4 * 256;
  static constexpr int NI = kMqActInst + WI;
};

__device__ __forceinline__ void mq_dma16(const uint8_t* sbase, uint32_t voff, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" : : "s"(m0), "v"(voff), "s"(sbase) : "memory");
}
__device__ __forceinline__ void mq_dma16v(const void* g, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" : : "s"(m0), "v"(g) : "memory");
}
template <int N>
__device__ __forceinline__ void mq_wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
__device__ __forceinline__ void mq_wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0x7f | (0 << 8) | (3 << 14)); }
__device__ __forceinline__ uint32_t mq_lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)p;
}

// Contribution of the staged block to this lane's 4 elements (tokens 4g + i, row n).
// `A` is token n's Q8_K block in LDS.
__device__ __forceinline__ void mq_block_q4k(const uint32_t* st, const uint32_t* A, int n, int g, float c[4]) {
  {  // token n's bsum pair sums for sub-blocks 2g, 2g+1, and its d
    const uint32_t v0 = A[65 + 2 * g], v1 = A[66 + 2 * g];
    const int s0 = (int)(int16_t)(v0 & 0xffffu) + (int)(int16_t)(v0 >> 16);
    const int s1 = (int)(int16_t)(v1 & 0xffffu) + (int)(int16_t)(v1 >> 16);
    uint32_t* scal = (uint32_t*)st + kMqScal;
    scal[g * 16 + n] = ((uint32_t)s0 & 0xffffu) | ((uint32_t)s1 << 16);
    if (g == 0) scal[64 + n] = A[0];
  }
  const uint32_t* Wr = st + kMqWt + n * 36;
  const u32x4 h = *(const u32x4*)Wr;
  // kquant.rs:83-92, four scales or mins per word
  const uint32_t scA = h.y & 0x3f3f3f3fu, mnA = h.z & 0x3f3f3f3fu;
  const uint32_t scB = (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
  const uint32_t mnB = ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
  i32x4 sub[8];
#pragma unroll
  for (int cc = 0; cc < 4; cc++) {
    const uint2 q = *(const uint2*)(Wr + 4 + 8 * cc + 2 * g);
    const uint32_t lo0 = q.x & 0x0f0f0f0fu, lo1 = q.y & 0x0f0f0f0fu;
    const uint32_t hi0 = (q.x >> 4) & 0x0f0f0f0fu, hi1 = (q.y >> 4) & 0x0f0f0f0fu;
    const int a = 1 + 16 * cc + 2 * g;  // sub-block 2cc: q8 bytes 64cc + 8g ..
    sub[2 * cc] = mfma16(A[a], A[a + 1], lo0, lo1);
    sub[2 * cc + 1] = mfma16(A[a + 8], A[a + 9], hi0, hi1);
  }
  // kquant.rs:207: sum_q += f32(sc) * f32(sub) in j order (the product is exact)
  float sq[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const float sc = (float)(((j < 4 ? scA : scB) >> (8 * (j & 3))) & 0xffu);
#pragma unroll
    for (int i = 0; i < 4; i++) sq[i] = fmaf(sc, (float)sub[j][i], sq[i]);
  }
  const uint32_t* scal = st + kMqScal;
  const u32x4 P0 = *(const u32x4*)(scal + 4 * g), P1 = *(const u32x4*)(scal + 16 + 4 * g);
  const u32x4 P2 = *(const u32x4*)(scal + 32 + 4 * g), P3 = *(const u32x4*)(scal + 48 + 4 * g);
  const u32x4 XD = *(const u32x4*)(scal + 64 + 4 * g);
  const uint32_t M0 = __builtin_amdgcn_perm(0u, mnA, 0x0c010c00u), M1 = __builtin_amdgcn_perm(0u, mnA, 0x0c030c02u);
  const uint32_t M2 = __builtin_amdgcn_perm(0u, mnB, 0x0c010c00u), M3 = __builtin_amdgcn_perm(0u, mnB, 0x0c030c02u);
  const float dw = f16_bits_to_f32(h.x & 0xffffu), dmw = f16_bits_to_f32(h.x >> 16);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    // kquant.rs:209-215
    int sum_m = sdot2(M0, P0[i], 0);
    sum_m = sdot2(M1, P1[i], sum_m);
    sum_m = sdot2(M2, P2[i], sum_m);
    sum_m = sdot2(M3, P3[i], sum_m);
    const float xd = __uint_as_float(XD[i]);
    const float d_all = dw * xd, dmin_all = dmw * xd;
    const float a = d_all * sq[i];
    const float m = dmin_all * (float)sum_m;
    c[i] = a - m;
  }
}

// `Wr` is row n's window, the block starting `sh` (0 or 2) bytes into Wr[0].
__device__ __forceinline__ void mq_block_q6k(const uint32_t* st, const uint32_t* A, const uint32_t* Wr, uint32_t sh,
                                             int n, int g, float c[4]) {
  if (g == 0) ((uint32_t*)st)[kMqScal + 64 + n] = A[0];  // token n's d
  const int gh = g & 1;
  const bool zh = g >= 2;  // k-groups 2-3: the -32 half
  uint32_t S[4];
#pragma unroll
  for (int t = 0; t < 4; t++) S[t] = __builtin_amdgcn_alignbyte(Wr[49 + t], Wr[48 + t], sh);  // scales[16]
  const uint32_t dbits = sh ? (Wr[52] >> 16) : (Wr[52] & 0xffffu);
  float sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int hh = 0; hh < 2; hh++) {
    uint32_t q6[2][4][2];  // [u][plane][dword]: quants l = 16u + 8gh + 0..7 of the half's planes
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const int la = 16 * hh + 4 * u + 2 * gh, lb = la + 8, qb = 32 + 8 * hh + 4 * u + 2 * gh;
      const uint32_t a0 = __builtin_amdgcn_alignbyte(Wr[la + 1], Wr[la], sh);
      const uint32_t a1 = __builtin_amdgcn_alignbyte(Wr[la + 2], Wr[la + 1], sh);
      const uint32_t b0 = __builtin_amdgcn_alignbyte(Wr[lb + 1], Wr[lb], sh);
      const uint32_t b1 = __builtin_amdgcn_alignbyte(Wr[lb + 2], Wr[lb + 1], sh);
      const uint32_t h0 = __builtin_amdgcn_alignbyte(Wr[qb + 1], Wr[qb], sh);
      const uint32_t h1 = __builtin_amdgcn_alignbyte(Wr[qb + 2], Wr[qb + 1], sh);
      uint32_t p0[4], p1[4];
      q6k_planes(a0, b0, h0, p0);
      q6k_planes(a1, b1, h1, p1);
#pragma unroll
      for (int pn = 0; pn < 4; pn++) {
        q6[u][pn][0] = zh ? 0xe0e0e0e0u : p0[pn];
        q6[u][pn][1] = zh ? 0xe0e0e0e0u : p1[pn];
      }
    }
#pragma unroll
    for (int pn = 0; pn < 4; pn++) {
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const int G = 8 * hh + 2 * pn + u;  // kquant.rs:232-246 group order
        const int a = 1 + 32 * hh + 8 * pn + 4 * u + 2 * gh;  // q8 bytes 128hh + 32pn + 16u + 8gh ..
        const i32x4 gs = mfma16(A[a], A[a + 1], q6[u][pn][0], q6[u][pn][1]);
        const float sc = (float)(int)(int8_t)((S[G >> 2] >> (8 * (G & 3))) & 0xffu);
        // kquant.rs:244: sum += f32(sc) * f32(gs); |sc * gs| <= 128 * 65536, exact
#pragma unroll
        for (int i = 0; i < 4; i++) sum[i] = fmaf(sc, (float)gs[i], sum[i]);
      }
    }
  }
  const u32x4 XD = *(const u32x4*)(st + kMqScal + 64 + 4 * g);
  const float dw = f16_bits_to_f32(dbits);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float d_all = dw * __uint_as_float(XD[i]);
    c[i] = d_all * sum[i];  // kquant.rs:246-247
  }
}

template <int FMT, int S>
__global__ __launch_bounds__(256) void mmq_lds_kernel(const uint8_t* __restrict__ W, const uint8_t* __restrict__ X,
                                                      float* __restrict__ Y, int rows, int bpr, int batch, int ntg,
                                                      int nrt) {
  constexpr int T = 4 / S;
  constexpr int NI = MQ<FMT>::NI, WI = MQ<FMT>::WI, STAGE = MQ<FMT>::STAGE;
  constexpr int NPER = S == 1 ? 1 : kMqMaxPer;
  extern __shared__ __align__(16) uint32_t lds[];
  // XCD-aware numbering: the token groups of one row tile share an XCD (and its L2)
  const int wg = blockIdx.x;
  const int xcd = wg & 7, slot = wg >> 3;
  const int tg = slot % ntg;
  const int rt = (slot / ntg) * 8 + xcd;
  if (rt >= nrt) return;  // padding workgroup (uniform, before any barrier)
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int tw = wave % T, sp = wave / T;
  const int n = lane & 15, g = lane >> 4;
  const int t0 = (tg * T + tw) * 16, r0 = rt * 16;
  uint32_t* stages = lds + wave * 2 * STAGE;
  const int per = (bpr + S - 1) / S;
  const int b_lo = sp * per;
  const int nmine = max(0, min(per, bpr - b_lo));
  const uintptr_t xu = (uintptr_t)X;

  // Per-lane DMA sources, fixed over blocks (clamped rows / tokens load valid memory, store nothing):
  // piece p of the activation = 16-byte piece p % 19 of token p / 19's window.
  uint32_t aoff[kMqActInst], aq[kMqActInst];
#pragma unroll
  for (int k = 0; k < kMqActInst; k++) {
    const int p = min(64 * k + lane, 16 * 19 - 1);
    const int tt = p / 19;
    aq[k] = 16u * (uint32_t)(p - tt * 19);
    aoff[k] = (uint32_t)min(t0 + tt, batch - 1) * (uint32_t)bpr * (uint32_t)kQ8KBytes;
  }
  uint32_t woff[WI];  // Q4_K: byte offset of the piece at block 0; Q6_K: the row's first block index
  uint32_t wq[WI];
#pragma unroll
  for (int k = 0; k < WI; k++) {
    if constexpr (FMT == kQ4K) {
      const int pc = min(64 * k + lane, 16 * 9 - 1);
      const int rr = pc / 9;
      woff[k] = (uint32_t)min(r0 + rr, rows - 1) * (uint32_t)bpr * (uint32_t)kQ4KBytes + 16u * (uint32_t)(pc - rr * 9);
      wq[k] = 0;
    } else {
      const int pc = min(64 * k + lane, 16 * 14 - 1);
      const int rr = pc / 14;
      woff[k] = (uint32_t)min(r0 + rr, rows - 1) * (uint32_t)bpr;
      wq[k] = 16u * (uint32_t)(pc - rr * 14);
    }
  }
  const uint32_t tok_n = (uint32_t)min(t0 + n, batch - 1) * (uint32_t)bpr * (uint32_t)kQ8KBytes;
  const uint32_t mrow = (uint32_t)min(r0 + n, rows - 1) * (uint32_t)bpr;  // this lane's row, in blocks

  auto issue = [&](int b, int stg) {
    const uint32_t sb = mq_lds_addr(stages + stg * STAGE);
    const uint32_t xb = (uint32_t)b * (uint32_t)kQ8KBytes;
#pragma unroll
    for (int k = 0; k < kMqActInst; k++) {
      const uintptr_t src = ((xu + aoff[k] + xb) & ~(uintptr_t)15) + aq[k];
      mq_dma16v((const void*)src, sb + (uint32_t)(kMqAct + 256 * k) * 4u);
    }
    if constexpr (FMT == kQ4K) {
      const uint8_t* wb = W + (size_t)b * kQ4KBytes;
#pragma unroll
      for (int k = 0; k < WI; k++) mq_dma16(wb, woff[k], sb + (uint32_t)(kMqWt + 256 * k) * 4u);
    } else {
#pragma unroll
      for (int k = 0; k < WI; k++) {
        const uint32_t start = (woff[k] + (uint32_t)b) * (uint32_t)kQ6KBytes;
        mq_dma16(W, (start & ~15u) + wq[k], sb + (uint32_t)(kMqWt + 256 * k) * 4u);
      }
    }
  };

  float cb[NPER][4];
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (nmine > 0) issue(b_lo, 0);
  if (nmine > 1) issue(b_lo + 1, 1);
  auto step = [&](int k) {
    if (k + 1 < nmine) mq_wait_vm<NI>();
    else mq_wait_vm<0>();
    asm volatile("" ::: "memory");
    const uint32_t b = (uint32_t)(b_lo + k);
    const uint32_t* st = stages + (k & 1) * STAGE;
    const uint32_t* A = st + kMqAct + n * 76 + (((xu + tok_n + b * (uint32_t)kQ8KBytes) & 15) >> 2);
    float c[4];
    if constexpr (FMT == kQ4K) {
      mq_block_q4k(st, A, n, g, c);
    } else {
      const uint32_t skew = ((mrow + b) * (uint32_t)kQ6KBytes) & 15u;
      mq_block_q6k(st, A, st + kMqWt + n * 56 + (skew >> 2), skew & 3u, n, g, c);
    }
    if constexpr (S == 1) {
#pragma unroll
      for (int i = 0; i < 4; i++) acc[i] = acc[i] + c[i];  // the `sumf +=` chain, block order
    } else {
#pragma unroll
      for (int kk = 0; kk < NPER; kk++)
        if (kk == k) {
#pragma unroll
          for (int i = 0; i < 4; i++) cb[kk][i] = c[i];
        }
    }
    if (k + 2 < nmine) {
      mq_wait_lgkm0();  // this stage's LDS reads are done before the DMA refills it
      asm volatile("" ::: "memory");
      issue(b_lo + k + 2, k & 1);
    }
  };
  if constexpr (S == 1) {
    for (int k = 0; k < nmine; k++) step(k);
  } else {
#pragma unroll
    for (int k = 0; k < NPER; k++)
      if (k < nmine) step(k);
    // chain across splits, in block order: split s continues from split s - 1
    float* hand = (float*)(lds + 4 * 2 * STAGE) + tw * 256;
    for (int s = 0; s < S; s++) {
      if (sp == s) {
        if (s > 0) {
#pragma unroll
          for (int i = 0; i < 4; i++) acc[i] = hand[i * 64 + lane];
        }
#pragma unroll
        for (int kk = 0; kk < NPER; kk++)
          if (kk < nmine) {
#pragma unroll
            for (int i = 0; i < 4; i++) acc[i] = acc[i] + cb[kk][i];
          }
        if (s + 1 < S) {
#pragma unroll
          for (int i = 0; i < 4; i++) hand[i * 64 + lane] = acc[i];
        }
      }
      __syncthreads();
    }
  }
  if (sp == S - 1) {
    const int row = r0 + n;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int tok = t0 + 4 * g + i;
      if (row < rows && tok < batch) Y[(size_t)tok * rows + row] = acc[i];
    }
  }
}

// Token tiles per workgroup: the most that still gives >= 512 workgroups (two
// per CU), so short matrices split the blocks instead; a split holds at most
// kMqMaxPer blocks in registers.
template <int FMT>
static int launch_mmq_lds(const MatmulLaunch& L) {
  const int nrt = (L.rows + 15) / 16, ntt = (L.batch + 15) / 16;
  const long rt_pad = (long)((nrt + 7) / 8) * 8;
  int T = 0;
  const int cand[3] = {4, 2, 1};
  for (int c = 0; c < 3; c++) {
    const int t = cand[c], sp = 4 / t;
    if (t > 1 && t > ntt) continue;                             // more token tiles than tokens
    if (sp > 1 && (L.bpr + sp - 1) / sp > kMqMaxPer) continue;  // splits too long for registers
    T = t;
    if (rt_pad * ((ntt + t - 1) / t) >= 512) break;
  }
  if (T == 0) T = 4;  // few tokens and long rows: no split, idle token tiles
  const int S = 4 / T;
  const int ntg = (ntt + T - 1) / T;
  const long nwg = rt_pad * ntg;
  if (nwg > 0x7fffffffL) return NRQ_LAUNCH_BAD_ARG;
  const size_t lds = (size_t)4 * 2 * MQ<FMT>::STAGE * 4 + (S > 1 ? (size_t)T * 256 * 4 : 0);
  hipStream_t st = (hipStream_t)L.stream;
  const uint8_t* w = (const uint8_t*)L.w;
  const uint8_t* x = (const uint8_t*)L.xs;
  if (S == 1)
    hipLaunchKernelGGL((mmq_lds_kernel<FMT, 1>), dim3((unsigned)nwg), dim3(256), lds, st, w, x, L.y, L.rows, L.bpr,
                       L.batch, ntg, nrt);
  else if (S == 2)
    hipLaunchKernelGGL((mmq_lds_kernel<FMT, 2>), dim3((unsigned)nwg), dim3(256), lds, st, w, x, L.y, L.rows, L.bpr,
                       L.batch, ntg, nrt);
  else
    hipLaunchKernelGGL((mmq_lds_kernel<FMT, 4>), dim3((unsigned)nwg), dim3(256), lds, st, w, x, L.y, L.rows, L.bpr,
                       L.batch, ntg, nrt);
  return hipGetLastError() == hipSuccess ? 0 : NRQ_LAUNCH_FAILED;
}

// The LDS-staged kernel forms 32-bit byte offsets into W and X.
static bool mmq_lds_fits(int dtype, const MatmulLaunch& L) {
  const unsigned long long wb = (unsigned long long)L.rows * L.bpr * (dtype == kQ4K ? kQ4KBytes : kQ6KBytes);
  const unsigned long long xb = (unsigned long long)L.batch * L.bpr * kQ8KBytes;
  return wb + 256 < (1ull << 32) && xb + 256 < (1ull << 32);
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
  if (L.variant == 0 && (dtype == kQ4K || dtype == kQ6K) && mmq_lds_fits(dtype, L))
    return dtype == kQ4K ? launch_mmq_lds<kQ4K>(L) : launch_mmq_lds<kQ6K>(L);
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
