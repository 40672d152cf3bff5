// Internal launch interface between the C ABI (nrq_api.hip) and the kernel
// files. Not installed; the public interface is include/nrq.h.
#pragma once

#include <stddef.h>
#include <stdint.h>

struct nrq_model;

namespace nrq {

enum {
  NRQ_LAUNCH_OK = 0,
  NRQ_LAUNCH_BAD_ARG = -1,
  NRQ_LAUNCH_TOO_WIDE = -2,  // row does not fit the kernel's LDS tile
  NRQ_LAUNCH_FAILED = -3,
};

struct MatvecLaunch {
  const void* w;  // device, 16-byte aligned, rows * bpr blocks
  const void* x;  // device activation blocks (Q8_0 or Q8_K), bpr blocks
  float* y;       // device, rows floats
  int rows;
  int bpr;
  int tile_rows;  // 0 = library choice, else rows per tile
  void* stream;   // hipStream_t
};

struct MatmulLaunch {
  const void* w;  // device, 16-byte aligned
  const void* xs; // device, batch * bpr activation blocks
  float* y;       // device, [batch][rows]
  int rows;
  int bpr;
  int batch;
  void* stream;
};

struct QuantLaunch {
  const float* src;  // device f32[n]
  void* dst;         // device blocks
  long long n;       // elements (multiple of the block size)
  void* stream;
  const float* up = nullptr;  // Q8_K only: quantize swiglu(src, up), written back over src
};

// Scalar order: the streaming kernel (nrq_wstream.hip); AVX2 order: the
// one-shot LDS tile kernel (nrq_matvec.hip).
int launch_matvec(int dtype, int order, const MatvecLaunch& L);
// Scalar-order decode, one lane per block, per-wave LDS streaming (nrq_wstream.hip).
int launch_wstream_scalar(int dtype, const MatvecLaunch& L);
// scalar-order matvecs of up to three matrices of one format sharing the
// activation x (bpr blocks per row), one launch
int launch_wstream_group(int dtype, const void* const* w, float* const* y, const int* rows, int n, const void* x,
                         int bpr, void* stream);
// Rmsnorm of x (after x += add when add != null; the sum is written to x_out)
// and its Q8_0 quantization, fused into one launch of up to three Q8_0 matvecs
// over that activation (nrq_wstream.hip). n = cols, a multiple of 256 up to
// 4096; returns NRQ_LAUNCH_TOO_WIDE when the shape is not supported.
struct NormMatvecLaunch {
  const float* x;
  const float* add;
  float* x_out;
  const float* norm_w;
  int n;
  float eps;
  float rscale = 1.0f;  // x + rscale * add
  int nmat;
  const void* w[3];
  float* y[3];
  int rows[3];
  // optional, for a gate|up pair: the Q8_0 blocks of swiglu(gate, up) are
  // written here (y is then not written); rows a multiple of 32
  uint8_t* swiglu_q8;
  // optional, K-quant weights: the activation's Q8_K blocks are also stored here
  uint8_t* xq_out;
  void* stream;
};
// Residual + rmsnorm + activation quantization fused into the matvec prologue,
// for 1-3 matrices of one dtype (Q8_0, Q4_K or Q6_K)
int launch_norm_matvec(int dtype, const NormMatvecLaunch& L);
// An f32 activation quantized to Q8_K in the prologue of one Q4_K / Q6_K matvec
int launch_quant_matvec(int dtype, const float* x, int n, const void* w, float* y, int rows, void* stream);
int launch_matmul(int dtype, int order, const MatmulLaunch& L);
// Scalar-order batched matmul on int8 MFMA: the 32 x 32 tiles of nrq_mmt.hip,
// or for Q8_0 below 1024 rows the 16 x 16 tiles of nrq_mmq.hip.
int launch_mmq(int dtype, const MatmulLaunch& L);
// Prefill on 32-row x 32-token wave tiles (nrq_mmt.hip); mmt_fits: the kernel
// handles the format and shape.
bool mmt_fits(int dtype, const MatmulLaunch& L);
int launch_mmt(int dtype, const MatmulLaunch& L);
// Up to three matrices of one format and width sharing one activation (q|k|v,
// gate|up) in one launch of the same kernel, y[i] = [batch][rows[i]].
// NRQ_LAUNCH_BAD_ARG when the kernel does not take the group.
struct MatmulGroupLaunch {
  const void* w[3];
  float* y[3];
  int rows[3];
  int nmat;
  const void* xs;
  int bpr;
  int batch;
  void* stream;
};
int launch_mmt_group(int dtype, const MatmulGroupLaunch& G);
// Two such groups, of two different K-quant formats over one activation (q|k
// Q4_K and v Q6_K), in one launch; NRQ_LAUNCH_BAD_ARG when the kernel does not
// take the pair.
int launch_mmt_group2(int dt0, const MatmulGroupLaunch& G0, int dt1, const MatmulGroupLaunch& G1);
// AVX2-order batched matmul on int8 MFMA (nrq_mma.hip): 32-row x 32-token
// K-quant tiles, 8-row x 32-token Q8_0 tiles.
int launch_mma(int dtype, const MatmulLaunch& L);
int launch_quantize_q8_0(const QuantLaunch& L);
// y[0..n) = +0.0 (a kernel, not hipMemsetAsync, so it is safe under graph capture)
int launch_fill_zero(float* y, long long n, void* stream);
int launch_stream_read(const void* p, long long bytes, uint32_t* out, void* stream);
int launch_quantize_q8k(const QuantLaunch& L);
// Q4_K/Q6_K/Q8_0 per-(row, block) exact integer sums (test/diagnostic path).
int launch_block_sums(int dtype, const void* w, const void* x, int32_t* out, int rows, int bpr, void* stream);

// Sets the message nrq_last_error() returns on this thread (nrq_api.hip).
void set_last_error(const char* msg);
// The model frees `dev` (a hipMalloc'd buffer its tensors point into) when destroyed.
void model_adopt_buffer(nrq_model* m, void* dev);
// Looks up the current device's address of the sampler's fixed scratch
// (nrq_model.hip), so that nrq_dev_sample_noalloc needs no lookup later.
int sample_scratch_setup();

}  // namespace nrq
