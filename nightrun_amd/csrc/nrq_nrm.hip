// .nrm v3 model files on one GPU.
//
//   * nrq_nrm_open: Model::parse (crates/nr-model/src/format.rs:260-406), host
//     C++, every bound checked without wrapping, the same ParseError variants.
//   * nrq_dev_crc32: the file's CRC-32 (crates/nr-model/src/crc32.rs:6-79) over
//     bytes already in HBM. Model::verify_data (format.rs:409-422) runs it on
//     the uploaded data section, so the host never makes a second pass over a
//     multi-GB model and the check covers the bytes the kernels will read.
//   * nrq_model_load_nrm: one upload of the 64-byte-aligned data section
//     (format.rs:376-378) and InferCtx::new's tensor binding and shape checks
//     (crates/nr-model/src/infer.rs:352-447) for the device decode.
//
// CRC-32 here is IEEE (reflected polynomial 0xEDB88320, preset and final
// inversion). Over GF(2) the register is linear in the message, which is what
// makes it parallel: with r(m) the register after m from a zero register,
//   r(a || b) = r(a) * x^(8|b|) mod P  xor  r(b),
// and a zero register stays zero across leading zero bytes. T_k[byte] below is
// r(byte followed by k zero bytes); "shift c by n bytes" is c * x^(8n) mod P,
// which is T_{n-1}[c0] ^ T_{n-2}[c1] ^ T_{n-3}[c2] ^ T_{n-4}[c3] for the bytes
// c0..c3 of c (n >= 4), or a carry-less multiply by a constant.
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/nrq.h"
#include "nrq_launch.h"

namespace nrq {
namespace {

constexpr uint32_t kCrcPoly = 0xEDB88320u;
constexpr int kCrcWaves = 4;          // waves per workgroup of the span kernel
constexpr int kCrcStripe = 2048;      // bytes a wave consumes per step: 64 lanes x 2 granules x 16 B
constexpr int kCrcTabs = 36;          // byte tables in LDS (9 KiB words, 36 KiB)
constexpr int kCrcMaxSpans = 4096;    // partial registers per call
constexpr int kCrcMinStripes = 16;    // a span is at least 32 KiB
constexpr int kCrcCombineNT = 256;    // threads of the combine kernel
// LDS table rows: 0..15 = T_0..T_15 (second granule of a lane, byte j -> T_{15-j}),
// 16..31 = T_1024..T_1039 (first granule, 1024 bytes earlier), 32..35 = T_2044..T_2047
// (the running register shifted by one stripe).
constexpr int kTabG1 = 0, kTabG0 = 16, kTabStripe = 32;

// a * b mod P with bit 31 the x^0 coefficient (reflected order).
__host__ __device__ inline uint32_t gf2_mulmod(uint32_t a, uint32_t b) {
  uint32_t p = 0;
#pragma unroll 8
  for (int i = 0; i < 32; i++) {
    p ^= ((a >> (31 - i)) & 1u) ? b : 0u;
    b = (b >> 1) ^ (kCrcPoly & (0u - (b & 1u)));
  }
  return p;
}

// x^(8n) mod P: the multiplier that shifts a register by n zero bytes.
uint32_t x_pow_8n(unsigned long long n) {
  uint32_t r = 0x80000000u, base = 0x00800000u;  // x^0, x^8
  while (n) {
    if (n & 1) r = gf2_mulmod(r, base);
    base = gf2_mulmod(base, base);
    n >>= 1;
  }
  return r;
}

struct CrcTables {
  uint32_t t0[256];                   // host slicing: T_0..T_7
  uint32_t slice[8][256];
  std::vector<uint32_t> dev;          // kCrcTabs x 256, the device layout
  CrcTables() : dev((size_t)kCrcTabs * 256) {
    for (uint32_t i = 0; i < 256; i++) {
      uint32_t c = i;
      for (int k = 0; k < 8; k++) c = (c >> 1) ^ (kCrcPoly & (0u - (c & 1u)));
      t0[i] = c;
    }
    std::vector<uint32_t> cur(t0, t0 + 256);
    auto keep = [&](int k) {
      if (k < 8) memcpy(slice[k], cur.data(), 1024);
      if (k < 16) memcpy(&dev[(size_t)(kTabG1 + k) * 256], cur.data(), 1024);
      if (k >= 1024 && k < 1040) memcpy(&dev[(size_t)(kTabG0 + k - 1024) * 256], cur.data(), 1024);
      if (k >= 2044 && k < 2048) memcpy(&dev[(size_t)(kTabStripe + k - 2044) * 256], cur.data(), 1024);
    };
    keep(0);
    for (int k = 1; k < 2048; k++) {
      for (uint32_t& v : cur) v = t0[v & 0xffu] ^ (v >> 8);  // one more zero byte
      keep(k);
    }
  }
};

const CrcTables& crc_tables() {
  static const CrcTables t;
  return t;
}

// Host CRC: eight bytes per step, each looked up in the table for its distance
// to the end of the step, the register folded into the first four.
uint32_t host_crc32(uint32_t crc, const uint8_t* p, size_t n) {
  const CrcTables& T = crc_tables();
  uint32_t c = ~crc;
  for (; n >= 8; p += 8, n -= 8) {
    uint32_t w;
    memcpy(&w, p, 4);
    w ^= c;
    c = T.slice[7][w & 0xffu] ^ T.slice[6][(w >> 8) & 0xffu] ^ T.slice[5][(w >> 16) & 0xffu] ^ T.slice[4][w >> 24] ^
        T.slice[3][p[4]] ^ T.slice[2][p[5]] ^ T.slice[1][p[6]] ^ T.slice[0][p[7]];
  }
  for (; n; n--, p++) c = T.t0[(c ^ *p) & 0xffu] ^ (c >> 8);
  return ~c;
}

// ---- device CRC ----------------------------------------------------------------------
//
// The body (the 16-byte-aligned middle of the buffer) is cut into spans, one
// per wave, each a whole number of 2 KiB stripes; the first span is padded in
// front with zero granules, which leave a zero register unchanged. Per stripe
// lane l reads granules l and 64 + l (two fully coalesced 1 KiB wave loads),
// so its register is r(g0, 1008 zero bytes, g1), and the lane keeps a running
// register across stripes (shift by a stripe, xor the stripe's value). Lanes
// then combine pairwise (shifts of 16, 32, ..., 512 bytes) into the span's
// register, which the wave shifts on to the end of the body (one multiply per
// set bit of the number of spans after it). The combine kernel xors the spans'
// registers and adds the unaligned head (with the incoming value) and tail.

struct CrcSpanArgs {
  const uint4* body;
  long long n16;       // real granules in the body
  long long pad16;     // zero granules in front of the first span
  int stripes;         // per span
  int n_spans;
  const uint32_t* tabs;
  uint32_t lane_mul[6];  // x^(8 * 16 * 2^k) mod P
  uint32_t span_mul[12];  // x^(8 * span * 2^k) mod P
  uint32_t* partial;
};

__device__ inline uint4 crc_granule(const CrcSpanArgs& A, long long vg) {
  const long long g = vg - A.pad16;
  uint4 v = A.body[g < 0 ? 0 : g];
  if (g < 0) v = make_uint4(0, 0, 0, 0);
  return v;
}

__device__ inline uint32_t crc_word(const uint32_t* t, int row_of_byte0, uint32_t w) {
  // bytes 0..3 of w use rows row_of_byte0, row_of_byte0 - 1, ...
  return t[(row_of_byte0) * 256 + (w & 0xffu)] ^ t[(row_of_byte0 - 1) * 256 + ((w >> 8) & 0xffu)] ^
         t[(row_of_byte0 - 2) * 256 + ((w >> 16) & 0xffu)] ^ t[(row_of_byte0 - 3) * 256 + (w >> 24)];
}

__global__ __launch_bounds__(64 * kCrcWaves) void crc_span_kernel(CrcSpanArgs A) {
  __shared__ uint32_t t[kCrcTabs * 256];
  for (int i = threadIdx.x; i < kCrcTabs * 256; i += blockDim.x) t[i] = A.tabs[i];
  __syncthreads();
  const int w = blockIdx.x * kCrcWaves + (threadIdx.x >> 6);
  if (w >= A.n_spans) return;
  const int lane = threadIdx.x & 63;
  const long long base = (long long)w * A.stripes * 128 + lane;
  uint32_t reg = 0;
  uint4 a0 = crc_granule(A, base), b0 = crc_granule(A, base + 64);
  const long long last = base + (long long)(A.stripes - 1) * 128;
  long long nxt = base + 128 < last ? base + 128 : last;
  uint4 a1 = crc_granule(A, nxt), b1 = crc_granule(A, nxt + 64);
  for (int s = 0; s < A.stripes; s++) {
    nxt = nxt + 128 < last ? nxt + 128 : last;  // two stripes ahead, clamped in bounds
    const uint4 a2 = crc_granule(A, nxt), b2 = crc_granule(A, nxt + 64);
    // second granule: byte j -> T_{15-j}; first granule: byte j -> T_{1039-j};
    // running register: byte j -> T_{2047-j}
    uint32_t acc = crc_word(t, kTabG1 + 15, b0.x) ^ crc_word(t, kTabG1 + 11, b0.y) ^ crc_word(t, kTabG1 + 7, b0.z) ^
                   crc_word(t, kTabG1 + 3, b0.w);
    acc ^= crc_word(t, kTabG0 + 15, a0.x) ^ crc_word(t, kTabG0 + 11, a0.y) ^ crc_word(t, kTabG0 + 7, a0.z) ^
           crc_word(t, kTabG0 + 3, a0.w);
    reg = acc ^ crc_word(t, kTabStripe + 3, reg);
    a0 = a1;
    b0 = b1;
    a1 = a2;
    b1 = b2;
  }
  // lane l's register ends 16 * (63 - l) bytes before the span's end
#pragma unroll
  for (int k = 0; k < 6; k++) {
    const uint32_t other = (uint32_t)__shfl_xor((int)reg, 1 << k);
    const bool right = (lane >> k) & 1;
    reg = right ? gf2_mulmod(other, A.lane_mul[k]) ^ reg : gf2_mulmod(reg, A.lane_mul[k]) ^ other;
  }
  // spans after this one (fewer than 2^12); the branch is uniform in the wave
  const int after = A.n_spans - 1 - w;
#pragma unroll 1
  for (int k = 0; k < 12; k++)
    if ((after >> k) & 1) reg = gf2_mulmod(reg, A.span_mul[k]);
  if (lane == 0) A.partial[w] = reg;
}

struct CrcCombineArgs {
  const uint32_t* partial;  // span registers, already shifted to the end of the body
  int n_spans;
  const uint8_t* head;      // unaligned leading bytes
  int n_head;
  const uint8_t* tail;      // trailing bytes after the last granule
  int n_tail;
  uint32_t body_mul;        // x^(8 * body bytes)
  uint32_t crc_in;
  const uint32_t* t0;       // T_0
  uint32_t* out;
};

__global__ __launch_bounds__(kCrcCombineNT) void crc_combine_kernel(CrcCombineArgs A) {
  __shared__ uint32_t v[kCrcCombineNT / 64];
  const int tid = threadIdx.x;
  uint32_t r = 0;
  for (int i = tid; i < A.n_spans; i += kCrcCombineNT) r ^= A.partial[i];
#pragma unroll
  for (int k = 1; k < 64; k <<= 1) r ^= (uint32_t)__shfl_xor((int)r, k);
  if ((tid & 63) == 0) v[tid >> 6] = r;
  __syncthreads();
  if (tid == 0) {
    uint32_t body = 0;
    for (int i = 0; i < kCrcCombineNT / 64; i++) body ^= v[i];
    uint32_t s = ~A.crc_in;
    for (int i = 0; i < A.n_head; i++) s = A.t0[(s ^ A.head[i]) & 0xffu] ^ (s >> 8);
    s = gf2_mulmod(s, A.body_mul) ^ body;
    for (int i = 0; i < A.n_tail; i++) s = A.t0[(s ^ A.tail[i]) & 0xffu] ^ (s >> 8);
    *A.out = ~s;
  }
}

// Per-device tables and partial registers, made at the first call on a device.
struct CrcDev {
  int device = -1;
  uint32_t* tabs = nullptr;
  uint32_t* partial = nullptr;
};
std::mutex g_crc_mu;
std::vector<CrcDev> g_crc_dev;

int crc_dev_state(CrcDev** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return NRQ_ERR_DEVICE;
  std::lock_guard<std::mutex> lk(g_crc_mu);
  for (CrcDev& d : g_crc_dev)
    if (d.device == dev) {
      *out = &d;
      return NRQ_OK;
    }
  CrcDev d;
  d.device = dev;
  const size_t tab_bytes = (size_t)kCrcTabs * 256 * 4;
  void* p = nullptr;
  if (hipMalloc(&p, tab_bytes + (size_t)kCrcMaxSpans * 4) != hipSuccess) return NRQ_ERR_DEVICE;
  if (hipMemcpy(p, crc_tables().dev.data(), tab_bytes, hipMemcpyHostToDevice) != hipSuccess) {
    hipFree(p);
    return NRQ_ERR_DEVICE;
  }
  d.tabs = (uint32_t*)p;
  d.partial = (uint32_t*)((uint8_t*)p + tab_bytes);
  g_crc_dev.reserve(16);
  g_crc_dev.push_back(d);
  *out = &g_crc_dev.back();
  return NRQ_OK;
}

int dev_crc32(const void* data, size_t n, uint32_t crc_in, uint32_t* out, hipStream_t stream) {
  CrcDev* D = nullptr;
  if (crc_dev_state(&D)) {
    set_last_error("nrq_dev_crc32: could not set up the device tables");
    return NRQ_ERR_DEVICE;
  }
  const uintptr_t addr = (uintptr_t)data;
  const size_t head = std::min<size_t>((16 - (addr & 15)) & 15, n);
  const size_t n16 = (n - head) / 16;
  const size_t tail = n - head - 16 * n16;
  CrcCombineArgs C{};
  C.n_spans = 0;
  if (n16) {
    const unsigned long long stripes_total = (n16 + 127) / 128;
    unsigned long long sps = (stripes_total + kCrcMaxSpans - 1) / kCrcMaxSpans;
    if (sps < kCrcMinStripes) sps = kCrcMinStripes;
    if (sps > (1ull << 30)) {
      set_last_error("nrq_dev_crc32: buffer too large");
      return NRQ_ERR_ARG;
    }
    const int n_spans = (int)((stripes_total + sps - 1) / sps);
    CrcSpanArgs A{};
    A.body = (const uint4*)((const uint8_t*)data + head);
    A.n16 = (long long)n16;
    A.pad16 = (long long)(n_spans * sps * 128 - n16);
    A.stripes = (int)sps;
    A.n_spans = n_spans;
    A.tabs = D->tabs;
    for (int k = 0; k < 6; k++) A.lane_mul[k] = x_pow_8n(16ull << k);
    for (int k = 0; k < 12; k++) A.span_mul[k] = x_pow_8n(sps * kCrcStripe << k);
    A.partial = D->partial;
    hipLaunchKernelGGL(crc_span_kernel, dim3((n_spans + kCrcWaves - 1) / kCrcWaves), dim3(64 * kCrcWaves), 0, stream,
                       A);
    if (hipGetLastError() != hipSuccess) {
      set_last_error("nrq_dev_crc32: span kernel launch failed");
      return NRQ_ERR_DEVICE;
    }
    C.n_spans = n_spans;
  }
  C.partial = D->partial;
  C.head = (const uint8_t*)data;
  C.n_head = (int)head;
  C.tail = (const uint8_t*)data + head + 16 * n16;
  C.n_tail = (int)tail;
  C.body_mul = x_pow_8n(16ull * n16);
  C.crc_in = crc_in;
  C.t0 = D->tabs + kTabG1 * 256;
  C.out = out;
  hipLaunchKernelGGL(crc_combine_kernel, dim3(1), dim3(kCrcCombineNT), 0, stream, C);
  if (hipGetLastError() != hipSuccess) {
    set_last_error("nrq_dev_crc32: combine kernel launch failed");
    return NRQ_ERR_DEVICE;
  }
  return NRQ_OK;
}

// ---- parser ---------------------------------------------------------------------------

constexpr size_t kHeader = 192, kEntry = 32, kAlign = 64, kNameLen = 48;

uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | p[1] << 8); }
uint32_t rd32(const uint8_t* p) {
  uint32_t v;
  memcpy(&v, p, 4);
  return v;
}
uint64_t rd64(const uint8_t* p) {
  uint64_t v;
  memcpy(&v, p, 8);
  return v;
}
float rdf(const uint8_t* p) {
  float v;
  memcpy(&v, p, 4);
  return v;
}

int perr(int code, const std::string& msg) {
  set_last_error(msg.c_str());
  return code;
}

const char* kind_name(int kind) {  // format.rs:444-465
  switch (kind) {
    case 1: return "token_embd";
    case 2: return "output_norm";
    case 3: return "output";
    case 4: return "rope_freqs";
    case 10: return "attn_norm";
    case 11: return "attn_q";
    case 12: return "attn_k";
    case 13: return "attn_v";
    case 14: return "attn_output";
    case 15: return "ffn_norm";
    case 16: return "ffn_gate";
    case 17: return "ffn_up";
    case 18: return "ffn_down";
    case 19: return "attn_q_norm";
    case 20: return "attn_k_norm";
    default: return "unknown";
  }
}

// TensorDtype::byte_size (format.rs:107-123): false where the Rust returns None.
bool byte_size(uint32_t dtype, unsigned long long n, unsigned long long* out) {
  unsigned long long per, qk;
  switch (dtype) {
    case NRQ_F32: per = 4, qk = 1; break;
    case NRQ_Q8_0: per = 34, qk = 32; break;
    case NRQ_Q4_K: per = 144, qk = 256; break;
    default: per = 210, qk = 256; break;
  }
  if (n % qk) return false;
  return !__builtin_mul_overflow(n / qk, per, out);
}

}  // namespace
}  // namespace nrq

struct nrq_nrm {
  const uint8_t* blob = nullptr;
  size_t len = 0;
  nrq_nrm_meta meta{};
  std::vector<nrq_nrm_tensor_info> entries;
};

namespace {

using namespace nrq;

int parse(const uint8_t* b, size_t len, nrq_nrm* f) {
  if (len < kHeader) return perr(NRQ_ERR_NRM_TOO_SHORT, "TooShort");
  if (memcmp(b, "NRUN", 4) != 0) return perr(NRQ_ERR_NRM_BAD_MAGIC, "BadMagic");
  const uint32_t version = rd32(b + 4);
  if (version != 3) return perr(NRQ_ERR_NRM_BAD_VERSION, "BadVersion(" + std::to_string(version) + ")");
  nrq_nrm_meta& m = f->meta;
  m.arch = rd32(b + 8);
  if (m.arch < NRQ_ARCH_LLAMA3 || m.arch > NRQ_ARCH_GRANITE) return perr(NRQ_ERR_NRM_BAD_TABLE, "BadTable");
  uint32_t* dims[] = {&m.dim, &m.n_layers, &m.n_heads, &m.n_kv_heads, &m.head_dim, &m.ffn_dim, &m.vocab, &m.ctx_train};
  for (int i = 0; i < 8; i++) *dims[i] = rd32(b + 12 + 4 * i);
  float* fa[] = {&m.rope_theta, &m.norm_eps, &m.rope_factor, &m.rope_low, &m.rope_high, &m.rope_orig_ctx};
  for (int i = 0; i < 6; i++) *fa[i] = rdf(b + 44 + 4 * i);
  m.flags = rd32(b + 68);
  float* fb[] = {&m.embed_scale, &m.attn_scale, &m.residual_scale, &m.logit_scale};
  for (int i = 0; i < 4; i++) *fb[i] = rdf(b + 72 + 4 * i);
  memcpy(m.name, b + 88, kNameLen);
  m.tok_off = rd64(b + 136);
  m.tok_size = rd64(b + 144);
  m.table_off = rd64(b + 152);
  m.tensor_count = rd32(b + 160);
  m.data_off = rd64(b + 168);
  m.data_size = rd64(b + 176);
  m.data_crc = rd32(b + 184);
  m.meta_crc = rd32(b + 188);
  // format.rs:316-327: NaN, inf and non-positive scales are rejected
  if (!std::isfinite(m.embed_scale) || !std::isfinite(m.attn_scale) || m.attn_scale < 0.0f ||
      !std::isfinite(m.residual_scale) || m.residual_scale <= 0.0f || !std::isfinite(m.logit_scale) ||
      m.logit_scale <= 0.0f)
    return perr(NRQ_ERR_NRM_BAD_TABLE, "BadTable");
  // format.rs:329-343: region ends without wrapping
  const unsigned long long table_len = (unsigned long long)m.tensor_count * kEntry;  // < 2^37
  unsigned long long table_end, data_end, tok_end;
  if (__builtin_add_overflow(m.table_off, table_len, &table_end) ||
      __builtin_add_overflow(m.data_off, m.data_size, &data_end) ||
      __builtin_add_overflow(m.tok_off, m.tok_size, &tok_end))
    return perr(NRQ_ERR_NRM_TOO_SHORT, "TooShort");
  if (len < table_end || len < data_end || len < tok_end) return perr(NRQ_ERR_NRM_TOO_SHORT, "TooShort");
  // format.rs:345-357: header with the two CRC fields hashed as zeros, then the
  // tokenizer blob, then the tensor table
  static const uint8_t zeros[8] = {0};
  uint32_t c = host_crc32(0, b, kHeader - 8);
  c = host_crc32(c, zeros, 8);
  c = host_crc32(c, b + m.tok_off, m.tok_size);
  c = host_crc32(c, b + m.table_off, table_len);
  if (c != m.meta_crc) {
    char msg[96];
    snprintf(msg, sizeof msg, "MetaCrc { expect: %u, got: %u }", m.meta_crc, c);
    return perr(NRQ_ERR_NRM_META_CRC, msg);
  }
  // format.rs:359-397: entries
  f->entries.clear();
  f->entries.reserve(m.tensor_count);
  for (uint32_t i = 0; i < m.tensor_count; i++) {
    const uint8_t* e = b + m.table_off + (size_t)i * kEntry;
    nrq_nrm_tensor_info t{};
    t.kind = rd16(e);
    t.layer = rd16(e + 2);
    t.dtype = rd16(e + 4);
    if (t.dtype > NRQ_Q6_K) return perr(NRQ_ERR_NRM_BAD_TABLE, "BadTable");
    t.offset = rd64(e + 8);
    t.size = rd64(e + 16);
    t.rows = rd32(e + 24);
    t.cols = rd32(e + 28);
    unsigned long long end, bytes;
    if (__builtin_add_overflow(t.offset, t.size, &end) || end > m.data_size)
      return perr(NRQ_ERR_NRM_BAD_TABLE, "BadTable");
    if (t.offset % kAlign) return perr(NRQ_ERR_NRM_BAD_TABLE, "BadTable");
    const unsigned long long n = (unsigned long long)t.rows * t.cols;  // u32 x u32 fits u64
    if (!byte_size(t.dtype, n, &bytes) || bytes != t.size) return perr(NRQ_ERR_NRM_BAD_TABLE, "BadTable");
    f->entries.push_back(t);
  }
  return NRQ_OK;
}

const nrq_nrm_tensor_info* find(const nrq_nrm* f, int kind, int layer) {
  for (const auto& e : f->entries)
    if ((int)e.kind == kind && (int)e.layer == layer) return &e;
  return nullptr;
}

bool has_kind(const nrq_nrm* f, int kind) {
  for (const auto& e : f->entries)
    if ((int)e.kind == kind) return true;
  return false;
}

int missing(const char* what) { return perr(NRQ_ERR_NRM_MISSING_TENSOR, std::string("MissingTensor(") + what + ")"); }

// The rope table of InferCtx::new (infer.rs:433-447, rope.rs:14-34): the base
// spectrum theta^(-2i/head_dim), then either divided by the file's RopeFreqs
// factors or, without them, Llama-3 wavelength scaling when factor > 0.
void infer_freqs(const nrq_nrm_meta& m, const float* factors, size_t n_factors, std::vector<float>& out) {
  const int hd = (int)m.head_dim;
  out.assign(hd / 2, 0.0f);
  const float pi = 3.14159265358979323846f;
  for (int i = 0; i < hd / 2; i++) {
    const float exponent = -2.0f * (float)i / (float)hd;
    float freq = powf(m.rope_theta, exponent);
    if (!factors && m.rope_factor > 0.0f) {
      const float wavelen = 2.0f * pi / freq;
      const float low_wavelen = m.rope_orig_ctx / m.rope_low;
      const float high_wavelen = m.rope_orig_ctx / m.rope_high;
      if (wavelen > low_wavelen) {
        freq /= m.rope_factor;
      } else if (wavelen > high_wavelen) {
        const float smooth = (m.rope_orig_ctx / wavelen - m.rope_low) / (m.rope_high - m.rope_low);
        freq = (1.0f - smooth) * freq / m.rope_factor + smooth * freq;
      }
    }
    if (factors && (size_t)i < n_factors) freq /= factors[i];  // zip: only as many as the tensor holds
    out[i] = freq;
  }
}

}  // namespace

extern "C" {

uint32_t nrq_crc32(uint32_t crc, const void* data, size_t n) {
  if (!n) return crc;
  return nrq::host_crc32(crc, (const uint8_t*)data, n);
}

int nrq_dev_crc32(const void* data, size_t n, uint32_t crc, uint32_t* out, void* stream) {
  if (!out || (n && !data)) return perr(NRQ_ERR_ARG, "nrq_dev_crc32: null pointer");
  return nrq::dev_crc32(data, n, crc, out, (hipStream_t)stream);
}

int nrq_nrm_open(const void* blob, size_t len, nrq_nrm** out) {
  if (!out || (len && !blob)) return perr(NRQ_ERR_ARG, "nrq_nrm_open: null pointer");
  *out = nullptr;
  nrq_nrm* f = new nrq_nrm();
  f->blob = (const uint8_t*)blob;
  f->len = len;
  const int rc = parse(f->blob, len, f);
  if (rc) {
    delete f;
    return rc;
  }
  *out = f;
  return NRQ_OK;
}

int nrq_nrm_get_meta(const nrq_nrm* f, nrq_nrm_meta* out) {
  if (!f || !out) return perr(NRQ_ERR_ARG, "nrq_nrm_get_meta: null pointer");
  *out = f->meta;
  return NRQ_OK;
}

int nrq_nrm_entry(const nrq_nrm* f, uint32_t i, nrq_nrm_tensor_info* out) {
  if (!f || !out) return perr(NRQ_ERR_ARG, "nrq_nrm_entry: null pointer");
  if (i >= f->entries.size()) return perr(NRQ_ERR_ARG, "nrq_nrm_entry: index out of range");
  *out = f->entries[i];
  return NRQ_OK;
}

int nrq_nrm_tensor(const nrq_nrm* f, int kind, int layer, nrq_nrm_tensor_info* out) {
  if (!f || !out) return perr(NRQ_ERR_ARG, "nrq_nrm_tensor: null pointer");
  const nrq_nrm_tensor_info* e = find(f, kind, layer);
  if (!e) return missing(kind_name(kind));
  *out = *e;
  return NRQ_OK;
}

int nrq_nrm_has_tensor(const nrq_nrm* f, int kind) { return f && has_kind(f, kind) ? 1 : 0; }

int nrq_nrm_verify_data(const nrq_nrm* f, const void* dev_data, void* stream) {
  if (!f || (f->meta.data_size && !dev_data)) return perr(NRQ_ERR_ARG, "nrq_nrm_verify_data: null pointer");
  uint32_t* d_out = nullptr;
  if (hipMalloc(&d_out, 4) != hipSuccess) return perr(NRQ_ERR_DEVICE, "nrq_nrm_verify_data: hipMalloc");
  const hipStream_t s = (hipStream_t)stream;
  int rc = nrq::dev_crc32(dev_data, f->meta.data_size, 0, d_out, s);
  uint32_t got = 0;
  if (!rc && (hipMemcpyAsync(&got, d_out, 4, hipMemcpyDeviceToHost, s) != hipSuccess ||
              hipStreamSynchronize(s) != hipSuccess))
    rc = perr(NRQ_ERR_DEVICE, "nrq_nrm_verify_data: copy back failed");
  hipFree(d_out);
  if (rc) return rc;
  if (got != f->meta.data_crc) {
    char msg[96];
    snprintf(msg, sizeof msg, "DataCrc { expect: %u, got: %u }", f->meta.data_crc, got);
    return perr(NRQ_ERR_NRM_DATA_CRC, msg);
  }
  return NRQ_OK;
}

int nrq_nrm_close(nrq_nrm* f) {
  delete f;
  return NRQ_OK;
}

int nrq_model_load_nrm(const nrq_nrm* f, int ctx, int flags, nrq_model** out) {
  if (!f || !out) return perr(NRQ_ERR_ARG, "nrq_model_load_nrm: null pointer");
  *out = nullptr;
  const nrq_nrm_meta& M = f->meta;
  if (ctx <= 0) return perr(NRQ_ERR_ARG, "nrq_model_load_nrm: ctx must be positive");
  const bool qwen = M.arch == NRQ_ARCH_QWEN3;
  // widths in 64 bits, as the reference's usize Dims (infer.rs:60-73): a header whose
  // n_heads * head_dim wraps 32 bits then fails the shape checks below, as it does there
  const uint64_t dim = M.dim, att = (uint64_t)M.n_heads * M.head_dim, kvd = (uint64_t)M.n_kv_heads * M.head_dim,
                 ffn = M.ffn_dim;
  // InferCtx::new (infer.rs:378-431): every tensor present with its shape
  auto mat = [&](int kind, int layer, uint64_t rows, uint64_t cols, const nrq_nrm_tensor_info** e) {
    *e = find(f, kind, layer);
    if (!*e) return missing(kind_name(kind));
    if ((*e)->rows != rows || (*e)->cols != cols) return missing("bad matrix shape");
    if ((*e)->dtype == NRQ_F32) return perr(NRQ_ERR_NRM_BAD_TABLE, "BadTable");
    return NRQ_OK;
  };
  auto vecf = [&](int kind, int layer, uint64_t len, const nrq_nrm_tensor_info** e) {
    *e = find(f, kind, layer);
    if (!*e) return missing(kind_name(kind));
    if ((*e)->dtype != NRQ_F32)
      return perr(NRQ_ERR_SHAPE, "assertion `left == right` failed: TensorView::f32 of a quantized tensor");
    if ((unsigned long long)(*e)->rows * (*e)->cols != len) return missing("bad f32 tensor shape");
    return NRQ_OK;
  };
  struct Bind {
    int kind, layer, dtype;
    uint64_t offset;
  };
  std::vector<Bind> binds;
  const nrq_nrm_tensor_info* e = nullptr;
  int rc;
  if ((rc = mat(NRQ_TENSOR_TOK_EMBED, 0, M.vocab, dim, &e))) return rc;
  binds.push_back({NRQ_TENSOR_TOK_EMBED, 0, (int)e->dtype, e->offset});
  if (!qwen && has_kind(f, NRQ_TENSOR_ATTN_Q_NORM)) return missing("unexpected attn_q_norm for this arch");
  for (uint32_t l = 0; l < M.n_layers; l++) {
    if ((rc = vecf(NRQ_TENSOR_ATTN_NORM, l, dim, &e))) return rc;
    binds.push_back({NRQ_TENSOR_ATTN_NORM, (int)l, NRQ_F32, e->offset});
    if (qwen) {  // per-head q/k RMSNorm weights (infer.rs:393-402)
      for (int kind : {NRQ_TENSOR_ATTN_Q_NORM, NRQ_TENSOR_ATTN_K_NORM}) {
        if ((rc = vecf(kind, l, M.head_dim, &e))) return rc;
        binds.push_back({kind, (int)l, NRQ_F32, e->offset});
      }
    }
    const struct {
      int kind;
      uint64_t rows, cols;
    } ms[] = {{NRQ_TENSOR_ATTN_Q, att, dim}, {NRQ_TENSOR_ATTN_K, kvd, dim}, {NRQ_TENSOR_ATTN_V, kvd, dim},
              {NRQ_TENSOR_ATTN_O, dim, att}};
    for (const auto& s : ms) {
      if ((rc = mat(s.kind, l, s.rows, s.cols, &e))) return rc;
      binds.push_back({s.kind, (int)l, (int)e->dtype, e->offset});
    }
    if ((rc = vecf(NRQ_TENSOR_FFN_NORM, l, dim, &e))) return rc;
    binds.push_back({NRQ_TENSOR_FFN_NORM, (int)l, NRQ_F32, e->offset});
    const struct {
      int kind;
      uint64_t rows, cols;
    } fs[] = {{NRQ_TENSOR_FFN_GATE, ffn, dim}, {NRQ_TENSOR_FFN_UP, ffn, dim}, {NRQ_TENSOR_FFN_DOWN, dim, ffn}};
    for (const auto& s : fs) {
      if ((rc = mat(s.kind, l, s.rows, s.cols, &e))) return rc;
      binds.push_back({s.kind, (int)l, (int)e->dtype, e->offset});
    }
  }
  if ((rc = vecf(NRQ_TENSOR_OUTPUT_NORM, 0, dim, &e))) return rc;
  binds.push_back({NRQ_TENSOR_OUTPUT_NORM, 0, NRQ_F32, e->offset});
  if (!(M.flags & NRQ_NRM_FLAG_TIED_EMBEDDINGS)) {
    if ((rc = mat(NRQ_TENSOR_OUTPUT, 0, M.vocab, dim, &e))) return rc;
    binds.push_back({NRQ_TENSOR_OUTPUT, 0, (int)e->dtype, e->offset});
  }
  std::vector<float> freqs;
  if (has_kind(f, NRQ_TENSOR_ROPE_FREQS)) {
    const nrq_nrm_tensor_info* r = find(f, NRQ_TENSOR_ROPE_FREQS, 0);
    if (!r) return missing(kind_name(NRQ_TENSOR_ROPE_FREQS));
    if (r->dtype != NRQ_F32)
      return perr(NRQ_ERR_SHAPE, "assertion `left == right` failed: TensorView::f32 of a quantized tensor");
    std::vector<float> fac(r->size / 4);
    if (!fac.empty()) memcpy(fac.data(), f->blob + M.data_off + r->offset, r->size);
    infer_freqs(M, fac.data(), fac.size(), freqs);
  } else {
    infer_freqs(M, nullptr, 0, freqs);
  }

  // the device model indexes with int: every width must fit one
  const uint64_t widths[] = {dim, M.n_layers, M.n_heads, M.n_kv_heads, M.head_dim, ffn, M.vocab, att, kvd};
  for (uint64_t v : widths)
    if (v == 0 || v > (uint64_t)INT_MAX)
      return perr(NRQ_ERR_UNSUPPORTED, "nrq_model_load_nrm: a model width is zero or does not fit an int");
  nrq_model_config cfg{};
  cfg.dim = (int)dim;
  cfg.n_layers = (int)M.n_layers;
  cfg.n_heads = (int)M.n_heads;
  cfg.n_kv_heads = (int)M.n_kv_heads;
  cfg.head_dim = (int)M.head_dim;
  cfg.ffn_dim = (int)ffn;
  cfg.vocab = (int)M.vocab;
  cfg.ctx = ctx;
  cfg.norm_eps = M.norm_eps;
  cfg.rope_theta = M.rope_theta;
  nrq_model* m = nullptr;
  if ((rc = nrq_model_create(&cfg, &m))) return rc;
  // one upload of the data section (format.rs:376-378); hipMalloc's base is
  // 256-byte aligned and every tensor offset 64-byte aligned
  void* dev = nullptr;
  const size_t bytes = (size_t)M.data_size;
  if (hipMalloc(&dev, bytes ? bytes : 1) != hipSuccess) {
    nrq_model_destroy(m);
    return perr(NRQ_ERR_DEVICE, "nrq_model_load_nrm: hipMalloc of the data section failed");
  }
  nrq::model_adopt_buffer(m, dev);
  if (bytes && hipMemcpy(dev, f->blob + M.data_off, bytes, hipMemcpyHostToDevice) != hipSuccess) {
    nrq_model_destroy(m);
    return perr(NRQ_ERR_DEVICE, "nrq_model_load_nrm: upload of the data section failed");
  }
  if ((flags & NRQ_NRM_VERIFY_DATA) && (rc = nrq_nrm_verify_data(f, dev, nullptr))) {
    nrq_model_destroy(m);
    return rc;
  }
  for (const Bind& b : binds)
    if ((rc = nrq_model_set_tensor(m, b.kind, b.layer, b.dtype, (const uint8_t*)dev + b.offset))) {
      nrq_model_destroy(m);
      return rc;
    }
  if ((rc = nrq_model_set_rope_freqs(m, freqs.data(), (int)freqs.size()))) {
    nrq_model_destroy(m);
    return rc;
  }
  // the recipe (infer.rs:447-461): Neox pairs for Qwen3, the file's muP scalars
  if ((rc = nrq_model_set_recipe(m, qwen ? NRQ_ROPE_NEOX : NRQ_ROPE_ADJACENT, M.embed_scale, M.attn_scale,
                                 M.residual_scale, M.logit_scale))) {
    nrq_model_destroy(m);
    return rc;
  }
  *out = m;
  return NRQ_OK;
}

}  // extern "C"
