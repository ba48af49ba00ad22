// ss_hip.hip - the C-ABI of include/ss_hip.h over the gfx950 kernels.
//
// Replaces the reference's Metal backend (src/backends/metal_backend.{h,m})
// and the per-token CPU sweep of src/core/layer_scheduler.c:291-679. The
// whole token (embedding, every layer, output norm, LM head, argmax) is
// enqueued on one stream with no host synchronisation; by default it is
// captured once into a HIP graph and replayed per token, with the token and
// position read from device memory so that greedy decoding can run many
// tokens back to back without the host.

#include "ss_hip.h"

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <unordered_map>
#include <vector>

#include "ss_kernels.h"
#include "ss_sweep.h"

namespace {

constexpr int32_t kErrParams = -5;   // SS_ERROR_INVALID_PARAMS
constexpr int32_t kErrOom = -3;      // SS_ERROR_OUT_OF_MEMORY
constexpr int32_t kErrBackend = -7;  // SS_ERROR_BACKEND
constexpr int32_t kErrCancel = -6;   // SS_ERROR_CANCELLED

thread_local char g_err[512] = "";
// compute units of the device the last context was created on (sizes matvec grids)
int g_n_cu = 0;

int32_t fail(int32_t code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

#define HIP_TRY(expr)                                                                   \
  do {                                                                                  \
    hipError_t e_ = (expr);                                                             \
    if (e_ != hipSuccess)                                                               \
      return fail(kErrBackend, "%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_),   \
                  __FILE__, __LINE__);                                                  \
  } while (0)

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// GGUF bytes of a row of cols weights (gguf_loader.c:22-62 block sizes)
size_t gguf_row_bytes(int type, int64_t cols) {
  switch (type) {
    case SS_HIP_F32: return (size_t)cols * 4;
    case SS_HIP_F16: return (size_t)cols * 2;
    case SS_HIP_Q4_0: return (size_t)cols / 32 * 18;
    case SS_HIP_Q4_1: return (size_t)cols / 32 * 20;
    case SS_HIP_Q5_0: return (size_t)cols / 32 * 22;
    case SS_HIP_Q5_1: return (size_t)cols / 32 * 24;
    case SS_HIP_Q8_0: return (size_t)cols / 32 * 34;
    case SS_HIP_Q8_1: return (size_t)cols / 32 * 40;
    case SS_HIP_Q2_K: return (size_t)cols / 256 * 84;
    case SS_HIP_Q3_K: return (size_t)cols / 256 * 110;
    case SS_HIP_Q4_K: return (size_t)cols / 256 * 144;
    case SS_HIP_Q5_K: return (size_t)cols / 256 * 176;
    case SS_HIP_Q6_K: return (size_t)cols / 256 * 210;
    default: return 0;
  }
}

// every matrix type of the reference's dequantiser (quantize.c:389-442)
bool quant_type_ok(int type) { return gguf_row_bytes(type, 256) > 0; }
// the prompt products take every block format (Q5_0 is stored as Q8_0), not F16 / F32
bool product_type(int type) { return ssk::product_format(ssk::dev_type(type)); }
constexpr const char* kTypesSupported = "F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q8_1 and Q2_K..Q6_K";
// columns a row of this type must be a multiple of (whole blocks, or super-blocks)
int col_unit(int type) { return ssk::is_kq(type) ? 256 : 32; }

ssk::PackedMat view(const void* base, int type, int64_t rows, int cols) {
  return ssk::packed_view(base, type, rows, cols);
}

// Algorithmic HBM bytes of one matvec launch: packed weights (18 or 34 bytes
// per 32 weights) + x + y.
double matvec_bytes(int type, int64_t rows, int cols, int nmat) {
  return (double)nmat * rows * gguf_row_bytes(type, cols) + 4.0 * cols + 4.0 * rows;
}

}  // namespace

struct ss_hip_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  int n_cu = 0;
  // scratch for the single-op entry points
  void* staging = nullptr;
  size_t staging_bytes = 0;
  float2* am_part = nullptr;

  float* rope_row = nullptr;
  int rope_row_len = 0;
  float* att_o = nullptr;
  float* att_ml = nullptr;
  uint32_t* att_cnt = nullptr;
  float* g_ssq = nullptr;      // prompt products: sums of squares of x
  uint16_t* g_xs = nullptr;    // prompt products: x split into fp16 parts

  size_t att_o_floats = 0, att_ml_floats = 0, att_cnt_bytes = 0, g_ssq_bytes = 0, g_xs_bytes = 0;
  float* smp = nullptr;        // sampling: probabilities [n]
  size_t smp_bytes = 0;
  uint64_t* smp_io = nullptr;  // sampling: [0] index, [1] advanced state

  // device address of this device's copy of `scratch` (ss_hip_attention_noalloc)
  void* scratch = nullptr;

  // host-pointer plug (metal_backend.m:190-235 registry)
  std::unordered_map<const void*, void*> registry;
  float* plug_x = nullptr;
  float* plug_y = nullptr;
  size_t plug_x_n = 0, plug_y_n = 0;
  // an open batch (ss_hip_begin_batch): the calls' device inputs and
  // outputs, one pair per call, and the host arrays the outputs go to
  static constexpr int kBatchSlots = 16;   // metal_backend.m:182-185
  bool batch = false;
  int batch_n = 0;
  float* batch_out[kBatchSlots] = {};
  int32_t batch_rows[kBatchSlots] = {};
  float* batch_x[kBatchSlots] = {};
  float* batch_y[kBatchSlots] = {};
  size_t batch_x_n[kBatchSlots] = {}, batch_y_n[kBatchSlots] = {};
};

// Scratch of ss_hip_attention_noalloc: the split partials (o, then (m, l))
// and the per-KV-head arrival counters of one attention call. Each device
// holds its own copy for the life of the process; host code reaches it only
// through the address hipGetSymbolAddress gives (ss_hip_ctx::scratch), never
// through the name, which on the host is a stand-in, not a device address.
constexpr size_t kNoAllocScratchBytes = (size_t)12 << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

// zero n words (a kernel rather than hipMemsetAsync, so that a caller may
// capture the call in a HIP graph)
__global__ void k_zero_words(uint32_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

namespace {

int32_t ensure(ss_hip_ctx* c, void** p, size_t* have, size_t need, bool zero) {
  if (*have >= need && *p) return 0;
  if (*p) hipFree(*p);
  *p = nullptr;
  *have = 0;
  HIP_TRY(hipMalloc(p, need));
  if (zero) HIP_TRY(hipMemset(*p, 0, need));
  *have = need;
  (void)c;
  return 0;
}

hipStream_t pick(ss_hip_ctx* c, void* stream) {
  return stream ? static_cast<hipStream_t>(stream) : c->stream;
}

int32_t set_device(ss_hip_ctx* c) {
  HIP_TRY(hipSetDevice(c->device));
  return 0;
}

// Pack rows [row_off, row_off+rows) of a combined [total_rows x cols]
// matrix from host GGUF blocks, in chunks through the context's staging buffer.
int32_t pack_rows(ss_hip_ctx* c, void* dst, int64_t total_rows, int64_t row_off,
                  const void* src, int type, int64_t rows, int cols) {
  const int nb = cols / 32;
  const size_t row_bytes = gguf_row_bytes(type, cols);
  const size_t chunk_target = 64u << 20;
  int64_t chunk_rows = (int64_t)(chunk_target / row_bytes);
  if (chunk_rows < 1) chunk_rows = 1;
  if (chunk_rows > rows) chunk_rows = rows;
  int32_t rc = ensure(c, &c->staging, &c->staging_bytes, (size_t)chunk_rows * row_bytes, false);
  if (rc) return rc;
  ssk::PackedMat v = view(dst, type, total_rows, cols);
  for (int64_t r = 0; r < rows; r += chunk_rows) {
    const int64_t n = rows - r < chunk_rows ? rows - r : chunk_rows;
    HIP_TRY(hipMemcpyAsync(c->staging, static_cast<const uint8_t*>(src) + (size_t)r * row_bytes,
                           (size_t)n * row_bytes, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(ssk::launch_pack(type, static_cast<const uint8_t*>(c->staging), v, n * nb, nb, row_off + r,
                             c->stream));
  }
  HIP_TRY(hipStreamSynchronize(c->stream));
  return 0;
}

// (cos, sin) of tensor.c:250-254 for one position, rope_dim/2 pairs.
void rope_row(float* cs, int rope_dim, int pos, float theta) {
  for (int i = 0; i < rope_dim; i += 2) {
    const float freq = 1.0f / powf(theta, (float)i / (float)rope_dim);
    const float angle = (float)pos * freq;
    cs[i] = cosf(angle);
    cs[i + 1] = sinf(angle);
  }
}

// Splits per KV head: enough that a split of the longest context is one round
// of attention loads (one HBM latency per split), but no more than the
// workgroups of all KV heads that are resident at once (a second generation
// of workgroups would cost a whole split's latency again), at most kMaxSplits.
int attn_splits(int head_dim, int group, int max_seq, int kv_type, int n_kv_heads, int n_cu) {
  const int round = ssk::attn_round_positions(head_dim, group);
  int ns = (max_seq + round - 1) / round;
  // every split resident at once (a second generation of workgroups costs
  // a whole split again)
  const int per_cu = ssk::attn_resident_groups(head_dim, group, kv_type);
  if (per_cu > 0 && n_cu > 0 && n_kv_heads > 0) {
    const int cap = per_cu * n_cu / n_kv_heads;
    if (ns > cap) ns = cap;
  }
  if (group >= 4 && ns > ssk::kMergeSplits && n_kv_heads > 0 && n_cu > 0) {
    // heads on lanes, merged by the last split: one workgroup per compute
    // unit, splits of at least 16 positions (measured at the 8B and 70B
    // shapes against 16 to 128 splits per KV head: 32 splits of 8 KV heads
    // ran 13.9 and 11.9 us per call, every split resident at once (64
    // splits) 15.8 and 14.9)
    ns = (n_cu + n_kv_heads - 1) / n_kv_heads;
    const int lim = (max_seq + 15) / 16;
    if (ns > lim) ns = lim;
  }
  if (ns > ssk::kMaxSplits) ns = ssk::kMaxSplits;
  if (ns < 1) ns = 1;
  return ns;
}

}  // namespace

// ============================================================== context
extern "C" {

const char* ss_hip_last_error(void) { return g_err; }

int32_t ss_hip_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

int32_t ss_hip_device_name(int32_t device, char* buf, int32_t len) {
  hipDeviceProp_t p;
  HIP_TRY(hipGetDeviceProperties(&p, device));
  if (buf && len > 0) snprintf(buf, (size_t)len, "%s (%s, %d CUs)", p.name, p.gcnArchName,
                               p.multiProcessorCount);
  return 0;
}

int32_t ss_hip_device_info(int32_t device, int32_t* n_cu, uint64_t* hbm_bytes) {
  hipDeviceProp_t p;
  HIP_TRY(hipGetDeviceProperties(&p, device));
  if (n_cu) *n_cu = p.multiProcessorCount;
  if (hbm_bytes) *hbm_bytes = (uint64_t)p.totalGlobalMem;
  return 0;
}

ss_hip_ctx_t* ss_hip_init(int32_t device) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
    fail(kErrBackend, "no HIP device available");
    return nullptr;
  }
  if (device < 0 || device >= n) {
    fail(kErrParams, "device %d out of range (%d devices)", device, n);
    return nullptr;
  }
  hipDeviceProp_t p;
  if (hipSetDevice(device) != hipSuccess || hipGetDeviceProperties(&p, device) != hipSuccess) {
    fail(kErrBackend, "cannot select HIP device %d", device);
    return nullptr;
  }
  if (strncmp(p.gcnArchName, "gfx950", 6) != 0) {
    fail(kErrBackend, "device %d is %s; this build targets gfx950 only", device, p.gcnArchName);
    return nullptr;
  }
  auto* c = new ss_hip_ctx();
  c->device = device;
  c->n_cu = p.multiProcessorCount;
  g_n_cu = c->n_cu;
  if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess ||
      hipMalloc(&c->am_part, sizeof(float2) * ssk::kArgmaxMaxBlocks) != hipSuccess) {
    fail(kErrBackend, "HIP context set-up failed on device %d", device);
    ss_hip_free(c);
    return nullptr;
  }
  // this device's copy of the no-allocation scratch (device is current here)
  if (hipGetSymbolAddress(&c->scratch, HIP_SYMBOL(scratch)) != hipSuccess || !c->scratch) {
    fail(kErrBackend, "no address for the scratch array on device %d", device);
    ss_hip_free(c);
    return nullptr;
  }
  return c;
}

void ss_hip_free(ss_hip_ctx_t* c) {
  if (!c) return;
  hipSetDevice(c->device);
  if (c->stream) hipStreamSynchronize(c->stream);
  for (auto& kv : c->registry) hipFree(kv.second);
  void* bufs[] = {c->staging, c->am_part, c->rope_row, c->att_o, c->att_ml, c->att_cnt,
                  c->g_ssq, c->g_xs, c->plug_x, c->plug_y, c->smp, c->smp_io};
  for (void* b : bufs)
    if (b) hipFree(b);
  for (int i = 0; i < ss_hip_ctx::kBatchSlots; ++i) {
    if (c->batch_x[i]) hipFree(c->batch_x[i]);
    if (c->batch_y[i]) hipFree(c->batch_y[i]);
  }
  if (c->stream) hipStreamDestroy(c->stream);
  delete c;
}

void* ss_hip_stream(ss_hip_ctx_t* c) { return c ? (void*)c->stream : nullptr; }

int32_t ss_hip_sync(ss_hip_ctx_t* c) {
  if (!c) return fail(kErrParams, "null context");
  HIP_TRY(hipStreamSynchronize(c->stream));
  return 0;
}

void* ss_hip_malloc(ss_hip_ctx_t* c, size_t bytes) {
  if (!c || set_device(c)) return nullptr;
  void* p = nullptr;
  if (hipMalloc(&p, bytes ? bytes : 1) != hipSuccess) {
    fail(kErrOom, "hipMalloc(%zu) failed", bytes);
    return nullptr;
  }
  return p;
}

int32_t ss_hip_mfree(ss_hip_ctx_t* c, void* p) {
  if (!c) return fail(kErrParams, "null context");
  if (p) HIP_TRY(hipFree(p));
  return 0;
}

int32_t ss_hip_memcpy_h2d(ss_hip_ctx_t* c, void* dev, const void* host, size_t bytes) {
  if (!c) return fail(kErrParams, "null context");
  HIP_TRY(hipStreamSynchronize(c->stream));
  HIP_TRY(hipMemcpy(dev, host, bytes, hipMemcpyHostToDevice));
  return 0;
}

int32_t ss_hip_memcpy_d2h(ss_hip_ctx_t* c, void* host, const void* dev, size_t bytes) {
  if (!c) return fail(kErrParams, "null context");
  HIP_TRY(hipStreamSynchronize(c->stream));
  HIP_TRY(hipMemcpy(host, dev, bytes, hipMemcpyDeviceToHost));
  return 0;
}

size_t ss_hip_packed_bytes(int32_t type, int32_t rows, int32_t cols) {
  if (!quant_type_ok(type) || rows <= 0 || cols <= 0 || cols % col_unit(type)) return 0;
  return ssk::packed_bytes(type, rows, cols);
}

int32_t ss_hip_pack_matrix(ss_hip_ctx_t* c, void* dst, const void* src, int32_t type,
                           int32_t rows, int32_t cols) {
  if (!c || !dst || !src) return fail(kErrParams, "null argument");
  if (!quant_type_ok(type) || rows <= 0 || cols <= 0 || cols % col_unit(type))
    return fail(kErrParams, "pack: unsupported type %d or shape %dx%d", type, rows, cols);
  if (set_device(c)) return kErrBackend;
  // rows are padded to a multiple of 64 with zero codes and zero scales
  HIP_TRY(hipMemsetAsync(dst, 0, ssk::packed_bytes(type, rows, cols), c->stream));
  return pack_rows(c, dst, rows, 0, src, type, rows, cols);
}

// ============================================================== single ops
static int32_t check_mv(int32_t rows, int32_t cols, int32_t type) {
  if (!quant_type_ok(type)) return fail(kErrParams, "matvec: type %d is not one of %s", type, kTypesSupported);
  if (rows <= 0 || cols <= 0 || cols % col_unit(type))
    return fail(kErrParams, "matvec: bad shape %dx%d (cols must be a multiple of %d)", rows, cols, col_unit(type));
  return 0;
}

static ssk::GemvArgs gemv_args(const void* w, const float* x, float* y, int rows, int cols,
                               int type) {
  ssk::GemvArgs a;
  memset(&a, 0, sizeof(a));
  a.w = view(w, type, rows, cols);
  a.x = x;
  a.y = y;
  a.rows = rows;
  a.cols = cols;
  a.type = type;
  a.n_cu = g_n_cu;
  a.out_scale = 1.f;
  return a;
}

int32_t ss_hip_matvec(ss_hip_ctx_t* c, float* y, const void* w, const float* x, int32_t rows,
                      int32_t cols, int32_t type, void* stream) {
  return ss_hip_matvec_fused(c, y, w, x, nullptr, 0.f, 0, rows, cols, type, stream);
}

int32_t ss_hip_gemm(ss_hip_ctx_t* c, float* y, const void* w, const float* x, const float* nw, float eps,
                    int32_t accumulate, int32_t rows, int32_t cols, int32_t n_tokens, int32_t type, void* stream) {
  // the MFMA products take every block type (F16 / F32 prompts run token by token)
  if (!c || !y || !w || !x || rows <= 0 || cols <= 0 || cols % col_unit(type) || n_tokens <= 0 ||
      !quant_type_ok(type) || !product_type(type))
    return fail(kErrParams, "gemm: bad argument (rows %d cols %d tokens %d type %d)", rows, cols, n_tokens, type);
  if (set_device(c)) return kErrBackend;
  int32_t rc = ensure(c, (void**)&c->g_ssq, &c->g_ssq_bytes, sizeof(float) * n_tokens, false);
  if (!rc) rc = ensure(c, (void**)&c->g_xs, &c->g_xs_bytes, 2 * ssk::gemm_split_elems(n_tokens, cols), false);
  if (rc) return rc;
  hipStream_t s = pick(c, stream);
  ssk::GemmArgs a;
  memset(&a, 0, sizeof(a));
  a.w = view(w, type, rows, cols);
  a.x = x;
  a.nw = nw;
  a.ssq = c->g_ssq;
  a.xs = c->g_xs;
  a.eps = eps;
  a.y = y;
  a.ldx = cols;
  a.ldy = rows;
  a.rows = rows;
  a.cols = cols;
  a.T = n_tokens;
  a.type = type;
  HIP_TRY(ssk::launch_gemm(accumulate ? ssk::EPI_ADD : ssk::EPI_STORE, a, s));
  return 0;
}

int32_t ss_hip_matvec_q4_0(ss_hip_ctx_t* c, float* y, const void* w, const float* x, int32_t rows,
                           int32_t cols, void* stream) {
  return ss_hip_matvec(c, y, w, x, rows, cols, SS_HIP_Q4_0, stream);
}

int32_t ss_hip_matvec_q8_0(ss_hip_ctx_t* c, float* y, const void* w, const float* x, int32_t rows,
                           int32_t cols, void* stream) {
  return ss_hip_matvec(c, y, w, x, rows, cols, SS_HIP_Q8_0, stream);
}

int32_t ss_hip_matvec_q4_k(ss_hip_ctx_t* c, float* y, const void* w, const float* x, int32_t rows,
                           int32_t cols, void* stream) {
  return ss_hip_matvec(c, y, w, x, rows, cols, SS_HIP_Q4_K, stream);
}

int32_t ss_hip_matvec_fused(ss_hip_ctx_t* c, float* y, const void* w, const float* x,
                            const float* nw, float eps, int32_t accumulate, int32_t rows,
                            int32_t cols, int32_t type, void* stream) {
  if (!c || !y || !w || !x) return fail(kErrParams, "matvec: null argument");
  if (int32_t rc = check_mv(rows, cols, type)) return rc;
  ssk::GemvArgs a = gemv_args(w, x, y, rows, cols, type);
  a.nw = nw;
  a.eps = eps;
  HIP_TRY(ssk::launch_gemv(accumulate ? ssk::EPI_ADD : ssk::EPI_STORE, a, pick(c, stream)));
  return 0;
}

int32_t ss_hip_ffn_gate_up(ss_hip_ctx_t* c, float* out, const void* wg, const void* wu,
                           const float* x, const float* nw, float eps, int32_t rows, int32_t cols,
                           int32_t type, void* stream) {
  if (!c || !out || !wg || !wu || !x) return fail(kErrParams, "ffn_gate_up: null argument");
  if (int32_t rc = check_mv(rows, cols, type)) return rc;
  ssk::GemvArgs a = gemv_args(wg, x, out, rows, cols, type);
  a.w2 = view(wu, type, rows, cols);
  a.nw = nw;
  a.eps = eps;
  HIP_TRY(ssk::launch_gemv(ssk::EPI_SWIGLU, a, pick(c, stream)));
  return 0;
}

int32_t ss_hip_rmsnorm(ss_hip_ctx_t* c, float* out, const float* x, const float* w, int32_t n,
                       float eps, void* stream) {
  if (!c || !out || !x || !w || n <= 0) return fail(kErrParams, "rmsnorm: bad argument");
  HIP_TRY(ssk::launch_rmsnorm(out, x, w, n, eps, pick(c, stream)));
  return 0;
}

int32_t ss_hip_rope(ss_hip_ctx_t* c, float* q, float* k, int32_t n_heads, int32_t n_kv_heads,
                    int32_t head_dim, int32_t rope_dim, int32_t pos, float theta, int32_t is_neox,
                    void* stream) {
  if (!c || !q || !k || n_heads <= 0 || n_kv_heads <= 0 || rope_dim <= 0 || rope_dim % 2 ||
      rope_dim > head_dim || pos < 0)
    return fail(kErrParams, "rope: bad argument");
  std::vector<float> cs((size_t)rope_dim);
  rope_row(cs.data(), rope_dim, pos, theta);
  if (c->rope_row_len < rope_dim) {
    if (c->rope_row) hipFree(c->rope_row);
    c->rope_row = nullptr;
    HIP_TRY(hipMalloc(&c->rope_row, sizeof(float) * rope_dim));
    c->rope_row_len = rope_dim;
  }
  hipStream_t s = pick(c, stream);
  HIP_TRY(hipStreamSynchronize(s));
  HIP_TRY(hipMemcpy(c->rope_row, cs.data(), sizeof(float) * rope_dim, hipMemcpyHostToDevice));
  HIP_TRY(ssk::launch_rope(q, k, n_heads, n_kv_heads, head_dim, rope_dim, c->rope_row, is_neox, s));
  return 0;
}

int32_t ss_hip_kv_append(ss_hip_ctx_t* c, void* kc, void* vc, float* ksc, float* vsc,
                         const float* k, const float* v, int32_t n_kv_heads, int32_t head_dim,
                         int32_t max_seq, int32_t pos, int32_t kv_type, void* stream) {
  if (!c || !kc || !vc || !k || !v || n_kv_heads <= 0 || head_dim <= 0 || pos < 0 ||
      pos >= max_seq || (kv_type != 0 && kv_type != 1) || (kv_type == 1 && (!ksc || !vsc)))
    return fail(kErrParams, "kv_append: bad argument");
  HIP_TRY(ssk::launch_kv_append(kc, vc, ksc, vsc, k, v, n_kv_heads, head_dim, max_seq, nullptr,
                                pos, kv_type, pick(c, stream)));
  return 0;
}

}  // extern "C"

namespace {

// Arguments and split count shared by ss_hip_attention and its
// allocation-free variant; returns 0 or the error already recorded.
int32_t attention_setup(ss_hip_ctx_t* c, const char* what, ssk::AttnArgs& a, int& group, int& ns,
                        float* out, const float* q, const void* kc, const void* vc, const float* ksc,
                        const float* vsc, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                        int32_t max_seq, int32_t seq_len, int32_t kv_type) {
  if (!c || !out || !q || !kc || !vc || n_kv_heads <= 0 || n_heads % n_kv_heads ||
      seq_len <= 0 || seq_len > max_seq || (kv_type != 0 && kv_type != 1) ||
      (kv_type == 1 && (!ksc || !vsc)))
    return fail(kErrParams, "%s: bad argument", what);
  group = n_heads / n_kv_heads;
  if (!ssk::attention_supported(head_dim, group))
    return fail(kErrParams, "%s: head_dim %d / group %d not supported", what, head_dim, group);
  ns = attn_splits(head_dim, group, max_seq, kv_type, n_kv_heads, c->n_cu);
  memset(&a, 0, sizeof(a));
  a.q = q;
  a.kc = kc;
  a.vc = vc;
  a.ks = ksc;
  a.vs = vsc;
  a.seq_len = seq_len;
  a.max_seq = max_seq;
  a.ns = ns;
  a.n_kv_heads = n_kv_heads;
  a.scale = 1.0f / sqrtf((float)head_dim);
  a.out = out;
  return 0;
}

size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }

}  // namespace

extern "C" {

int32_t ss_hip_attention(ss_hip_ctx_t* c, float* out, const float* q, const void* kc,
                         const void* vc, const float* ksc, const float* vsc, int32_t n_heads,
                         int32_t n_kv_heads, int32_t head_dim, int32_t max_seq, int32_t seq_len,
                         int32_t kv_type, void* stream) {
  ssk::AttnArgs a;
  int group = 0, ns = 0;
  if (int32_t rc = attention_setup(c, "attention", a, group, ns, out, q, kc, vc, ksc, vsc, n_heads, n_kv_heads,
                                   head_dim, max_seq, seq_len, kv_type))
    return rc;
  int32_t rc = ensure(c, (void**)&c->att_o, &c->att_o_floats,
                      sizeof(float) * (size_t)n_kv_heads * ns * group * head_dim, false);
  if (!rc) rc = ensure(c, (void**)&c->att_ml, &c->att_ml_floats,
                       sizeof(float) * (size_t)n_kv_heads * ns * group * 2, false);
  if (!rc) rc = ensure(c, (void**)&c->att_cnt, &c->att_cnt_bytes, sizeof(uint32_t) * (size_t)n_kv_heads, true);
  if (rc) return rc;
  a.part_o = c->att_o;
  a.part_ml = c->att_ml;
  a.cnt = c->att_cnt;
  HIP_TRY(ssk::launch_attention(head_dim, group, kv_type, a, pick(c, stream)));
  return 0;
}

int32_t ss_hip_attention_rows(ss_hip_ctx_t* c, float* out, const float* q, const void* kc, const void* vc,
                              int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, int32_t max_seq,
                              int32_t pos0, int32_t n_tokens, void* stream) {
  if (!c || !out || !q || !kc || !vc || n_kv_heads <= 0 || n_heads % n_kv_heads || pos0 < 0 || n_tokens <= 0 ||
      (int64_t)pos0 + n_tokens > max_seq)
    return fail(kErrParams, "attention_rows: bad argument (pos0 %d, %d tokens, max_seq %d)", pos0, n_tokens,
                max_seq);
  const int group = n_heads / n_kv_heads;
  if (!ssk::attention_supported(head_dim, group))
    return fail(kErrParams, "attention_rows: head_dim %d / group %d not supported", head_dim, group);
  if (set_device(c)) return kErrBackend;
  ssk::AttnArgs a;
  memset(&a, 0, sizeof(a));
  a.q = q;
  a.kc = kc;
  a.vc = vc;
  a.max_seq = max_seq;
  a.ns = 1;
  a.n_kv_heads = n_kv_heads;
  a.scale = 1.0f / sqrtf((float)head_dim);
  a.out = out;
  a.n_tok = n_tokens;
  a.pos0 = pos0;
  a.tok_q = a.tok_o = n_heads * head_dim;
  HIP_TRY(ssk::launch_attention_rows(head_dim, group, a, pick(c, stream)));
  return 0;
}

int32_t ss_hip_attention_noalloc(ss_hip_ctx_t* c, float* out, const float* q, const void* kc,
                                 const void* vc, const float* ksc, const float* vsc, int32_t n_heads,
                                 int32_t n_kv_heads, int32_t head_dim, int32_t max_seq, int32_t seq_len,
                                 int32_t kv_type, void* stream) {
  ssk::AttnArgs a;
  int group = 0, ns = 0;
  if (int32_t rc = attention_setup(c, "attention_noalloc", a, group, ns, out, q, kc, vc, ksc, vsc, n_heads,
                                   n_kv_heads, head_dim, max_seq, seq_len, kv_type))
    return rc;
  if (!c->scratch) return fail(kErrBackend, "attention_noalloc: no scratch address for this context");
  const size_t o_bytes = round256(sizeof(float) * (size_t)n_kv_heads * ns * group * head_dim);
  const size_t ml_bytes = round256(sizeof(float) * (size_t)n_kv_heads * ns * group * 2);
  const size_t cnt_bytes = sizeof(uint32_t) * (size_t)n_kv_heads;
  if (o_bytes + ml_bytes + cnt_bytes > kNoAllocScratchBytes)
    return fail(kErrParams, "attention_noalloc: needs %zu bytes of scratch, more than its %zu (%d KV heads, "
                "%d splits, group %d, head_dim %d)", o_bytes + ml_bytes + cnt_bytes, kNoAllocScratchBytes,
                n_kv_heads, ns, group, head_dim);
  uint8_t* base = static_cast<uint8_t*>(c->scratch);
  a.part_o = reinterpret_cast<float*>(base);
  a.part_ml = reinterpret_cast<float*>(base + o_bytes);
  a.cnt = reinterpret_cast<uint32_t*>(base + o_bytes + ml_bytes);
  hipStream_t s = pick(c, stream);
  // the arrival counters must start at zero; the array keeps the last call's contents
  hipLaunchKernelGGL(k_zero_words, dim3((n_kv_heads + 255) / 256), dim3(256), 0, s, a.cnt, n_kv_heads);
  HIP_TRY(hipGetLastError());
  HIP_TRY(ssk::launch_attention(head_dim, group, kv_type, a, s));
  return 0;
}

int32_t ss_hip_swiglu(ss_hip_ctx_t* c, float* out, const float* g, const float* u, int32_t n,
                      void* stream) {
  if (!c || !out || !g || !u || n <= 0) return fail(kErrParams, "swiglu: bad argument");
  HIP_TRY(ssk::launch_swiglu(out, g, u, n, pick(c, stream)));
  return 0;
}

int32_t ss_hip_argmax(ss_hip_ctx_t* c, int32_t* out, const float* x, int32_t n, void* stream) {
  if (!c || !out || !x || n <= 0) return fail(kErrParams, "argmax: bad argument");
  HIP_TRY(ssk::launch_argmax(out, x, n, c->am_part, pick(c, stream)));
  return 0;
}

int32_t ss_hip_sample_logits(ss_hip_ctx_t* c, const float* logits, int32_t n, float temperature, float top_p,
                             int32_t top_k, uint64_t* rng_state, int32_t* out_host) {
  if (!c || !logits || n <= 0 || !rng_state || !out_host) return fail(kErrParams, "sample: bad argument");
  if (int32_t rc = set_device(c)) return rc;
  if (!c->smp_io) HIP_TRY(hipMalloc((void**)&c->smp_io, 2 * sizeof(uint64_t)));
  hipStream_t s = c->stream;
  if (!(temperature > 0.0f)) {   // tensor.c:366-368
    HIP_TRY(ssk::launch_argmax(reinterpret_cast<int*>(c->smp_io), logits, n, c->am_part, s));
  } else {
    if (int32_t rc = ensure(c, (void**)&c->smp, &c->smp_bytes, sizeof(float) * (size_t)n, false)) return rc;
    ssk::SampleArgs a;
    memset(&a, 0, sizeof(a));
    a.logits = logits;
    a.V = n;
    a.temperature = temperature;
    a.top_p = top_p;
    a.top_k = top_k;
    a.rng = *rng_state;
    a.probs = c->smp;
    a.out = reinterpret_cast<int*>(c->smp_io);
    a.rng_out = c->smp_io + 1;
    HIP_TRY(ssk::launch_sample(a, s));
  }
  uint64_t io[2];
  HIP_TRY(hipMemcpyAsync(io, c->smp_io, sizeof(io), hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  *out_host = (int32_t)(uint32_t)(io[0] & 0xffffffffu);
  if (temperature > 0.0f) *rng_state = io[1];
  return 0;
}

int32_t ss_hip_embed_row(ss_hip_ctx_t* c, float* out, const void* table, int32_t type,
                         int32_t rows, int32_t cols, int32_t token, void* stream) {
  if (!c || !out || !table || token < 0 || token >= rows) return fail(kErrParams, "embed: bad argument");
  if (int32_t rc = check_mv(rows, cols, type)) return rc;
  HIP_TRY(ssk::launch_embed(type, view(table, type, rows, cols), cols, nullptr, nullptr, token, out, nullptr,
                            nullptr, 1.f, pick(c, stream)));
  return 0;
}

// ---- Metal-shaped host plug (metal_backend.h:27-58) ----
int32_t ss_hip_should_use_gpu(int32_t rows, int32_t cols) {   // metal_backend.m:336-340
  return (int64_t)rows * cols > 1024;
}

int32_t ss_hip_matvec_host(ss_hip_ctx_t* c, float* out, const void* mat, const float* vec,
                           int32_t rows, int32_t cols, int32_t type) {
  if (!c || !out || !mat || !vec || check_mv(rows, cols, type)) return 0;
  if (set_device(c)) return 0;
  void* dev = nullptr;
  auto it = c->registry.find(mat);
  if (it != c->registry.end()) {
    dev = it->second;
  } else {
    if (hipMalloc(&dev, ss_hip_packed_bytes(type, rows, cols)) != hipSuccess) return 0;
    if (hipMemset(dev, 0, ss_hip_packed_bytes(type, rows, cols)) != hipSuccess) {
      hipFree(dev);
      return 0;
    }
    if (pack_rows(c, dev, rows, 0, mat, type, rows, cols)) {
      hipFree(dev);
      return 0;
    }
    c->registry[mat] = dev;
  }
  // in a batch: this call's own input and output, the copy to out deferred
  // to ss_hip_end_batch; a full batch leaves the call to the CPU
  const bool batched = c->batch;
  const int slot = c->batch_n;
  if (batched && slot >= ss_hip_ctx::kBatchSlots) return 0;
  float** px = batched ? &c->batch_x[slot] : &c->plug_x;
  float** py = batched ? &c->batch_y[slot] : &c->plug_y;
  size_t* nx = batched ? &c->batch_x_n[slot] : &c->plug_x_n;
  size_t* ny = batched ? &c->batch_y_n[slot] : &c->plug_y_n;
  if (ensure(c, (void**)px, nx, sizeof(float) * cols, false) || ensure(c, (void**)py, ny, sizeof(float) * rows, false))
    return 0;
  if (hipMemcpyAsync(*px, vec, sizeof(float) * cols, hipMemcpyHostToDevice, c->stream) != hipSuccess) return 0;
  if (ss_hip_matvec(c, *py, dev, *px, rows, cols, type, nullptr)) return 0;
  if (batched) {
    c->batch_out[slot] = out;
    c->batch_rows[slot] = rows;
    c->batch_n = slot + 1;
    return 1;
  }
  if (hipMemcpyAsync(out, *py, sizeof(float) * rows, hipMemcpyDeviceToHost, c->stream) != hipSuccess ||
      hipStreamSynchronize(c->stream) != hipSuccess)
    return 0;
  return 1;
}

void ss_hip_begin_batch(ss_hip_ctx_t* c) {   // metal_backend.m:307-312
  if (!c || c->batch) return;
  c->batch = true;
  c->batch_n = 0;
}

int32_t ss_hip_end_batch(ss_hip_ctx_t* c) {   // metal_backend.m:314-330
  if (!c || !c->batch) return 0;
  const int n = c->batch_n;
  c->batch = false;
  c->batch_n = 0;
  if (set_device(c)) return kErrBackend;
  // every copy is attempted, so one failure does not leave the other
  // outputs stale; the first error is reported (the caller then recomputes
  // the whole batch on the CPU)
  hipError_t first = hipSuccess;
  for (int i = 0; i < n; ++i) {
    const hipError_t e = hipMemcpyAsync(c->batch_out[i], c->batch_y[i], sizeof(float) * c->batch_rows[i],
                                        hipMemcpyDeviceToHost, c->stream);
    if (e != hipSuccess && first == hipSuccess) first = e;
  }
  const hipError_t e = hipStreamSynchronize(c->stream);
  if (first == hipSuccess) first = e;
  if (first != hipSuccess)
    return fail(kErrBackend, "end_batch: %s (the batch's outputs must be recomputed)", hipGetErrorString(first));
  return 0;
}

}  // extern "C"

// ============================================================== model
namespace {

struct DevLayer {
  float* attn_norm = nullptr;
  float* ffn_norm = nullptr;
  void* wqkv = nullptr;   // packed [Wq;Wk;Wv]
  float* bqkv = nullptr;  // q/k/v biases [qdim + 2*kvdim] in fp32, or nullptr
  void* wo = nullptr;
  void* wg = nullptr;
  void* wu = nullptr;
  void* wd = nullptr;
  int t_qkv = 0, t_o = 0, t_gu = 0, t_d = 0;
  float* post_attn = nullptr;   // Gemma 2 post norms as (1 + w), or nullptr
  float* post_ffn = nullptr;
};

enum ProfClass { PC_Q4 = 0, PC_Q8 = 1, PC_ATTN = 2, PC_OTHER = 3, PC_SWEEP = 4, PC_N = 5 };

struct ProfRec {
  int cls;
  double bytes;
  hipEvent_t a, b;
};

}  // namespace

struct ss_hip_model {
  ss_hip_ctx* ctx = nullptr;
  int L = 0, d = 0, H = 0, KVH = 0, hd = 0, rope_dim = 0, ffn = 0, vocab = 0, max_seq = 0;
  int qdim = 0, kvdim = 0, group = 0, ns = 0, embd_rows = 0;
  // decode attention, query groups of 1 or 2: while splits of one round of
  // loads cover the context, at most kMergeSplits are active and the Wo
  // matvec merges them; past that, with more than kMergeSplits splits
  // allocated, the last split of each KV head merges them (decided per
  // token from the active count)
  int split_fill = 0;
  bool wo_merge_dyn = false;
  // query groups of 4 or 8 with more splits than Wo merges: a separate
  // kernel merges them after the attention (ssk::launch_attention_merge)
  bool merge_kernel = false;
  float eps = 1e-5f, theta = 10000.f;
  int kv_type = 0;
  int launch = SS_HIP_LAUNCH_SWEEP;   // mode in effect
  std::vector<DevLayer> layers;
  void* embd = nullptr;
  int t_embd = 0;
  void* out = nullptr;   // == embd when tied
  int t_out = 0;
  // some layer matrix has no prompt-product kernel (F16 or F32): prompts run
  // token by token
  bool no_products = false;
  // Gemma and the optional branches (layer_scheduler.c:446-448, 474-481,
  // 529-531, 553-560, 597-602, 667-676); the (1 + w) norms are uploaded as 1 + w
  bool gemma = false;
  float emb_scale = 1.f;     // sqrt(d) for Gemma
  float logit_scale = 1.f;   // 1/sqrt(d) for Gemma
  float attn_softcap = 0.f, final_softcap = 0.f;
  bool any_post = false;     // some layer has a post norm
  float* post_y = nullptr;   // [d]: a projection's output before its post norm
  // prompts run token by token (the prompt products take no F16 / F32 layer
  // matrices)
  bool token_only = false;
  float* out_norm = nullptr;
  // KV cache: [L][KVH][max_seq][hd] (+ [L][max_seq] scales for int8)
  void* kc = nullptr;
  void* vc = nullptr;
  float* ks = nullptr;
  float* vs = nullptr;
  size_t kv_layer_elems = 0;
  // activations
  float *hidden = nullptr, *q = nullptr, *attn = nullptr, *ffn_act = nullptr, *logits = nullptr;
  float *kv_f32 = nullptr, *rope_cs = nullptr, *dbg = nullptr;
  int* dpos = nullptr;
  int* tokens = nullptr;   // [max_seq + 1]
  int* argmax = nullptr;
  float2* lm_part = nullptr;
  int lm_grid = 0;
  float *att_o = nullptr, *att_ml = nullptr;
  uint32_t* att_cnt = nullptr;   // [KVH] split arrivals of the attention merge (zero between launches)
  // x records (ss_device.h) passed from each matvec to the next: xr_hid holds
  // the residual stream times the next RMSNorm weight (written by the
  // embedding, Wo and down), xr_ffn the SwiGLU output (written by gate/up)
  uint32_t *xr_hid = nullptr, *xr_ffn = nullptr;
  uint32_t* xr_att = nullptr;   // the attention output (written by its split merge) for Wo

  int* h_io = nullptr;   // pinned host scratch
  hipGraphExec_t g_full = nullptr, g_nohead = nullptr;
  int host_pos = -1;     // position of the last evaluated token (-1 = none)
  const volatile int32_t* cancel = nullptr;
  uint64_t bytes = 0;
  // profiling (eager launches bracketed by events)
  bool prof = false;
  std::vector<ProfRec> prof_recs;
  std::vector<hipEvent_t> ev_pool;
  size_t ev_used = 0;
  std::vector<void*> allocs;
  // persistent sweep (launch == SS_HIP_LAUNCH_SWEEP)
  ssk::SweepArgs sw;                 // host copy of the argument block
  ssk::SweepArgs* sw_dev = nullptr;  // device copy read by the kernel
  int sw_type = 0;                   // layer matrix type
  uint32_t sw_epoch = 0;             // flag value every workgroup holds between launches
  double sw_bytes = 0;               // algorithmic bytes of one token at the last launch
  uint64_t* sw_trace = nullptr;      // phase stamps of the last launch (when enabled)
  // streaming mode: the layer matrices stay in pinned host memory and are
  // uploaded into a ring of device slots as the layers are evaluated
  bool streaming = false;
  int n_slots = 0;
  std::vector<void*> host_layers;    // pinned, one packed block per layer
  std::vector<size_t> layer_size;    // bytes of each block
  std::vector<size_t> layer_off;     // [L][5] offsets of [Wq;Wk;Wv], Wo, gate, up, down in a block
  std::vector<void*> slots;          // device slots (largest block each)
  std::vector<hipEvent_t> ev_ready, ev_free, ev_half;
  hipStream_t copy_stream = nullptr, copy_stream2 = nullptr;   // each upload is split over both
  uint64_t up_issued = 0, up_used = 0;   // uploads issued / consumed
  uint64_t host_bytes = 0;           // pinned bytes held
  int* pos_iota = nullptr;           // device [max_seq]: value i at index i
  float* hid_all = nullptr;          // device [max_seq][d]: residual streams of a prompt
  uint32_t* xr_all = nullptr;        // device [max_seq][xrec_words(d)]: their x records
  // prompts as matrix products (fp16 KV): up to pf_cap tokens per pass over the
  // layers, in row-major [token][...] buffers
  int pf_min = 0;                    // shortest prompt evaluated this way (0: the default)
  int pf_cap = 0;                    // chunk capacity (0: not set up)
  float *pf_h = nullptr, *pf_qkv = nullptr, *pf_att = nullptr, *pf_f = nullptr, *pf_ssq = nullptr;
  float* pf_y = nullptr;   // [chunk][d]: projections before their post norm (Gemma 2)
  uint16_t* pf_xs = nullptr;         // x of a product split into fp16 parts
  float* emb = nullptr;              // [2d + 64]: pooled sum, embedding, a sum of squares
};

namespace {

int32_t m_alloc(ss_hip_model* m, void** p, size_t bytes, bool zero = true) {
  *p = nullptr;
  hipError_t e = hipMalloc(p, bytes ? bytes : 1);
  if (e != hipSuccess)
    return fail(kErrOom, "hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
  m->allocs.push_back(*p);
  m->bytes += bytes;
  if (zero) HIP_TRY(hipMemset(*p, 0, bytes ? bytes : 1));
  return 0;
}

// An F32 or F16 vector of n elements widened to fp32 into h.
int32_t host_f32(const ss_hip_tensor_t& t, int n, const char* what, float* h);

// An F32/F16 vector widened to fp32, plus add (1 for the (1 + w) norms of
// tensor.c:133-152: the one fp32 rounding of w + 1.0f done once here).
int32_t upload_vec(ss_hip_model* m, float** dst, const ss_hip_tensor_t& t, int n, const char* what,
                   float add = 0.f) {
  std::vector<float> h((size_t)n);
  if (int32_t rc = host_f32(t, n, what, h.data())) return rc;
  if (add != 0.f)
    for (float& v : h) v = v + add;
  if (int32_t rc = m_alloc(m, (void**)dst, sizeof(float) * n, false)) return rc;
  HIP_TRY(hipMemcpy(*dst, h.data(), sizeof(float) * n, hipMemcpyHostToDevice));
  return 0;
}

int32_t host_f32(const ss_hip_tensor_t& t, int n, const char* what, float* h) {
  if (!t.data) return fail(kErrParams, "model: missing %s", what);
  if (t.type != SS_HIP_F32 && t.type != SS_HIP_F16)
    return fail(kErrParams, "model: %s has type %d (F32/F16 expected)", what, t.type);
  if ((int64_t)t.rows * t.cols != n) return fail(kErrParams, "model: %s has %d x %d elements, %d expected", what, t.rows, t.cols, n);
  if (t.type == SS_HIP_F32) {
    memcpy(h, t.data, sizeof(float) * n);
  } else {
    // exact binary16 widening (quantize.c:20-56)
    const uint16_t* s = static_cast<const uint16_t*>(t.data);
    for (int i = 0; i < n; i++) {
      const uint32_t hv = s[i];
      const uint32_t sign = (hv & 0x8000u) << 16;
      uint32_t e = (hv >> 10) & 0x1F, mant = hv & 0x3FF, bits;
      if (e == 0) {
        if (mant == 0) {
          bits = sign;
        } else {
          e = 1;
          while (!(mant & 0x400)) { mant <<= 1; e--; }
          bits = sign | ((e + 112) << 23) | ((mant & 0x3FF) << 13);
        }
      } else if (e == 31) {
        bits = sign | 0x7F800000u | (mant << 13);
      } else {
        bits = sign | ((e + 112) << 23) | (mant << 13);
      }
      memcpy(&h[i], &bits, 4);
    }
  }
  return 0;
}

// into: null to allocate the packed matrix, else a zeroed device buffer to pack into
int32_t upload_mat(ss_hip_model* m, void** dst, const ss_hip_tensor_t* parts, int nparts, int rows_expect_total,
                   int cols, int* type_out, const char* what, void* into = nullptr) {
  int type = parts[0].type;
  int64_t total = 0;
  for (int i = 0; i < nparts; i++) {
    if (!parts[i].data) return fail(kErrParams, "model: missing %s", what);
    if (parts[i].type != type)
      return fail(kErrParams, "model: %s parts have mixed types (%d vs %d)", what, type, parts[i].type);
    if (parts[i].cols != cols) return fail(kErrParams, "model: %s has %d columns, %d expected", what, parts[i].cols, cols);
    total += parts[i].rows;
  }
  if (!quant_type_ok(type))
    return fail(kErrParams, "model: %s has type %d; %s are supported", what, type, kTypesSupported);
  if (total != rows_expect_total) return fail(kErrParams, "model: %s has %lld rows, %d expected", what, (long long)total, rows_expect_total);
  if (cols % col_unit(type))
    return fail(kErrParams, "model: %s columns %d not a multiple of %d", what, cols, col_unit(type));
  // zero-filled: rows are padded to a multiple of 64 with zero codes and scales
  if (into)
    *dst = into;
  else if (int32_t rc = m_alloc(m, dst, ss_hip_packed_bytes(type, (int)total, cols), true))
    return rc;
  int64_t off = 0;
  for (int i = 0; i < nparts; i++) {
    if (int32_t rc = pack_rows(m->ctx, *dst, total, off, parts[i].data, type, parts[i].rows, cols)) return rc;
    off += parts[i].rows;
  }
  *type_out = type;
  return 0;
}

hipEvent_t next_event(ss_hip_model* m) {
  if (m->ev_used == m->ev_pool.size()) {
    hipEvent_t e;
    hipEventCreate(&e);
    m->ev_pool.push_back(e);
  }
  return m->ev_pool[m->ev_used++];
}

// Launch with timing events (profiling mode only; never inside a capture):
// matvec and attention launches hand the events to their dispatch, which
// records them at kernel start and end; other launches are bracketed by
// events on the stream.
template <class F>
hipError_t timed(ss_hip_model* m, int cls, double bytes, F&& launch) {
  if (!m->prof) return launch();
  ProfRec r{cls, bytes, next_event(m), next_event(m)};
  ssk::KernelEvents& ke = ssk::kernel_events();
  if (cls == PC_Q4 || cls == PC_Q8 || cls == PC_ATTN) {
    ke.start = r.a;
    ke.stop = r.b;
    ke.used = false;
  } else {
    hipEventRecord(r.a, m->ctx->stream);
  }
  hipError_t e = launch();
  if (ke.start) {
    if (!ke.used) {   // the launch failed before its dispatch: empty interval
      hipEventRecord(r.a, m->ctx->stream);
      hipEventRecord(r.b, m->ctx->stream);
    }
    ke = ssk::KernelEvents();
  }
  if (cls != PC_Q4 && cls != PC_Q8 && cls != PC_ATTN) hipEventRecord(r.b, m->ctx->stream);
  m->prof_recs.push_back(r);
  return e;
}

// Rows the LM-head table was packed with: the embedding's (tied, possibly
// more than the vocabulary) or the vocabulary (output.weight is packed
// clamped). The packed planes' offsets depend on it.
int out_rows(const ss_hip_model* m) { return m->out == m->embd ? m->embd_rows : m->vocab; }

// 8-bit codes on the device (Q8_0, Q5_K, Q6_K), or 4-bit (the rest)
int q_class(int type) { return ssk::code_bytes_of(type) == 32 ? PC_Q8 : PC_Q4; }

// Algorithmic HBM bytes of one token at context ctx: every weight byte once
// (GGUF block sizes), the fp16 K/V read and appended, the norm weights.
double token_bytes(const ss_hip_model* m, int ctx, bool with_head) {
  double b = 0;
  for (const DevLayer& ly : m->layers) {
    b += matvec_bytes(ly.t_qkv, m->qdim + 2 * m->kvdim, m->d, 1) + matvec_bytes(ly.t_o, m->d, m->qdim, 1) +
         matvec_bytes(ly.t_gu, m->ffn, m->d, 2) + matvec_bytes(ly.t_d, m->d, m->ffn, 1);
    b += 2.0 * 2 * ((double)ctx * m->kvdim + m->kvdim) + 2.0 * 4 * m->d;
  }
  if (with_head) b += matvec_bytes(m->t_out, m->vocab, m->d, 1) + 4.0 * m->d;
  b += (double)gguf_row_bytes(m->t_embd, m->d);
  return b;
}

// One persistent launch per token when the shape allows it: fp16 KV, one
// quantisation type (Q4_0 or Q8_0) for all layer matrices and the head, a
// Q4_0/Q8_0 embedding, a supported head shape, and the
// workgroups (one per compute unit) co-resident. Otherwise the model keeps
// the per-kernel launches (graph mode).
int32_t sweep_setup(ss_hip_model* m) {
  if (m->kv_type != SS_HIP_KV_F16) return 1;
  const int lt = m->layers[0].t_qkv;
  for (const DevLayer& ly : m->layers)
    if (ly.t_qkv != lt || ly.t_o != lt || ly.t_gu != lt || ly.t_d != lt) return 1;
  if (!ssk::sweep_supported(m->hd, m->group, lt, m->t_out)) return 1;
  if (m->t_embd != SS_HIP_Q4_0 && m->t_embd != SS_HIP_Q8_0) return 1;   // the sweep stages Q4_0/Q8_0 rows only
  if (m->gemma || m->any_post || m->attn_softcap > 0.f || m->final_softcap > 0.f) return 1;   // llama blocks only
  int nwg = m->ctx->n_cu < ssk::kSweepMaxWg ? m->ctx->n_cu : ssk::kSweepMaxWg;
  if (m->KVH > nwg) return 1;
  ssk::SweepArgs& a = m->sw;
  memset(&a, 0, sizeof(a));
  a.embd = view(m->embd, m->t_embd, m->embd_rows, m->d);
  a.out = view(m->out, m->t_out, out_rows(m), m->d);
  a.embd_type = m->t_embd;
  a.out_norm = m->out_norm;
  a.rope_cs = m->rope_cs;
  a.n_layers = m->L;
  a.d = m->d;
  a.qdim = m->qdim;
  a.kvdim = m->kvdim;
  a.ffn = m->ffn;
  a.vocab = m->vocab;
  a.max_seq = m->max_seq;
  a.rope_dim = m->rope_dim;
  a.n_kv_heads = m->KVH;
  a.eps = m->eps;
  a.attn_scale = 1.0f / sqrtf((float)m->hd);
  a.timeout_ticks = 200000000ull;   // 2 s at the 100 MHz s_memrealtime clock
  size_t lds = 0;
  for (;;) {   // the shared-memory plan depends on the workgroup count
    a.nwg = nwg;
    a.ns = nwg / m->KVH;
    lds = ssk::sweep_lds_bytes(a, m->hd, m->group);
    if (lds > 160 * 1024) return 1;
    int max_wg = 0;
    HIP_TRY(ssk::sweep_max_workgroups(m->hd, m->group, lt, m->t_out, lds, &max_wg));
    if (max_wg >= nwg) break;
    if (max_wg < m->KVH || max_wg < 1) return 1;
    nwg = max_wg;
  }
  std::vector<ssk::SweepLayer> ls(m->L);
  for (int l = 0; l < m->L; l++) {
    const DevLayer& ly = m->layers[l];
    ssk::SweepLayer& s = ls[l];
    s.qkv = view(ly.wqkv, lt, m->qdim + 2 * m->kvdim, m->d);
    s.o = view(ly.wo, lt, m->d, m->qdim);
    s.gate = view(ly.wg, lt, m->ffn, m->d);
    s.up = view(ly.wu, lt, m->ffn, m->d);
    s.down = view(ly.wd, lt, m->d, m->ffn);
    s.attn_norm = ly.attn_norm;
    s.ffn_norm = ly.ffn_norm;
    s.kc = reinterpret_cast<uint16_t*>(static_cast<char*>(m->kc) + (size_t)l * m->kv_layer_elems * 2);
    s.vc = reinterpret_cast<uint16_t*>(static_cast<char*>(m->vc) + (size_t)l * m->kv_layer_elems * 2);
  }
  void* layers = nullptr;
  if (int32_t rc = m_alloc(m, &layers, sizeof(ssk::SweepLayer) * m->L, false)) return rc;
  HIP_TRY(hipMemcpy(layers, ls.data(), sizeof(ssk::SweepLayer) * m->L, hipMemcpyHostToDevice));
  a.layers = static_cast<const ssk::SweepLayer*>(layers);
  a.tokens = m->tokens;
  a.dpos = m->dpos;
  a.argmax = m->argmax;
  a.hidden = m->hidden;
  a.logits = m->logits;
  const size_t rec = 64;   // bytes per x record of 16 values
  const size_t L = (size_t)m->L;
  if (int32_t rc = m_alloc(m, (void**)&a.hrec, rec * (m->d / 16) * 2 * L)) return rc;
  if (int32_t rc = m_alloc(m, (void**)&a.frec, rec * (m->ffn / 16) * L)) return rc;
  if (int32_t rc = m_alloc(m, (void**)&a.arec, rec * (m->qdim / 16) * L)) return rc;
  if (int32_t rc = m_alloc(m, (void**)&a.q, sizeof(float) * m->qdim * L)) return rc;
  if (int32_t rc = m_alloc(m, (void**)&a.part, sizeof(float) * (size_t)m->KVH * a.ns * m->group * (m->hd + 2) * L))
    return rc;
  if (int32_t rc = m_alloc(m, (void**)&a.att_cnt, sizeof(uint32_t) * (size_t)m->L * m->KVH)) return rc;
  if (int32_t rc = m_alloc(m, (void**)&a.cand, sizeof(float2) * nwg)) return rc;
  if (int32_t rc = m_alloc(m, (void**)&a.flags, sizeof(uint32_t) * ssk::kSweepFlagWords)) return rc;
  if (int32_t rc = m_alloc(m, (void**)&m->sw_dev, sizeof(ssk::SweepArgs), false)) return rc;
  HIP_TRY(hipMemcpy(m->sw_dev, &a, sizeof(a), hipMemcpyHostToDevice));
  m->sw_type = lt;
  m->sw_epoch = 0;
  m->launch = SS_HIP_LAUNCH_SWEEP;
  return 0;
}

// Zero the progress flags and split counters (after a launch gave up, or a reset).
int32_t sweep_clear(ss_hip_model* m) {
  hipStream_t s = m->ctx->stream;
  HIP_TRY(hipMemsetAsync(m->sw.flags, 0, sizeof(uint32_t) * ssk::kSweepFlagWords, s));
  HIP_TRY(hipMemsetAsync(m->sw.att_cnt, 0, sizeof(uint32_t) * (size_t)m->L * m->KVH, s));
  m->sw_epoch = 0;
  return 0;
}

// After the stream has been synchronised: did a launch give up waiting?
int32_t sweep_check(ss_hip_model* m) {
  if (m->launch != SS_HIP_LAUNCH_SWEEP) return 0;
  uint32_t w[2] = {0, 0};
  HIP_TRY(hipMemcpy(w, m->sw.flags + ssk::kSweepAbort, sizeof(w), hipMemcpyDeviceToHost));
  if (!w[0]) return 0;
  sweep_clear(m);
  hipStreamSynchronize(m->ctx->stream);
  m->host_pos = -1;
  return fail(kErrBackend, "token launch abandoned: workgroup %u timed out waiting in phase %u",
              w[1] & 0xffffu, w[1] >> 16);
}

// Token embedding of tokens[*dpos] into hidden (layer_scheduler.c:578-595),
// and the x records of hidden * attn_norm[0] into xr for the first layer's
// QKV matvec.
int32_t enqueue_embed(ss_hip_model* m, const int* dpos, float* hidden, uint32_t* xr) {
  hipStream_t s = m->ctx->stream;
  HIP_TRY(timed(m, PC_OTHER, 0, [&] {
    return ssk::launch_embed(m->t_embd, view(m->embd, m->t_embd, m->embd_rows, m->d), m->d, m->tokens,
                             dpos, 0, hidden, m->layers[0].attn_norm, xr, m->emb_scale, s);
  }));
  return 0;
}

// One decoder layer (process_layer, layer_scheduler.c:291-567) for the token
// at position *dpos whose residual stream is hidden; ly holds the layer's
// weights (resident, or the streaming slot it was uploaded to). xr holds the
// token's hidden * attn_norm as x records (written by the embedding or the
// previous layer's down matvec), which the QKV matvec reads; down writes the
// records of the next layer's attn_norm (or output_norm after the last) back
// into xr. Inside the layer, Wo writes the records (xr_hid) gate/up reads
// and gate/up those (xr_ffn) down reads.
int32_t enqueue_layer(ss_hip_model* m, int l, const DevLayer& ly, float* hidden, const int* dpos,
                      uint32_t* xr) {
  hipStream_t s = m->ctx->stream;
  int* dp = const_cast<int*>(dpos);
  char* kc = static_cast<char*>(m->kc) + (size_t)l * m->kv_layer_elems * (m->kv_type ? 1 : 2);
  char* vc = static_cast<char*>(m->vc) + (size_t)l * m->kv_layer_elems * (m->kv_type ? 1 : 2);
  float* ksl = m->ks ? m->ks + (size_t)l * m->max_seq : nullptr;
  float* vsl = m->vs ? m->vs + (size_t)l * m->max_seq : nullptr;

  // 1. rmsnorm(attn_norm) -> [Wq;Wk;Wv] -> RoPE -> KV append   (layer_scheduler.c:320-413)
  ssk::GemvArgs a = gemv_args(ly.wqkv, hidden, m->q, m->qdim + 2 * m->kvdim, m->d, ly.t_qkv);
  a.nw = ly.attn_norm;
  a.eps = m->eps;
  a.qdim = m->qdim;
  a.kvdim = m->kvdim;
  a.head_dim = m->hd;
  a.rope_dim = m->rope_dim;
  a.max_seq = m->max_seq;
  a.kv_type = m->kv_type;
  a.rope_cs = m->rope_cs;
  a.dpos = dp;
  a.kcache = kc;
  a.vcache = vc;
  a.kv_f32 = m->kv_f32;
  a.xr = xr;
  a.bias = ly.bqkv;
  HIP_TRY(timed(m, q_class(ly.t_qkv), matvec_bytes(ly.t_qkv, a.rows, m->d, 1),
                [&] { return ssk::launch_gemv(ssk::EPI_QKV, a, s); }));
  if (m->kv_type == 1)
    HIP_TRY(timed(m, PC_OTHER, 0, [&] {
      return ssk::launch_kv_append(kc, vc, ksl, vsl, m->kv_f32, m->kv_f32 + m->kvdim, m->KVH, m->hd,
                                   m->max_seq, dp, 0, 1, s);
    }));

  // 2. attention over positions 0..pos                          (:415-468)
  ssk::AttnArgs at;
  memset(&at, 0, sizeof(at));
  at.q = m->q;
  at.kc = kc;
  at.vc = vc;
  at.ks = ksl;
  at.vs = vsl;
  at.dpos = dp;
  at.max_seq = m->max_seq;
  at.ns = m->ns;
  at.n_kv_heads = m->KVH;
  at.scale = 1.0f / sqrtf((float)m->hd);
  at.softcap = m->attn_softcap;
  at.softcap_inv = m->attn_softcap > 0.f ? 1.0f / m->attn_softcap : 0.f;
  at.out = m->attn;
  at.part_o = m->att_o;
  at.part_ml = m->att_ml;
  at.split_fill = m->split_fill;
  // with few splits the Wo matvec merges them while staging (measured
  // faster than the last-arriver merge for up to kMergeSplits splits); with
  // more, the last split of each KV head merges them and writes the output
  // as x records for Wo, or (wo_merge_dyn) only when more than kMergeSplits
  // are active at this token's context
  const bool fused = m->ns <= ssk::kMergeSplits;
  const bool direct = m->group <= 2;   // one active split writes Wo's records itself
  at.cnt = fused || m->merge_kernel ? nullptr : m->att_cnt;
  at.xr_out = fused && !direct ? nullptr : m->xr_att;
  at.wo_merge = m->wo_merge_dyn;
  HIP_TRY(timed(m, PC_ATTN, 0, [&] { return ssk::launch_attention(m->hd, m->group, m->kv_type, at, s); }));
  if (m->merge_kernel)
    HIP_TRY(timed(m, PC_ATTN, 0, [&] { return ssk::launch_attention_merge(m->hd, m->group, at, s); }));

  // 3. hidden += Wo attn                                         (:470-484)
  // (with a post norm: y = Wo attn, then hidden += y * (1 + w) / rms(y), :474-481)
  ssk::GemvArgs o = gemv_args(ly.wo, m->attn, ly.post_attn ? m->post_y : hidden, m->d, m->qdim, ly.t_o);
  if (fused || m->wo_merge_dyn) {
    o.att_o = m->att_o;
    o.att_ml = m->att_ml;
    o.att_ns = m->ns;
    o.att_group = m->group;
    o.att_split_fill = m->split_fill;
    o.head_dim = m->hd;
    o.dpos = dp;
  }
  if (!fused || direct) o.xr = m->xr_att;
  if (ly.post_attn) {
    HIP_TRY(timed(m, q_class(ly.t_o), matvec_bytes(ly.t_o, m->d, m->qdim, 1),
                  [&] { return ssk::launch_gemv(ssk::EPI_STORE, o, s); }));
    HIP_TRY(timed(m, PC_OTHER, 0, [&] {
      return ssk::launch_post_norm(hidden, m->post_y, ly.post_attn, m->d, m->eps, m->xr_hid, ly.ffn_norm, s);
    }));
  } else {
    o.xr_out = m->xr_hid;
    o.nw_out = ly.ffn_norm;
    HIP_TRY(timed(m, q_class(ly.t_o), matvec_bytes(ly.t_o, m->d, m->qdim, 1),
                  [&] { return ssk::launch_gemv(ssk::EPI_ADD, o, s); }));
  }

  // 4. rmsnorm(ffn_norm) -> gate, up -> silu(gate) * up           (:486-550)
  ssk::GemvArgs gu = gemv_args(ly.wg, hidden, m->ffn_act, m->ffn, m->d, ly.t_gu);
  gu.w2 = view(ly.wu, ly.t_gu, m->ffn, m->d);
  gu.nw = ly.ffn_norm;
  gu.eps = m->eps;
  gu.xr = m->xr_hid;
  gu.xr_out = m->xr_ffn;
  gu.act = m->gemma ? 1 : 0;   // GeGLU for Gemma (:529-531)
  HIP_TRY(timed(m, q_class(ly.t_gu), matvec_bytes(ly.t_gu, m->ffn, m->d, 2),
                [&] { return ssk::launch_gemv(ssk::EPI_SWIGLU, gu, s); }));

  // 5. hidden += Wdown act                                       (:552-566)
  // (with a post norm, as for Wo: :553-560)
  ssk::GemvArgs dn = gemv_args(ly.wd, m->ffn_act, ly.post_ffn ? m->post_y : hidden, m->d, m->ffn, ly.t_d);
  dn.xr = m->xr_ffn;
  const float* nw_next = l + 1 < m->L ? m->layers[l + 1].attn_norm : m->out_norm;
  if (ly.post_ffn) {
    HIP_TRY(timed(m, q_class(ly.t_d), matvec_bytes(ly.t_d, m->d, m->ffn, 1),
                  [&] { return ssk::launch_gemv(ssk::EPI_STORE, dn, s); }));
    HIP_TRY(timed(m, PC_OTHER, 0, [&] {
      return ssk::launch_post_norm(hidden, m->post_y, ly.post_ffn, m->d, m->eps, xr, nw_next, s);
    }));
  } else {
    dn.xr_out = xr;
    dn.nw_out = nw_next;
    HIP_TRY(timed(m, q_class(ly.t_d), matvec_bytes(ly.t_d, m->d, m->ffn, 1),
                  [&] { return ssk::launch_gemv(ssk::EPI_ADD, dn, s); }));
  }
  return 0;
}

// output_norm + LM head + first-max argmax (:634-662, tensor.c:318-328) of the
// token at *m->dpos: the winner goes to tokens[pos + 1] and pos advances.
// With xr set, it holds hidden * output_norm as x records (the last layer's
// down matvec wrote them); otherwise the matvec stages hidden itself.
int32_t enqueue_head(ss_hip_model* m, const float* hidden, const uint32_t* xr) {
  hipStream_t s = m->ctx->stream;
  ssk::GemvArgs h = gemv_args(m->out, hidden, m->logits, m->vocab, m->d, m->t_out);
  h.w = view(m->out, m->t_out, out_rows(m), m->d);   // the first vocab rows of the table
  h.nw = m->out_norm;
  h.eps = m->eps;
  h.xr = xr;
  h.part = m->lm_part;
  h.out_scale = m->logit_scale;   // Gemma 1/sqrt(d) (:667-672), then the final softcap (:674-676)
  h.softcap = m->final_softcap;
  h.softcap_inv = m->final_softcap > 0.f ? 1.0f / m->final_softcap : 0.f;
  HIP_TRY(timed(m, q_class(m->t_out), matvec_bytes(m->t_out, m->vocab, m->d, 1),
                [&] { return ssk::launch_gemv(ssk::EPI_LOGITS, h, s); }));
  HIP_TRY(timed(m, PC_OTHER, 0, [&] {
    return ssk::launch_argmax_merge(m->lm_part, m->lm_grid, m->logits, m->argmax, m->tokens, m->dpos, s);
  }));
  return 0;
}

// ---- streaming mode (layer_scheduler.c:608-616 prefetch, gguf_loader.c:494-507)
// Layer uploads form one sequence over tokens: upload k carries layer k % L
// into slot k % n_slots. Upload k starts on the copy stream once the layer
// that last used its slot has been computed (ev_free), and the compute
// stream waits for it (ev_ready) before the layer's kernels; up to n_slots
// uploads are in flight, so the next layers (and the first layers of the
// next token) copy while the current layer computes.
// An upload is split in two halves on two copy streams (two DMA engines):
// one stream alone leaves the link idle between consecutive uploads.
int32_t stream_issue(ss_hip_model* m) {
  const uint64_t k = m->up_issued;
  const int slot = (int)(k % (uint64_t)m->n_slots), l = (int)(k % (uint64_t)m->L);
  const size_t half = (m->layer_size[l] / 2 + 255) & ~(size_t)255;
  char* dst = static_cast<char*>(m->slots[slot]);
  const char* src = static_cast<const char*>(m->host_layers[l]);
  HIP_TRY(hipStreamWaitEvent(m->copy_stream, m->ev_free[slot], 0));
  HIP_TRY(hipStreamWaitEvent(m->copy_stream2, m->ev_free[slot], 0));
  HIP_TRY(hipMemcpyAsync(dst, src, half, hipMemcpyHostToDevice, m->copy_stream));
  HIP_TRY(hipMemcpyAsync(dst + half, src + half, m->layer_size[l] - half, hipMemcpyHostToDevice,
                         m->copy_stream2));
  HIP_TRY(hipEventRecord(m->ev_half[slot], m->copy_stream2));
  HIP_TRY(hipStreamWaitEvent(m->copy_stream, m->ev_half[slot], 0));
  HIP_TRY(hipEventRecord(m->ev_ready[slot], m->copy_stream));
  m->up_issued++;
  return 0;
}

// The weights of layer l for the next kernels on the model stream.
int32_t stream_acquire(ss_hip_model* m, int l, DevLayer* out) {
  if (m->up_used % (uint64_t)m->L != (uint64_t)l) {
    // an evaluation stopped part way (cancel, error): drain both streams and
    // restart the upload sequence at this layer
    HIP_TRY(hipStreamSynchronize(m->copy_stream));
    HIP_TRY(hipStreamSynchronize(m->copy_stream2));
    HIP_TRY(hipStreamSynchronize(m->ctx->stream));
    m->up_used = m->up_issued = (uint64_t)l;
  }
  while (m->up_issued < m->up_used + (uint64_t)m->n_slots)
    if (int32_t rc = stream_issue(m)) return rc;
  const int slot = (int)(m->up_used % (uint64_t)m->n_slots);
  HIP_TRY(hipStreamWaitEvent(m->ctx->stream, m->ev_ready[slot], 0));
  char* base = static_cast<char*>(m->slots[slot]);
  const size_t* off = &m->layer_off[(size_t)l * 5];
  *out = m->layers[l];
  out->wqkv = base + off[0];
  out->wo = base + off[1];
  out->wg = base + off[2];
  out->wu = base + off[3];
  out->wd = base + off[4];
  return 0;
}

// The kernels of the acquired layer are enqueued: its slot may be refilled.
int32_t stream_release(ss_hip_model* m) {
  const int slot = (int)(m->up_used % (uint64_t)m->n_slots);
  HIP_TRY(hipEventRecord(m->ev_free[slot], m->ctx->stream));
  m->up_used++;
  while (m->up_issued < m->up_used + (uint64_t)m->n_slots)
    if (int32_t rc = stream_issue(m)) return rc;
  return 0;
}

// Enqueue one token on the model stream. The token is tokens[*dpos]. With
// the head, the last workgroup of the LM-head matvec writes the argmax to
// tokens[*dpos + 1] and advances *dpos; without it, k_advance does.
int32_t enqueue_token(ss_hip_model* m, bool with_head) {
  hipStream_t s = m->ctx->stream;
  if (m->launch == SS_HIP_LAUNCH_SWEEP) {
    ssk::SweepLaunch sl;
    sl.args = m->sw_dev;
    sl.epoch0 = m->sw_epoch;
    sl.with_head = with_head ? 1 : 0;
    HIP_TRY(timed(m, PC_SWEEP, m->sw_bytes,
                  [&] { return ssk::launch_sweep(m->sw, sl, m->hd, m->group, m->sw_type, m->t_out, s); }));
    m->sw_epoch += (uint32_t)ssk::sweep_phases(m->L, with_head);
    return 0;
  }
  if (int32_t rc = enqueue_embed(m, m->dpos, m->hidden, m->xr_hid)) return rc;
  for (int l = 0; l < m->L; l++) {
    if (m->cancel && *m->cancel && !m->prof) return fail(kErrCancel, "cancelled");
    if (m->streaming) {
      DevLayer ly;
      if (int32_t rc = stream_acquire(m, l, &ly)) return rc;
      if (int32_t rc = enqueue_layer(m, l, ly, m->hidden, m->dpos, m->xr_hid)) return rc;
      if (int32_t rc = stream_release(m)) return rc;
    } else {
      if (int32_t rc = enqueue_layer(m, l, m->layers[l], m->hidden, m->dpos, m->xr_hid)) return rc;
    }
  }
  if (with_head) return enqueue_head(m, m->hidden, m->xr_hid);
  HIP_TRY(timed(m, PC_OTHER, 0, [&] { return ssk::launch_advance(m->dpos, s); }));
  return 0;
}

// Streaming mode prompt, layer-major like ss_scheduler_prefill
// (layer_scheduler.c:681-803): every layer is uploaded once for the whole
// prompt and applied to each token in order (a token's attention reads the
// K/V the earlier tokens of the prompt appended to this layer's cache).
// x records of prompt token i in the layer-major order
uint32_t* xr_of(ss_hip_model* m, int i) { return m->xr_all + (size_t)i * ssk::xrec_words(m->d); }

int32_t enqueue_prompt_layer_major(ss_hip_model* m, const int32_t* tokens, int n, int start) {
  hipStream_t s = m->ctx->stream;
  for (int i = 0; i < n; i++)
    if (int32_t rc = enqueue_embed(m, m->pos_iota + start + i, m->hid_all + (size_t)i * m->d, xr_of(m, i))) return rc;
  for (int l = 0; l < m->L; l++) {
    if (m->cancel && *m->cancel) return fail(kErrCancel, "cancelled");
    DevLayer ly;
    if (int32_t rc = stream_acquire(m, l, &ly)) return rc;
    for (int i = 0; i < n; i++)
      if (int32_t rc = enqueue_layer(m, l, ly, m->hid_all + (size_t)i * m->d, m->pos_iota + start + i, xr_of(m, i)))
        return rc;
    if (int32_t rc = stream_release(m)) return rc;
  }
  HIP_TRY(hipMemcpyAsync(m->hidden, m->hid_all + (size_t)(n - 1) * m->d, sizeof(float) * m->d,
                         hipMemcpyDeviceToDevice, s));
  HIP_TRY(ssk::launch_set_state(m->dpos, m->tokens, start + n - 1, tokens[n - 1], s));
  return enqueue_head(m, m->hidden, xr_of(m, n - 1));
}

// ---- prompts as matrix products (ss_scheduler_prefill, layer_scheduler.c:681-803)
// The reference evaluates a prompt layer by layer, each layer's matvecs once
// per token. Here a chunk of up to kPrefillChunk tokens goes through each
// layer as MFMA products of the quantised matrices with the chunk's rows
// (ss_gemm.hip), one RoPE + fp16 append kernel and one attention launch
// whose grid z is the token (each token attends to positions 0..its own, the
// chunk's K/V having been appended first). Later chunks read the earlier
// chunks' cache. Prompts shorter than kPrefillMin tokens, and int8 caches,
// run token by token.
constexpr int kPrefillChunk = 512;
constexpr int kPrefillMin = 8;

int32_t prefill_setup(ss_hip_model* m) {
  if (m->pf_cap) return 0;
  const int cap = std::min(kPrefillChunk, m->max_seq);
  if (!m->pos_iota) {
    if (int32_t rc = m_alloc(m, (void**)&m->pos_iota, sizeof(int) * m->max_seq, false)) return rc;
    std::vector<int> iota(m->max_seq);
    for (int i = 0; i < m->max_seq; i++) iota[i] = i;
    HIP_TRY(hipMemcpy(m->pos_iota, iota.data(), sizeof(int) * m->max_seq, hipMemcpyHostToDevice));
  }
  const size_t c = (size_t)cap;
  if (int32_t rc = m_alloc(m, (void**)&m->pf_h, sizeof(float) * c * m->d, false)) return rc;
  if (int32_t rc = m_alloc(m, (void**)&m->pf_qkv, sizeof(float) * c * (m->qdim + 2 * m->kvdim), false)) return rc;
  if (int32_t rc = m_alloc(m, (void**)&m->pf_att, sizeof(float) * c * m->qdim, false)) return rc;
  if (int32_t rc = m_alloc(m, (void**)&m->pf_f, sizeof(float) * c * m->ffn, false)) return rc;
  if (int32_t rc = m_alloc(m, (void**)&m->pf_ssq, sizeof(float) * c, false)) return rc;
  if (m->any_post)
    if (int32_t rc = m_alloc(m, (void**)&m->pf_y, sizeof(float) * c * m->d, false)) return rc;
  const int widest = std::max(std::max(m->d, m->qdim), m->ffn);
  if (int32_t rc = m_alloc(m, (void**)&m->pf_xs, 2 * ssk::gemm_split_elems(cap, widest), false)) return rc;
  m->pf_cap = cap;
  return 0;
}

ssk::GemmArgs gemm_args(ss_hip_model* m, const void* w, int type, int rows, int cols, const float* x, float* y,
                        int T) {
  ssk::GemmArgs a;
  memset(&a, 0, sizeof(a));
  a.w = view(w, type, rows, cols);
  a.x = x;
  a.y = y;
  a.ssq = m->pf_ssq;
  a.xs = m->pf_xs;
  a.ldx = cols;
  a.ldy = rows;
  a.rows = rows;
  a.cols = cols;
  a.T = T;
  a.type = ssk::dev_type(type);
  return a;
}

// One decoder layer (process_layer, layer_scheduler.c:291-567) for the T
// prompt tokens at positions p0 .. p0+T-1 whose residual streams are the rows
// of pf_h.
int32_t enqueue_layer_rows(ss_hip_model* m, int l, const DevLayer& ly, int T, int p0) {
  hipStream_t s = m->ctx->stream;
  const int* dpos = m->pos_iota + p0;
  uint16_t* kc = static_cast<uint16_t*>(m->kc) + (size_t)l * m->kv_layer_elems;
  uint16_t* vc = static_cast<uint16_t*>(m->vc) + (size_t)l * m->kv_layer_elems;
  const int ldq = m->qdim + 2 * m->kvdim;

  // 1. rmsnorm(attn_norm) -> [Wq;Wk;Wv] -> RoPE -> KV append   (layer_scheduler.c:320-413)
  ssk::GemmArgs a = gemm_args(m, ly.wqkv, ly.t_qkv, ldq, m->d, m->pf_h, m->pf_qkv, T);
  a.nw = ly.attn_norm;
  a.eps = m->eps;
  HIP_TRY(timed(m, PC_OTHER, 0, [&] { return ssk::launch_gemm(ssk::EPI_STORE, a, s); }));
  HIP_TRY(timed(m, PC_OTHER, 0, [&] {
    return ssk::launch_rope_kv_rows(m->pf_qkv, ly.bqkv, ldq, m->qdim, m->kvdim, m->hd, m->rope_dim, m->rope_cs, dpos,
                                    kc, vc, m->max_seq, T, s);
  }));

  // 2. attention of every token over positions 0..its own        (:415-468)
  ssk::AttnArgs at;
  memset(&at, 0, sizeof(at));
  at.q = m->pf_qkv;
  at.tok_q = ldq;
  at.kc = kc;
  at.vc = vc;
  at.dpos = dpos;
  at.max_seq = m->max_seq;
  at.ns = 1;
  at.n_kv_heads = m->KVH;
  at.scale = 1.0f / sqrtf((float)m->hd);
  at.out = m->pf_att;
  at.tok_o = m->qdim;
  at.part_o = m->att_o;
  at.part_ml = m->att_ml;
  at.n_tok = T;
  at.softcap = m->attn_softcap;   // (:446-448)
  at.softcap_inv = m->attn_softcap > 0.f ? 1.0f / m->attn_softcap : 0.f;
  HIP_TRY(timed(m, PC_OTHER, 0, [&] { return ssk::launch_attention_rows(m->hd, m->group, at, s); }));

  // 3. hidden += Wo attn, through the post-attention norm when the layer
  //    has one (:470-484)
  ssk::GemmArgs o = gemm_args(m, ly.wo, ly.t_o, m->d, m->qdim, m->pf_att, ly.post_attn ? m->pf_y : m->pf_h, T);
  HIP_TRY(timed(m, PC_OTHER, 0, [&] { return ssk::launch_gemm(ly.post_attn ? ssk::EPI_STORE : ssk::EPI_ADD, o, s); }));
  if (ly.post_attn)
    HIP_TRY(timed(m, PC_OTHER, 0, [&] {
      return ssk::launch_post_norm_rows(m->pf_h, m->pf_y, ly.post_attn, m->d, T, m->eps, s);
    }));

  // 4. rmsnorm(ffn_norm) -> gate, up -> silu(gate) * up           (:486-550)
  ssk::GemmArgs gu = gemm_args(m, ly.wg, ly.t_gu, m->ffn, m->d, m->pf_h, m->pf_f, T);
  gu.w2 = view(ly.wu, ly.t_gu, m->ffn, m->d);
  gu.nw = ly.ffn_norm;
  gu.eps = m->eps;
  gu.act = m->gemma ? 1 : 0;   // GeGLU for Gemma (:529-531)
  HIP_TRY(timed(m, PC_OTHER, 0, [&] { return ssk::launch_gemm(ssk::EPI_SWIGLU, gu, s); }));

  // 5. hidden += Wdown act, through the post-FFN norm when the layer has
  //    one (:552-566)
  ssk::GemmArgs dn = gemm_args(m, ly.wd, ly.t_d, m->d, m->ffn, m->pf_f, ly.post_ffn ? m->pf_y : m->pf_h, T);
  HIP_TRY(timed(m, PC_OTHER, 0, [&] { return ssk::launch_gemm(ly.post_ffn ? ssk::EPI_STORE : ssk::EPI_ADD, dn, s); }));
  if (ly.post_ffn)
    HIP_TRY(timed(m, PC_OTHER, 0, [&] {
      return ssk::launch_post_norm_rows(m->pf_h, m->pf_y, ly.post_ffn, m->d, T, m->eps, s);
    }));
  return 0;
}

// The prompt m->tokens[start .. start+n) at positions start.., chunk by
// chunk through every layer; with pool, each chunk's final hidden states
// through the output norm are added to m->emb (ss_scheduler_embed). Returns
// in *last the rows of the last chunk (its last row is the last token).
int32_t enqueue_rows(ss_hip_model* m, int n, int start, bool pool, int* last) {
  hipStream_t s = m->ctx->stream;
  int T = 0;
  for (int c0 = 0; c0 < n; c0 += T) {
    T = std::min(m->pf_cap, n - c0);
    const int p0 = start + c0;
    HIP_TRY(timed(m, PC_OTHER, 0, [&] {
      return ssk::launch_embed_rows(m->t_embd, view(m->embd, m->t_embd, m->embd_rows, m->d), m->d, m->tokens,
                                    m->pos_iota + p0, T, m->pf_h, m->emb_scale, s);
    }));
    for (int l = 0; l < m->L; l++) {
      if (m->cancel && *m->cancel) return fail(kErrCancel, "cancelled");
      if (m->streaming) {
        DevLayer ly;
        if (int32_t rc = stream_acquire(m, l, &ly)) return rc;
        if (int32_t rc = enqueue_layer_rows(m, l, ly, T, p0)) return rc;
        if (int32_t rc = stream_release(m)) return rc;
      } else {
        if (int32_t rc = enqueue_layer_rows(m, l, m->layers[l], T, p0)) return rc;
      }
    }
    if (pool) {
      if (m->out_norm) HIP_TRY(ssk::launch_sumsq(m->pf_h, m->d, T, m->pf_ssq, s));
      HIP_TRY(ssk::launch_pool_rows(m->pf_h, T, m->d, m->out_norm, m->pf_ssq, m->eps, m->emb, s));
    }
  }
  *last = T;
  return 0;
}

// The prompt tokens[0..n) (already at m->tokens[start..]) at positions
// start.., then the LM head of the last one.
int32_t enqueue_prompt_rows(ss_hip_model* m, const int32_t* tokens, int n, int start) {
  hipStream_t s = m->ctx->stream;
  int T = 0;
  if (int32_t rc = enqueue_rows(m, n, start, false, &T)) return rc;
  HIP_TRY(hipMemcpyAsync(m->hidden, m->pf_h + (size_t)(T - 1) * m->d, sizeof(float) * m->d,
                         hipMemcpyDeviceToDevice, s));
  HIP_TRY(ssk::launch_set_state(m->dpos, m->tokens, start + n - 1, tokens[n - 1], s));
  return enqueue_head(m, m->hidden, nullptr);
}

int32_t capture(ss_hip_model* m, bool with_head, hipGraphExec_t* out) {
  hipStream_t s = m->ctx->stream;
  HIP_TRY(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
  int32_t rc = enqueue_token(m, with_head);
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(s, &g);
  if (rc) {
    if (g) hipGraphDestroy(g);
    return rc;
  }
  if (e != hipSuccess) return fail(kErrBackend, "graph capture failed: %s", hipGetErrorString(e));
  e = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
  hipGraphDestroy(g);
  if (e != hipSuccess) return fail(kErrBackend, "graph instantiate failed: %s", hipGetErrorString(e));
  return 0;
}

// pos: the position of the token (sizes the profiled byte count only)
int32_t run_token(ss_hip_model* m, bool with_head, int pos) {
  if (m->prof) m->sw_bytes = token_bytes(m, pos + 1, with_head);
  if (m->launch == SS_HIP_LAUNCH_GRAPH && !m->prof) {
    HIP_TRY(hipGraphLaunch(with_head ? m->g_full : m->g_nohead, m->ctx->stream));
    return 0;
  }
  return enqueue_token(m, with_head);
}

constexpr int kStreamSlots = 3;

// Streaming mode: block layout of every layer, the device slots, the copy
// stream and its events.
int32_t stream_setup(ss_hip_model* m, const ss_hip_model_desc_t* d) {
  m->n_slots = kStreamSlots;
  m->layer_off.assign((size_t)m->L * 5, 0);
  m->layer_size.assign(m->L, 0);
  m->host_layers.assign(m->L, nullptr);
  size_t max_block = 0;
  for (int l = 0; l < m->L; l++) {
    const ss_hip_tensor_t* t = d->layers + (size_t)l * SS_HIP_LAYER_TENSORS;
    const int rows[5] = {m->qdim + 2 * m->kvdim, m->d, m->ffn, m->ffn, m->d};
    const int cols[5] = {m->d, m->qdim, m->d, m->d, m->ffn};
    const int types[5] = {t[SS_HIP_WQ].type, t[SS_HIP_WO].type, t[SS_HIP_W_GATE].type, t[SS_HIP_W_UP].type,
                          t[SS_HIP_W_DOWN].type};
    size_t o = 0;
    for (int i = 0; i < 5; i++) {
      if (!quant_type_ok(types[i]))
        return fail(kErrParams, "model: blk.%d matrix %d has type %d; %s are supported", l,
                    i, types[i], kTypesSupported);
      m->layer_off[(size_t)l * 5 + i] = o;
      o += align256(ss_hip_packed_bytes(types[i], rows[i], cols[i]));
    }
    m->layer_size[l] = o;
    if (o > max_block) max_block = o;
  }
  m->slots.assign(m->n_slots, nullptr);
  for (int i = 0; i < m->n_slots; i++)
    if (int32_t rc = m_alloc(m, &m->slots[i], max_block, false)) return rc;
  HIP_TRY(hipStreamCreateWithFlags(&m->copy_stream, hipStreamNonBlocking));
  HIP_TRY(hipStreamCreateWithFlags(&m->copy_stream2, hipStreamNonBlocking));
  m->ev_ready.assign(m->n_slots, nullptr);
  m->ev_free.assign(m->n_slots, nullptr);
  m->ev_half.assign(m->n_slots, nullptr);
  for (int i = 0; i < m->n_slots; i++) {
    HIP_TRY(hipEventCreateWithFlags(&m->ev_ready[i], hipEventDisableTiming));
    HIP_TRY(hipEventCreateWithFlags(&m->ev_half[i], hipEventDisableTiming));
    HIP_TRY(hipEventCreateWithFlags(&m->ev_free[i], hipEventDisableTiming));
    HIP_TRY(hipEventRecord(m->ev_free[i], m->ctx->stream));
  }
  if (int32_t rc = m_alloc(m, (void**)&m->pos_iota, sizeof(int) * m->max_seq, false)) return rc;
  std::vector<int> iota(m->max_seq);
  for (int i = 0; i < m->max_seq; i++) iota[i] = i;
  HIP_TRY(hipMemcpy(m->pos_iota, iota.data(), sizeof(int) * m->max_seq, hipMemcpyHostToDevice));
  if (int32_t rc = m_alloc(m, (void**)&m->hid_all, sizeof(float) * (size_t)m->max_seq * m->d, false)) return rc;
  return m_alloc(m, (void**)&m->xr_all, sizeof(uint32_t) * (size_t)m->max_seq * ssk::xrec_words(m->d));
}

// Streaming mode: layer l's matrices were packed into slot 0; keep them in
// pinned host memory.
int32_t stream_keep_layer(ss_hip_model* m, int l) {
  HIP_TRY(hipDeviceSynchronize());
  void* h = nullptr;
  if (hipHostMalloc(&h, m->layer_size[l], hipHostMallocDefault) != hipSuccess)
    return fail(kErrOom, "pinned host allocation of %zu bytes for blk.%d failed", m->layer_size[l], l);
  m->host_layers[l] = h;
  m->host_bytes += m->layer_size[l];
  HIP_TRY(hipMemcpy(h, m->slots[0], m->layer_size[l], hipMemcpyDeviceToHost));
  DevLayer& ly = m->layers[l];
  ly.wqkv = ly.wo = ly.wg = ly.wu = ly.wd = nullptr;   // set per use by stream_acquire
  return 0;
}

void model_release(ss_hip_model* m) {
  if (!m) return;
  hipSetDevice(m->ctx->device);
  hipStreamSynchronize(m->ctx->stream);
  if (m->g_full) hipGraphExecDestroy(m->g_full);
  if (m->g_nohead) hipGraphExecDestroy(m->g_nohead);
  for (void* p : m->allocs) hipFree(p);
  for (hipEvent_t e : m->ev_pool) hipEventDestroy(e);
  if (m->h_io) hipHostFree(m->h_io);
  for (hipStream_t cs : {m->copy_stream, m->copy_stream2})
    if (cs) {
      hipStreamSynchronize(cs);
      hipStreamDestroy(cs);
    }
  for (void* p : m->host_layers)
    if (p) hipHostFree(p);
  for (hipEvent_t e : m->ev_ready) hipEventDestroy(e);
  for (hipEvent_t e : m->ev_free) hipEventDestroy(e);
  for (hipEvent_t e : m->ev_half) hipEventDestroy(e);
  delete m;
}

}  // namespace

extern "C" {

ss_hip_model_t* ss_hip_model_create(ss_hip_ctx_t* c, const ss_hip_model_desc_t* d) {
  if (!c || !d || !d->layers) {
    fail(kErrParams, "model: null argument");
    return nullptr;
  }
  if (set_device(c)) return nullptr;
  if (d->n_layers <= 0 || d->hidden <= 0 || d->n_heads <= 0 || d->n_kv_heads <= 0 ||
      d->head_dim <= 0 || d->ffn <= 0 || d->vocab <= 0 || d->max_seq <= 0 ||
      d->n_heads % d->n_kv_heads || d->rope_dim <= 0 || d->rope_dim > d->head_dim ||
      d->rope_dim % 2 || d->hidden % 32 || d->ffn % 32 || (d->n_heads * d->head_dim) % 32 ||
      (d->kv_type != 0 && d->kv_type != 1)) {
    fail(kErrParams, "model: unsupported shape (L=%d d=%d H=%d KVH=%d hd=%d rope=%d ffn=%d V=%d ctx=%d kv=%d)",
         d->n_layers, d->hidden, d->n_heads, d->n_kv_heads, d->head_dim, d->rope_dim, d->ffn,
         d->vocab, d->max_seq, d->kv_type);
    return nullptr;
  }
  const int group = d->n_heads / d->n_kv_heads;
  if (!ssk::attention_supported(d->head_dim, group)) {
    fail(kErrParams, "model: head_dim %d with %d query heads per KV head is not supported",
         d->head_dim, group);
    return nullptr;
  }
  auto* m = new ss_hip_model();
  m->ctx = c;
  m->L = d->n_layers;
  m->d = d->hidden;
  m->H = d->n_heads;
  m->KVH = d->n_kv_heads;
  m->hd = d->head_dim;
  m->rope_dim = d->rope_dim;
  m->ffn = d->ffn;
  m->vocab = d->vocab;
  m->max_seq = d->max_seq;
  m->eps = d->rms_eps;
  m->theta = d->rope_theta;
  m->kv_type = d->kv_type;
  m->streaming = d->streaming != 0;
  // streaming mode launches per kernel (the slot of a layer changes per token)
  m->launch = d->launch == SS_HIP_LAUNCH_EAGER || m->streaming ? SS_HIP_LAUNCH_EAGER : SS_HIP_LAUNCH_GRAPH;
  m->qdim = m->H * m->hd;
  m->kvdim = m->KVH * m->hd;
  m->group = group;
  m->ns = attn_splits(m->hd, m->group, m->max_seq, m->kv_type, m->KVH, c->n_cu);
  if (m->group <= 2) {
    m->split_fill = ssk::attn_round_positions(m->hd, m->group);
    m->wo_merge_dyn = m->ns > ssk::kMergeSplits;
  } else {
    m->merge_kernel = m->ns > ssk::kMergeSplits;
  }

  auto bail = [&](void) -> ss_hip_model_t* {
    model_release(m);
    return nullptr;
  };

  // weights
  for (int i = 0; i < m->L * SS_HIP_LAYER_TENSORS; i++) {
    const int slot = i % SS_HIP_LAYER_TENSORS;
    if (slot != SS_HIP_ATTN_NORM && slot != SS_HIP_FFN_NORM && d->layers[i].data &&
        !product_type(d->layers[i].type))
      m->no_products = true;
  }
  m->gemma = d->gemma != 0;
  m->emb_scale = m->gemma ? sqrtf((float)m->d) : 1.f;                       // layer_scheduler.c:597-602
  m->logit_scale = m->gemma ? 1.0f / sqrtf((float)m->d) : 1.f;              // :667-672
  m->attn_softcap = d->attn_softcap > 0.f ? d->attn_softcap : 0.f;
  m->final_softcap = d->final_softcap > 0.f ? d->final_softcap : 0.f;
  if (d->post_norms)
    for (int i = 0; i < 2 * m->L; i++)
      if (d->post_norms[i].data) m->any_post = true;
  // (and head_dim 256: the prompt attention kernel covers 64 and 128)
  m->token_only = m->no_products;
  const float norm_add = m->gemma ? 1.f : 0.f;   // (1 + w) norms, tensor.c:133-152
  if (!d->token_embd.data || d->token_embd.cols != m->d || d->token_embd.rows < m->vocab) {
    fail(kErrParams, "model: token_embd must be [>= vocab x hidden]");
    return bail();
  }
  m->embd_rows = d->token_embd.rows;
  if (upload_mat(m, &m->embd, &d->token_embd, 1, m->embd_rows, m->d, &m->t_embd, "token_embd"))
    return bail();
  if (d->output.data && d->output.data != d->token_embd.data) {
    if (d->output.rows < m->vocab) {
      fail(kErrParams, "model: output has %d rows < vocab %d", d->output.rows, m->vocab);
      return bail();
    }
    ss_hip_tensor_t o = d->output;
    o.rows = m->vocab;   // rows beyond the vocab clamp are never read (layer_scheduler.c:660)
    if (upload_mat(m, &m->out, &o, 1, m->vocab, m->d, &m->t_out, "output")) return bail();
  } else {
    m->out = m->embd;   // tied embeddings, layer_scheduler.c:652-655
    m->t_out = m->t_embd;
  }
  if (d->output_norm.data && upload_vec(m, &m->out_norm, d->output_norm, m->d, "output_norm", norm_add))
    return bail();
  m->layers.resize(m->L);
  if (m->streaming && stream_setup(m, d)) return bail();
  for (int l = 0; l < m->L; l++) {
    const ss_hip_tensor_t* t = d->layers + (size_t)l * SS_HIP_LAYER_TENSORS;
    DevLayer& ly = m->layers[l];
    // streaming: pack into slot 0 at the block offsets, then keep on the host
    char* blk = m->streaming ? static_cast<char*>(m->slots[0]) : nullptr;
    const size_t* off = m->streaming ? &m->layer_off[(size_t)l * 5] : nullptr;
    if (blk && hipMemset(blk, 0, m->layer_size[l]) != hipSuccess) {
      fail(kErrBackend, "slot clear failed");
      return bail();
    }
    char what[64];
    snprintf(what, sizeof(what), "blk.%d attn_norm", l);
    if (upload_vec(m, &ly.attn_norm, t[SS_HIP_ATTN_NORM], m->d, what, norm_add)) return bail();
    snprintf(what, sizeof(what), "blk.%d ffn_norm", l);
    if (upload_vec(m, &ly.ffn_norm, t[SS_HIP_FFN_NORM], m->d, what, norm_add)) return bail();
    if (d->post_norms) {   // always the (1 + w) form (layer_scheduler.c:474-481, 553-560)
      for (int k = 0; k < 2; k++) {
        const ss_hip_tensor_t& pn = d->post_norms[(size_t)l * 2 + k];
        if (!pn.data) continue;
        snprintf(what, sizeof(what), "blk.%d %s", l, k ? "post_ffw_norm" : "post_attention_norm");
        if (upload_vec(m, k ? &ly.post_ffn : &ly.post_attn, pn, m->d, what, 1.f)) return bail();
      }
    }
    snprintf(what, sizeof(what), "blk.%d attn_q/k/v", l);
    if (upload_mat(m, &ly.wqkv, t + SS_HIP_WQ, 3, m->qdim + 2 * m->kvdim, m->d, &ly.t_qkv, what,
                   blk ? blk + off[0] : nullptr))
      return bail();
    if (t[SS_HIP_WQ].rows != m->qdim || t[SS_HIP_WK].rows != m->kvdim) {
      fail(kErrParams, "model: blk.%d q/k/v row counts do not match the head shape", l);
      return bail();
    }
    if (d->qkv_bias) {   // layer_scheduler.c:367-402: q, k, v biases as one fp32 vector
      const ss_hip_tensor_t* b = d->qkv_bias + (size_t)l * 3;
      if (b[0].data || b[1].data || b[2].data) {
        if (d->launch == SS_HIP_LAUNCH_SWEEP) {
          fail(kErrParams, "model: the persistent launch does not apply q/k/v biases");
          return bail();
        }
        const int n3[3] = {m->qdim, m->kvdim, m->kvdim};
        std::vector<float> h((size_t)m->qdim + 2 * m->kvdim, 0.f);
        for (int k = 0, o = 0; k < 3; o += n3[k], k++) {
          snprintf(what, sizeof(what), "blk.%d attn_%c.bias", l, "qkv"[k]);
          if (b[k].data && host_f32(b[k], n3[k], what, h.data() + o)) return bail();
        }
        if (m_alloc(m, (void**)&ly.bqkv, sizeof(float) * h.size(), false) ||
            hipMemcpy(ly.bqkv, h.data(), sizeof(float) * h.size(), hipMemcpyHostToDevice) != hipSuccess) {
          fail(kErrBackend, "bias upload failed");
          return bail();
        }
      }
    }
    snprintf(what, sizeof(what), "blk.%d attn_output", l);
    if (upload_mat(m, &ly.wo, t + SS_HIP_WO, 1, m->d, m->qdim, &ly.t_o, what, blk ? blk + off[1] : nullptr))
      return bail();
    snprintf(what, sizeof(what), "blk.%d ffn_gate", l);
    int tu = 0;
    if (upload_mat(m, &ly.wg, t + SS_HIP_W_GATE, 1, m->ffn, m->d, &ly.t_gu, what, blk ? blk + off[2] : nullptr))
      return bail();
    snprintf(what, sizeof(what), "blk.%d ffn_up", l);
    if (upload_mat(m, &ly.wu, t + SS_HIP_W_UP, 1, m->ffn, m->d, &tu, what, blk ? blk + off[3] : nullptr))
      return bail();
    if (tu != ly.t_gu) {
      fail(kErrParams, "model: blk.%d ffn_gate and ffn_up types differ", l);
      return bail();
    }
    snprintf(what, sizeof(what), "blk.%d ffn_down", l);
    if (upload_mat(m, &ly.wd, t + SS_HIP_W_DOWN, 1, m->d, m->ffn, &ly.t_d, what, blk ? blk + off[4] : nullptr))
      return bail();
    if (m->streaming && stream_keep_layer(m, l)) return bail();
  }

  // KV cache and working state
  const size_t esz = m->kv_type ? 1 : 2;
  m->kv_layer_elems = (size_t)m->KVH * m->max_seq * m->hd;
  if (m_alloc(m, &m->kc, m->kv_layer_elems * m->L * esz) ||
      m_alloc(m, &m->vc, m->kv_layer_elems * m->L * esz))
    return bail();
  if (m->kv_type == 1 && (m_alloc(m, (void**)&m->ks, sizeof(float) * m->L * m->max_seq) ||
                          m_alloc(m, (void**)&m->vs, sizeof(float) * m->L * m->max_seq)))
    return bail();
  m->lm_grid = ssk::gemv_plan(m->vocab, m->d, m->t_out, 1).grid;
  const int lm_grid = m->lm_grid;
  if (m_alloc(m, (void**)&m->hidden, sizeof(float) * m->d) ||
      m_alloc(m, (void**)&m->q, sizeof(float) * m->qdim) ||
      m_alloc(m, (void**)&m->attn, sizeof(float) * m->qdim) ||
      m_alloc(m, (void**)&m->ffn_act, sizeof(float) * m->ffn) ||
      m_alloc(m, (void**)&m->logits, sizeof(float) * m->vocab) ||
      m_alloc(m, (void**)&m->kv_f32, sizeof(float) * 2 * m->kvdim) ||
      m_alloc(m, (void**)&m->dbg, sizeof(float) * m->d) ||
      m_alloc(m, (void**)&m->dpos, sizeof(int) * 4) ||
      m_alloc(m, (void**)&m->tokens, sizeof(int) * (m->max_seq + 1)) ||
      m_alloc(m, (void**)&m->argmax, sizeof(int) * 4) ||
      m_alloc(m, (void**)&m->lm_part, sizeof(float2) * lm_grid) ||
      m_alloc(m, (void**)&m->att_o, sizeof(float) * (size_t)m->KVH * m->ns * m->group * m->hd) ||
      m_alloc(m, (void**)&m->att_ml, sizeof(float) * (size_t)m->KVH * m->ns * m->group * 2) ||
      m_alloc(m, (void**)&m->att_cnt, sizeof(uint32_t) * m->KVH) ||
      m_alloc(m, (void**)&m->xr_hid, sizeof(uint32_t) * ssk::xrec_words(m->d)) ||
      m_alloc(m, (void**)&m->xr_ffn, sizeof(uint32_t) * ssk::xrec_words(m->ffn)) ||
      m_alloc(m, (void**)&m->xr_att, sizeof(uint32_t) * ssk::xrec_words(m->qdim)) ||
      m_alloc(m, (void**)&m->emb, sizeof(float) * (2 * (size_t)m->d + 64)) ||
      (m->any_post && m_alloc(m, (void**)&m->post_y, sizeof(float) * m->d)))
    return bail();
  // RoPE (cos, sin) table for every position, computed with the host libm
  // exactly as tensor.c:250-254 computes each pair.
  {
    std::vector<float> cs((size_t)m->max_seq * m->rope_dim);
    for (int p = 0; p < m->max_seq; p++) rope_row(cs.data() + (size_t)p * m->rope_dim, m->rope_dim, p, m->theta);
    if (m_alloc(m, (void**)&m->rope_cs, sizeof(float) * cs.size(), false)) return bail();
    if (hipMemcpy(m->rope_cs, cs.data(), sizeof(float) * cs.size(), hipMemcpyHostToDevice) != hipSuccess) {
      fail(kErrBackend, "rope table upload failed");
      return bail();
    }
  }
  if (hipHostMalloc((void**)&m->h_io, 64 * sizeof(int), hipHostMallocDefault) != hipSuccess) {
    fail(kErrBackend, "pinned host buffer allocation failed");
    return bail();
  }
  if (hipDeviceSynchronize() != hipSuccess) {
    fail(kErrBackend, "model upload failed");
    return bail();
  }
  if (d->launch == SS_HIP_LAUNCH_SWEEP && !m->streaming && sweep_setup(m) < 0) return bail();
  if (m->launch == SS_HIP_LAUNCH_GRAPH && (capture(m, true, &m->g_full) || capture(m, false, &m->g_nohead)))
    return bail();
  return m;
}

void ss_hip_model_free(ss_hip_model_t* m) { model_release(m); }

uint64_t ss_hip_model_bytes(const ss_hip_model_t* m) { return m ? m->bytes : 0; }

uint64_t ss_hip_model_host_bytes(const ss_hip_model_t* m) { return m ? m->host_bytes : 0; }

int32_t ss_hip_model_launch(const ss_hip_model_t* m) { return m ? m->launch : -1; }

int32_t ss_hip_gemm_launch_counts(int64_t* out, int32_t n) {
  if (!out || n < 0) return fail(kErrParams, "gemm_launch_counts: null output");
  const int64_t* c = ssk::gemm_h_launch_counts();
  for (int i = 0; i < n && i < ssk::kGemmVariants; ++i) out[i] = c[i];
  return 0;
}

int32_t ss_hip_trace_enable(ss_hip_model_t* m, int32_t on) {
  if (!m) return fail(kErrParams, "null model");
  if (m->launch != SS_HIP_LAUNCH_SWEEP) return fail(kErrParams, "trace: the model does not use the persistent launch");
  if (set_device(m->ctx)) return kErrBackend;
  HIP_TRY(hipStreamSynchronize(m->ctx->stream));
  if (on && !m->sw_trace) {
    const size_t bytes = sizeof(uint64_t) * ssk::sweep_trace_words(m->L, m->sw.nwg);
    if (int32_t rc = m_alloc(m, (void**)&m->sw_trace, bytes)) return rc;
  }
  m->sw.trace = on ? m->sw_trace : nullptr;
  HIP_TRY(hipMemcpy(m->sw_dev, &m->sw, sizeof(m->sw), hipMemcpyHostToDevice));
  return 0;
}

int64_t ss_hip_trace_read(ss_hip_model_t* m, uint64_t* host, size_t n_words) {
  if (!m || !host) return fail(kErrParams, "trace: bad argument");
  if (!m->sw_trace) return fail(kErrParams, "trace: not enabled");
  if (set_device(m->ctx)) return kErrBackend;
  size_t n = ssk::sweep_trace_words(m->L, m->sw.nwg);
  if (n > n_words) n = n_words;
  HIP_TRY(hipStreamSynchronize(m->ctx->stream));
  HIP_TRY(hipMemcpy(host, m->sw_trace, sizeof(uint64_t) * n, hipMemcpyDeviceToHost));
  return (int64_t)n;
}

void ss_hip_set_cancel_flag(ss_hip_model_t* m, const volatile int32_t* flag) {
  if (m) m->cancel = flag;
}

static int32_t finish_eval(ss_hip_model_t* m, float* logits_host, int32_t* argmax_out) {
  hipStream_t s = m->ctx->stream;
  if (argmax_out) HIP_TRY(hipMemcpyAsync(m->h_io, m->argmax, sizeof(int), hipMemcpyDeviceToHost, s));
  if (logits_host)
    HIP_TRY(hipMemcpyAsync(logits_host, m->logits, sizeof(float) * m->vocab, hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  if (int32_t rc = sweep_check(m)) return rc;
  if (argmax_out) *argmax_out = m->h_io[0];
  return 0;
}

int32_t ss_hip_eval_token(ss_hip_model_t* m, int32_t token, int32_t pos, float* logits_host,
                          int32_t* argmax_out) {
  if (!m) return fail(kErrParams, "null model");
  if (pos < 0 || pos >= m->max_seq) return fail(kErrParams, "pos %d outside [0, %d)", pos, m->max_seq);
  if (token < 0 || token >= m->embd_rows) return fail(kErrParams, "token %d outside [0, %d)", token, m->embd_rows);
  if (set_device(m->ctx)) return kErrBackend;
  if (m->cancel && *m->cancel) return fail(kErrCancel, "cancelled");
  HIP_TRY(ssk::launch_set_state(m->dpos, m->tokens, pos, token, m->ctx->stream));
  if (int32_t rc = run_token(m, true, pos)) return rc;
  m->host_pos = pos;
  return finish_eval(m, logits_host, argmax_out);
}

int32_t ss_hip_eval_prompt(ss_hip_model_t* m, const int32_t* tokens, int32_t n, int32_t start,
                           float* logits_host, int32_t* argmax_out) {
  if (!m || !tokens || n <= 0) return fail(kErrParams, "eval_prompt: bad argument");
  if (start < 0 || start + n > m->max_seq)
    return fail(kErrParams, "prompt [%d, %d) exceeds the context of %d", start, start + n, m->max_seq);
  for (int i = 0; i < n; i++)
    if (tokens[i] < 0 || tokens[i] >= m->embd_rows)
      return fail(kErrParams, "prompt token %d = %d outside [0, %d)", i, tokens[i], m->embd_rows);
  if (set_device(m->ctx)) return kErrBackend;
  hipStream_t s = m->ctx->stream;
  HIP_TRY(hipStreamSynchronize(s));
  HIP_TRY(hipMemcpy(m->tokens + start, tokens, sizeof(int) * n, hipMemcpyHostToDevice));
  HIP_TRY(ssk::launch_set_state(m->dpos, m->tokens, start, tokens[0], s));
  const int pf_min = m->pf_min > 0 ? m->pf_min : kPrefillMin;
  if (m->kv_type == 0 && m->pf_min >= 0 && n >= pf_min && !m->token_only) {
    if (int32_t rc = prefill_setup(m)) return rc;
    if (int32_t rc = enqueue_prompt_rows(m, tokens, n, start)) {
      hipStreamSynchronize(s);
      return rc;
    }
    m->host_pos = start + n - 1;
    return finish_eval(m, logits_host, argmax_out);
  }
  if (m->streaming) {
    if (int32_t rc = enqueue_prompt_layer_major(m, tokens, n, start)) {
      hipStreamSynchronize(s);
      return rc;
    }
    m->host_pos = start + n - 1;
    return finish_eval(m, logits_host, argmax_out);
  }
  for (int i = 0; i < n; i++) {
    if (m->cancel && *m->cancel) {
      hipStreamSynchronize(s);
      return fail(kErrCancel, "cancelled");
    }
    if (int32_t rc = run_token(m, i == n - 1, start + i)) return rc;
  }
  m->host_pos = start + n - 1;
  return finish_eval(m, logits_host, argmax_out);
}

int32_t ss_hip_set_prompt_batch(ss_hip_model_t* m, int32_t min_tokens) {
  if (!m) return fail(kErrParams, "null model");
  m->pf_min = min_tokens;
  return 0;
}

int32_t ss_hip_embed(ss_hip_model_t* m, const int32_t* tokens, int32_t n, float* out_host) {
  if (!m || !tokens || n <= 0 || !out_host) return fail(kErrParams, "embed: bad argument");
  if (n > m->max_seq) return fail(kErrParams, "embed: %d tokens exceed the context of %d", n, m->max_seq);
  for (int i = 0; i < n; i++)
    if (tokens[i] < 0 || tokens[i] >= m->embd_rows)
      return fail(kErrParams, "embed token %d = %d outside [0, %d)", i, tokens[i], m->embd_rows);
  if (set_device(m->ctx)) return kErrBackend;
  hipStream_t s = m->ctx->stream;
  HIP_TRY(hipStreamSynchronize(s));
  HIP_TRY(hipMemcpy(m->tokens, tokens, sizeof(int) * n, hipMemcpyHostToDevice));
  HIP_TRY(hipMemsetAsync(m->emb, 0, sizeof(float) * m->d, s));
  m->host_pos = -1;   // the cache holds positions 0..n-1, but no token to continue from
  int32_t rc = 0;
  if (m->kv_type == 0 && m->pf_min >= 0 && !m->token_only) {
    int T = 0;
    rc = prefill_setup(m);
    if (!rc) rc = enqueue_rows(m, n, 0, true, &T);
  } else {
    float* ssq = m->emb + 2 * (size_t)m->d;
    HIP_TRY(ssk::launch_set_state(m->dpos, m->tokens, 0, tokens[0], s));
    for (int i = 0; i < n && !rc; i++) {
      if (m->cancel && *m->cancel) {
        rc = fail(kErrCancel, "cancelled");
        break;
      }
      rc = run_token(m, false, i);
      if (!rc && m->out_norm) rc = ssk::launch_sumsq(m->hidden, m->d, 1, ssq, s) ? kErrBackend : 0;
      if (!rc) rc = ssk::launch_pool_rows(m->hidden, 1, m->d, m->out_norm, ssq, m->eps, m->emb, s) ? kErrBackend : 0;
    }
  }
  if (rc) {
    hipStreamSynchronize(s);
    return rc < 0 ? rc : kErrBackend;
  }
  HIP_TRY(ssk::launch_embed_finish(m->emb, m->d, n, m->emb + m->d, s));
  HIP_TRY(hipMemcpyAsync(out_host, m->emb + m->d, sizeof(float) * m->d, hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  return sweep_check(m);
}

int32_t ss_hip_sample(ss_hip_model_t* m, float temperature, float top_p, int32_t top_k, uint64_t* rng_state,
                      int32_t* token_out) {
  if (!m) return fail(kErrParams, "sample: no model");
  if (m->host_pos < 0) return fail(kErrParams, "sample: evaluate a token or prompt first");
  if (int32_t rc = sweep_check(m)) return rc;
  return ss_hip_sample_logits(m->ctx, m->logits, m->vocab, temperature, top_p, top_k, rng_state, token_out);
}

int32_t ss_hip_decode_greedy(ss_hip_model_t* m, int32_t n_steps, int32_t* tokens_out) {
  if (!m || n_steps < 0) return fail(kErrParams, "decode_greedy: bad argument");
  if (m->host_pos < 0) return fail(kErrParams, "decode_greedy: evaluate a token or prompt first");
  if (m->host_pos + n_steps >= m->max_seq)
    return fail(kErrParams, "decode_greedy: %d steps from position %d exceed the context of %d",
                n_steps, m->host_pos, m->max_seq);
  if (n_steps == 0) return 0;
  if (set_device(m->ctx)) return kErrBackend;
  hipStream_t s = m->ctx->stream;
  for (int i = 0; i < n_steps; i++) {
    if (m->cancel && *m->cancel) {
      hipStreamSynchronize(s);
      return fail(kErrCancel, "cancelled");
    }
    if (int32_t rc = run_token(m, true, m->host_pos + 1 + i)) return rc;
  }
  const int p0 = m->host_pos;
  m->host_pos += n_steps;
  if (tokens_out)
    HIP_TRY(hipMemcpyAsync(tokens_out, m->tokens + p0 + 2, sizeof(int) * n_steps,
                           hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  return sweep_check(m);
}

int32_t ss_hip_kv_reset(ss_hip_model_t* m) {
  if (!m) return fail(kErrParams, "null model");
  if (set_device(m->ctx)) return kErrBackend;
  hipStream_t s = m->ctx->stream;
  const size_t esz = m->kv_type ? 1 : 2;
  HIP_TRY(hipMemsetAsync(m->kc, 0, m->kv_layer_elems * m->L * esz, s));
  HIP_TRY(hipMemsetAsync(m->vc, 0, m->kv_layer_elems * m->L * esz, s));
  if (m->ks) HIP_TRY(hipMemsetAsync(m->ks, 0, sizeof(float) * m->L * m->max_seq, s));
  if (m->vs) HIP_TRY(hipMemsetAsync(m->vs, 0, sizeof(float) * m->L * m->max_seq, s));
  HIP_TRY(hipMemsetAsync(m->hidden, 0, sizeof(float) * m->d, s));
  HIP_TRY(hipStreamSynchronize(s));
  m->host_pos = -1;
  return 0;
}

int32_t ss_hip_kv_write(ss_hip_model_t* m, int32_t layer, int32_t pos0, int32_t n_pos,
                        const uint16_t* k, const uint16_t* v) {
  if (!m || !k || !v || layer < 0 || layer >= m->L || pos0 < 0 || n_pos <= 0 ||
      pos0 + n_pos > m->max_seq)
    return fail(kErrParams, "kv_write: bad argument");
  if (set_device(m->ctx)) return kErrBackend;
  HIP_TRY(hipStreamSynchronize(m->ctx->stream));
  const size_t esz = m->kv_type ? 1 : 2;
  char* kc = static_cast<char*>(m->kc) + (size_t)layer * m->kv_layer_elems * esz;
  char* vc = static_cast<char*>(m->vc) + (size_t)layer * m->kv_layer_elems * esz;
  if (m->kv_type == 0) {
    // the rows of one KV head are contiguous in the cache: gather them on the
    // host and copy each head's slab at once
    std::vector<uint16_t> slab((size_t)n_pos * m->hd);
    for (int which = 0; which < 2; which++) {
      const uint16_t* src = which ? v : k;
      char* cache = which ? vc : kc;
      for (int g = 0; g < m->KVH; g++) {
        for (int p = 0; p < n_pos; p++)
          memcpy(slab.data() + (size_t)p * m->hd, src + (size_t)p * m->kvdim + (size_t)g * m->hd,
                 (size_t)m->hd * 2);
        HIP_TRY(hipMemcpy(cache + ((size_t)g * m->max_seq + pos0) * m->hd * 2, slab.data(),
                          (size_t)n_pos * m->hd * 2, hipMemcpyHostToDevice));
      }
    }
    return 0;
  }
  // int8 mode: widen to fp32 and encode as layer_scheduler.c:101-118 does
  std::vector<int8_t> qk((size_t)n_pos * m->kvdim), qv((size_t)n_pos * m->kvdim);
  std::vector<float> sk(n_pos), sv(n_pos), f(m->kvdim);
  for (int which = 0; which < 2; which++) {
    const uint16_t* src = which ? v : k;
    std::vector<int8_t>& q = which ? qv : qk;
    std::vector<float>& sc = which ? sv : sk;
    for (int p = 0; p < n_pos; p++) {
      float amax = 0.f;
      for (int i = 0; i < m->kvdim; i++) {
        const uint16_t h = src[(size_t)p * m->kvdim + i];
        const _Float16 hf = __builtin_bit_cast(_Float16, h);
        f[i] = (float)hf;
        if (fabsf(f[i]) > amax) amax = fabsf(f[i]);
      }
      const float s = amax / 127.0f;
      const float inv = s > 0.0f ? 1.0f / s : 0.0f;
      sc[p] = s;
      for (int i = 0; i < m->kvdim; i++) q[(size_t)p * m->kvdim + i] = (int8_t)roundf(f[i] * inv);
    }
  }
  for (int g = 0; g < m->KVH; g++) {
    const size_t dst = ((size_t)g * m->max_seq + pos0) * m->hd;
    HIP_TRY(hipMemcpy2D(kc + dst, (size_t)m->hd, qk.data() + (size_t)g * m->hd, (size_t)m->kvdim,
                        (size_t)m->hd, n_pos, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy2D(vc + dst, (size_t)m->hd, qv.data() + (size_t)g * m->hd, (size_t)m->kvdim,
                        (size_t)m->hd, n_pos, hipMemcpyHostToDevice));
  }
  HIP_TRY(hipMemcpy(m->ks + (size_t)layer * m->max_seq + pos0, sk.data(), sizeof(float) * n_pos,
                    hipMemcpyHostToDevice));
  HIP_TRY(hipMemcpy(m->vs + (size_t)layer * m->max_seq + pos0, sv.data(), sizeof(float) * n_pos,
                    hipMemcpyHostToDevice));
  return 0;
}

int32_t ss_hip_hidden(ss_hip_model_t* m, float* host_out) {
  if (!m || !host_out) return fail(kErrParams, "hidden: bad argument");
  if (set_device(m->ctx)) return kErrBackend;
  hipStream_t s = m->ctx->stream;
  if (m->out_norm)
    HIP_TRY(ssk::launch_rmsnorm(m->dbg, m->hidden, m->out_norm, m->d, m->eps, s));
  else
    HIP_TRY(hipMemcpyAsync(m->dbg, m->hidden, sizeof(float) * m->d, hipMemcpyDeviceToDevice, s));
  HIP_TRY(hipMemcpyAsync(host_out, m->dbg, sizeof(float) * m->d, hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  return 0;
}

int32_t ss_hip_profile_begin(ss_hip_model_t* m) {
  if (!m) return fail(kErrParams, "null model");
  HIP_TRY(hipStreamSynchronize(m->ctx->stream));
  m->prof = true;
  m->prof_recs.clear();
  m->ev_used = 0;
  return 0;
}

// ms_out receives, per class (0 = Q4_0 matvec, 1 = Q8_0 matvec,
// 2 = attention, 3 = other), three doubles: total ms, launches, algorithmic
// bytes; n is the capacity in doubles (12 for all classes).
int32_t ss_hip_profile_end(ss_hip_model_t* m, double* out, int32_t n) {
  if (!m) return fail(kErrParams, "null model");
  HIP_TRY(hipStreamSynchronize(m->ctx->stream));
  double acc[PC_N * 3] = {0};
  for (const ProfRec& r : m->prof_recs) {
    float ms = 0.f;
    HIP_TRY(hipEventElapsedTime(&ms, r.a, r.b));
    acc[r.cls * 3] += ms;
    acc[r.cls * 3 + 1] += 1;
    acc[r.cls * 3 + 2] += r.bytes;
  }
  for (int i = 0; i < n && i < PC_N * 3; i++) out[i] = acc[i];
  m->prof = false;
  m->prof_recs.clear();
  m->ev_used = 0;
  return 0;
}

}  // extern "C"
