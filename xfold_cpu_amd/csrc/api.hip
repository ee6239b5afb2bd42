// C ABI of libxfold_hip.so: validation, workspace carving and kernel sequencing.
// Declarations and their reference counterparts are in include/xfold_hip.h.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "common.h"
#include "kernels.h"

namespace xfh {

static thread_local std::string g_last_error;

void set_error(const std::string &message) { g_last_error = message; }

int fail(int code, const std::string &message) {
  g_last_error = message;
  return code;
}

int check_launch(const char *what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return fail(XFH_EHIP, std::string(what) + ": launch failed: " + hipGetErrorString(err));
  return XFH_OK;
}

int device_cu_count(int *cus) {
  static std::mutex mu;
  static std::vector<int> cache;
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return fail(XFH_EHIP, std::string("hipGetDevice: ") + hipGetErrorString(err));
  std::lock_guard<std::mutex> lock(mu);
  if (dev >= int(cache.size())) cache.resize(dev + 1, 0);
  if (cache[dev] == 0) {
    int n = 0;
    err = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    if (err != hipSuccess || n <= 0)
      return fail(XFH_EHIP, std::string("hipDeviceGetAttribute: ") + hipGetErrorString(err));
    cache[dev] = n;
  }
  *cus = cache[dev];
  return XFH_OK;
}

// ------------------------------------------------------------------ kernel timing
namespace {
struct TimedEvent {
  std::string name;
  hipEvent_t start, stop;
  double work;
};
std::mutex g_timing_mutex;
bool g_timing_enabled = false;
std::vector<TimedEvent> g_timed;
}  // namespace

KernelTimer::KernelTimer(const char *name, hipStream_t stream, double work, bool dispatch)
    : name_(name), stream_(stream), work_(work) {
  if (!g_timing_enabled) return;
  enabled_ = true;
  if (dispatch) return;
  hipEvent_t e;
  if (hipEventCreate(&e) != hipSuccess) return;
  if (hipEventRecord(e, stream_) != hipSuccess) {   // untimed launch: no record is kept
    (void)hipEventDestroy(e);
    return;
  }
  start_ = e;
}

bool KernelTimer::dispatch_events() {
  hipEvent_t a, b;
  if (hipEventCreate(&a) != hipSuccess) return false;
  if (hipEventCreate(&b) != hipSuccess) {
    (void)hipEventDestroy(a);
    return false;
  }
  if (start_) (void)hipEventDestroy(static_cast<hipEvent_t>(start_));   // no bracket start
  start_ = a;
  stop_ = b;
  return true;
}

KernelTimer::~KernelTimer() {
  if (!start_) return;
  hipEvent_t e = static_cast<hipEvent_t>(stop_);
  if (!e) {                                                  // bracket: record the end now
    const bool created = hipEventCreate(&e) == hipSuccess;
    if (!created || hipEventRecord(e, stream_) != hipSuccess) {
      if (created) (void)hipEventDestroy(e);
      (void)hipEventDestroy(static_cast<hipEvent_t>(start_));
      return;
    }
  }
  std::lock_guard<std::mutex> lock(g_timing_mutex);
  g_timed.push_back({name_, static_cast<hipEvent_t>(start_), e, work_});
}

static bool float_dtype(int d) { return d == XFH_F32 || d == XFH_BF16; }
static bool mask_dtype_ok(int d) { return d == XFH_F32 || d == XFH_BF16 || d == XFH_BOOL; }
static int64_t dsize(int d) { return d == XFH_F32 ? 4 : d == XFH_BF16 ? 2 : 1; }

static GemmArgs gemm_args(const void *A, int64_t lda, const void *B, int64_t ldb, void *C,
                          int64_t ldc, int64_t M, int64_t N, int64_t K) {
  GemmArgs g;
  std::memset(&g, 0, sizeof(g));
  g.A = A; g.lda = lda; g.B = B; g.ldb = ldb; g.C = C; g.ldc = ldc;
  g.M = int(M); g.N = int(N); g.K = int(K);
  g.epi = XFH_EPI_STORE;
  return g;
}

// ------------------------------------------------------------------ triangle multiplication
struct TriMulPlan {
  void *normed, *proj, *gate, *left, *right, *contracted, *centered, *gating;
};

static bool trimul_fast_path(int64_t c, int dtype) { return dtype == XFH_BF16 && c == 128; }


static int64_t trimul_carve(Carver &cv, TriMulPlan &p, int64_t n, int64_t c, int dtype, int out_dtype) {
  const int64_t es = dsize(dtype), plane = n * n;
  std::memset(&p, 0, sizeof(p));
  if (trimul_fast_path(c, dtype)) {
    p.left = cv.take(contraction_operand_elems(n, c) * es);
    p.right = cv.take(contraction_operand_elems(n, c) * es);
    p.contracted = cv.take(contraction_result_elems(n, c) * es);
    return cv.used;
  }
  p.normed = cv.take(plane * c * es);
  p.proj = cv.take(plane * 2 * c * es);
  p.gate = cv.take(plane * 2 * c * es);
  p.left = cv.take(plane * c * es);
  p.right = cv.take(plane * c * es);
  p.contracted = cv.take(plane * c * es);
  p.centered = cv.take(plane * c * es);
  p.gating = cv.take(plane * c * dsize(out_dtype));
  return cv.used;
}

// ------------------------------------------------------------------ grid self-attention
struct GridPlan {
  void *normed, *bias, *qkv, *wcat, *attn;
  // fast bf16 path (c = 128, 4 heads x 32)
  void *qh, *kh, *vt;
  float *bias_t;
  uint64_t *maskbits;
  // bf16 at other widths: the pipelined attention kernel's operands (mha.hip)
  void *mha_ws;
  int64_t mha_bytes;
};

static bool grid_fast_path(int64_t n, int64_t c, int64_t heads, int dtype) {
  return dtype == XFH_BF16 && c == 128 && heads == 4 && n <= grid_attention_max_n();
}

static int64_t grid_carve(Carver &cv, GridPlan &p, int64_t n, int64_t c, int64_t heads, int dtype) {
  const int64_t es = dsize(dtype), plane = n * n;
  std::memset(&p, 0, sizeof(p));
  if (grid_fast_path(n, c, heads, dtype)) {
    const int64_t npad = grid_attention_pad(n);
    p.qh = cv.take(plane * c * es);
    p.kh = cv.take(n * c * npad * es);
    p.vt = cv.take(n * c * npad * es);
    p.bias_t = static_cast<float *>(cv.take(heads * n * npad * 4));
    p.maskbits = static_cast<uint64_t *>(cv.take(n * (npad / 64) * 8));
    p.attn = cv.take(plane * c * es);
    return cv.used;
  }
  p.normed = cv.take(plane * c * es);
  p.bias = cv.take(plane * heads * es);
  p.qkv = cv.take(plane * 3 * c * es);
  p.wcat = cv.take(3 * c * c * es);
  p.attn = cv.take(plane * c * es);
  if (dtype == XFH_BF16 && c % heads == 0 && align_up(n, 64) <= grid_attention_max_n()) {
    AttentionArgs a;
    std::memset(&a, 0, sizeof(a));
    a.B = n; a.H = heads; a.Q = n; a.K = n; a.D = c / heads; a.Dv = c / heads;
    p.mha_bytes = mha_workspace_size(a);
    if (p.mha_bytes > 0) p.mha_ws = cv.take(p.mha_bytes);
  }
  return cv.used;
}

}  // namespace xfh

using namespace xfh;

extern "C" {

int xfh_abi_version(void) { return XFH_ABI_VERSION; }

const char *xfh_runtime_info(void) {
  static char info[256];
  std::snprintf(info, sizeof(info),
                "{\"library\": \"xfold_hip\", \"abi\": %d, \"arch\": \"gfx950\", \"hip_version\": %d, "
                "\"mfma\": [\"16x16x32_bf16\", \"16x16x4_f32\"]}",
                XFH_ABI_VERSION, HIP_VERSION);
  return info;
}

const char *xfh_last_error(void) { return g_last_error.c_str(); }

void xfh_set_kernel_timing(int enable) {
  std::lock_guard<std::mutex> lock(g_timing_mutex);
  g_timing_enabled = enable != 0;
}

int xfh_kernel_timing_read(const char *name, double *total_ms, int64_t *launches) {
  double work = 0.0;
  return xfh_kernel_timing_read_work(name, total_ms, launches, &work);
}

int xfh_kernel_timing_read_work(const char *name, double *total_ms, int64_t *launches, double *work) {
  XFH_REQUIRE(name && total_ms && launches && work, "kernel_timing_read: null argument");
  std::lock_guard<std::mutex> lock(g_timing_mutex);
  double total = 0.0, done = 0.0;
  int64_t count = 0;
  std::vector<TimedEvent> keep;
  const char *error = nullptr;                 // every record of `name` is consumed, even after a failure
  for (auto &t : g_timed) {
    if (t.name != name) {
      keep.push_back(t);
      continue;
    }
    float ms = 0.f;
    if (!error && hipEventSynchronize(t.stop) != hipSuccess) error = "kernel_timing_read: sync failed";
    if (!error && hipEventElapsedTime(&ms, t.start, t.stop) != hipSuccess)
      error = "kernel_timing_read: elapsed time failed";
    total += ms;
    done += t.work;
    ++count;
    (void)hipEventDestroy(t.start);
    (void)hipEventDestroy(t.stop);
  }
  g_timed.swap(keep);
  if (error) return fail(XFH_EHIP, error);
  *total_ms = total;
  *launches = count;
  *work = done;
  return XFH_OK;
}

int xfh_layer_norm(const void *x, int x_dtype, int64_t rows, int64_t cols, const float *weight,
                   const float *bias, float eps, void *y, int y_dtype, void *stream) {
  XFH_REQUIRE(rows >= 0 && cols >= 0, "layer_norm: negative size");
  XFH_REQUIRE(float_dtype(x_dtype) && float_dtype(y_dtype), "layer_norm: dtypes must be f32/bf16");
  XFH_REQUIRE(rows == 0 || (x && y), "layer_norm: null tensor");
  XFH_REQUIRE(eps >= 0.f, "layer_norm: eps must be nonnegative");
  return layer_norm_rows(x, x_dtype, rows, cols, weight, bias, eps, y, y_dtype, as_stream(stream));
}

int xfh_adaptive_layer_norm(const void *x, int x_dtype, int64_t rows, int64_t cols,
                            const void *scale, const void *shift, int aux_dtype, int64_t cond_rows,
                            float eps, void *y, int y_dtype, void *stream) {
  XFH_REQUIRE(rows >= 0 && cols >= 0 && cond_rows > 0, "adaptive_layer_norm: bad size");
  XFH_REQUIRE(rows == 0 || (x && y && scale && shift), "adaptive_layer_norm: null tensor");
  XFH_REQUIRE(float_dtype(x_dtype) && float_dtype(y_dtype) && float_dtype(aux_dtype),
              "adaptive_layer_norm: dtypes must be f32/bf16");
  return adaptive_layer_norm_rows(x, x_dtype, rows, cols, scale, shift, aux_dtype, cond_rows, eps,
                                  y, y_dtype, as_stream(stream));
}

int xfh_linear(const void *x, int64_t ldx, const void *w, const float *bias, int64_t m, int64_t k,
               int64_t n, int dtype, void *y, int64_t ldy, int y_dtype, int epilogue,
               const void *aux, int64_t ldaux, int64_t aux_rows, void *stream) {
  XFH_REQUIRE(m >= 0 && k >= 0 && n >= 0, "linear: negative size");
  XFH_REQUIRE(m < (int64_t(1) << 31) && n < (int64_t(1) << 31) && k < (int64_t(1) << 31),
              "linear: sizes must fit in 32 bits");
  XFH_REQUIRE(float_dtype(dtype) && float_dtype(y_dtype), "linear: dtypes must be f32/bf16");
  XFH_REQUIRE(epilogue >= XFH_EPI_STORE && epilogue <= XFH_EPI_MUL_SIGMOID_AUX_ACCUMULATE,
              "linear: unknown epilogue");
  const bool needs_aux = epilogue == XFH_EPI_MUL_SIGMOID_AUX || epilogue == XFH_EPI_SIGMOID_MUL_AUX ||
                         epilogue == XFH_EPI_MUL_SIGMOID_AUX_ACCUMULATE;
  XFH_REQUIRE(!needs_aux || aux, "linear: epilogue needs aux");
  XFH_REQUIRE(ldx >= k && ldy >= n && (!aux || ldaux >= n), "linear: leading dims too small");
  if (m == 0 || n == 0) return XFH_OK;
  XFH_REQUIRE(x && w && y, "linear: null tensor");
  GemmArgs g = gemm_args(x, ldx, w, k, y, ldy, m, n, k);
  g.bias = bias;
  g.epi = epilogue;
  g.aux = needs_aux ? aux : nullptr;
  g.ldaux = ldaux;
  g.aux_rows = aux_rows;
  return gemm_nt(g, 1, dtype, y_dtype, false, as_stream(stream));
}

int xfh_linear_batched(const void *x, int64_t ldx, int64_t sx, const void *w, int64_t sw,
                       const float *bias, int64_t sbias, int64_t m, int64_t k, int64_t n, int64_t batch,
                       int dtype, void *y, int64_t ldy, int64_t sy, int y_dtype, void *stream) {
  XFH_REQUIRE(m >= 0 && k >= 0 && n >= 0 && batch >= 0, "linear_batched: negative size");
  XFH_REQUIRE(m < (int64_t(1) << 31) && n < (int64_t(1) << 31) && k < (int64_t(1) << 31),
              "linear_batched: sizes must fit in 32 bits");
  XFH_REQUIRE(batch <= 65535, "linear_batched: at most 65535 batch entries");
  XFH_REQUIRE(float_dtype(dtype) && float_dtype(y_dtype), "linear_batched: dtypes must be f32/bf16");
  XFH_REQUIRE(ldx >= k && ldy >= n && sx >= 0 && sw >= 0 && sbias >= 0 && sy >= 0,
              "linear_batched: leading dims or batch strides invalid");
  XFH_REQUIRE(batch <= 1 || sy >= m * ldy, "linear_batched: outputs of batch entries overlap");
  if (m == 0 || n == 0 || batch == 0) return XFH_OK;
  XFH_REQUIRE(x && w && y, "linear_batched: null tensor");
  GemmArgs g = gemm_args(x, ldx, w, k, y, ldy, m, n, k);
  g.sA = sx; g.sB = sw; g.sC = sy;
  g.bias = bias; g.sBias = bias ? sbias : 0;
  return gemm_nt(g, batch, dtype, y_dtype, false, as_stream(stream));
}

int64_t xfh_glu_packed_rows(int64_t f) { return 2 * align_up(f, 16); }

int xfh_glu_pack_weight(const void *w, int64_t f, int64_t k, int dtype, void *packed, void *stream) {
  XFH_REQUIRE(f >= 0 && k >= 0, "glu_pack_weight: negative size");
  XFH_REQUIRE(float_dtype(dtype), "glu_pack_weight: dtype must be f32/bf16");
  XFH_REQUIRE((f == 0 || k == 0) || (w && packed), "glu_pack_weight: null tensor");
  return glu_pack(w, f, k, dtype, packed, as_stream(stream));
}

int xfh_gated_linear_unit(const void *x, const void *w_packed, int64_t m, int64_t k, int64_t f,
                          int dtype, void *y, int y_dtype, void *stream) {
  XFH_REQUIRE(m >= 0 && k >= 0 && f >= 0, "gated_linear_unit: negative size");
  XFH_REQUIRE(m < (int64_t(1) << 31) && k < (int64_t(1) << 31), "gated_linear_unit: sizes must fit in 32 bits");
  XFH_REQUIRE(float_dtype(dtype) && float_dtype(y_dtype), "gated_linear_unit: dtypes must be f32/bf16");
  if (m == 0 || f == 0) return XFH_OK;
  XFH_REQUIRE(x && w_packed && y, "gated_linear_unit: null tensor");
  GemmArgs g = gemm_args(x, k, w_packed, k, y, f, m, xfh_glu_packed_rows(f), k);
  g.glu_f = int(f);
  return gemm_nt(g, 1, dtype, y_dtype, true, as_stream(stream));
}

int64_t xfh_dot_product_attention_workspace_size(const int64_t *shape, int dtype) {
  if (!shape || !float_dtype(dtype)) return -1;
  for (int i = 0; i < 6; ++i)
    if (shape[i] < 0) return -1;
  if (dtype != XFH_BF16) return 0;
  AttentionArgs a;
  std::memset(&a, 0, sizeof(a));
  a.B = shape[0]; a.H = shape[1]; a.Q = shape[2]; a.K = shape[3]; a.D = shape[4]; a.Dv = shape[5];
  return mha_workspace_size(a);
}

int xfh_dot_product_attention(const void *q, const void *k, const void *v, int dtype,
                              const void *mask, int mask_dtype, const void *bias, int bias_dtype,
                              void *out, int out_dtype, const int64_t *shape, const int64_t *strides,
                              float scale, void *workspace, int64_t workspace_bytes, void *stream) {
  XFH_REQUIRE(shape && strides, "dot_product_attention: null shape/strides");
  XFH_REQUIRE(float_dtype(dtype), "dot_product_attention: dtype must be f32/bf16");
  XFH_REQUIRE(!mask || mask_dtype_ok(mask_dtype), "dot_product_attention: bad mask dtype");
  XFH_REQUIRE(!bias || float_dtype(bias_dtype) || bias_dtype == XFH_BIAS_PACKED ||
                  bias_dtype == XFH_BIAS_PACKED_BF16,
              "dot_product_attention: bias must be f32/bf16 or packed");
  AttentionArgs a;
  std::memset(&a, 0, sizeof(a));
  a.q = q; a.k = k; a.v = v; a.o = out;
  a.mask = mask; a.mask_dtype = mask_dtype;
  a.bias = bias; a.bias_dtype = bias_dtype; a.out_dtype = out_dtype;
  XFH_REQUIRE(float_dtype(out_dtype), "dot_product_attention: out dtype must be f32/bf16");
  a.B = shape[0]; a.H = shape[1]; a.Q = shape[2]; a.K = shape[3]; a.D = shape[4]; a.Dv = shape[5];
  for (int i = 0; i < 6; ++i) XFH_REQUIRE(shape[i] >= 0, "dot_product_attention: negative size");
  for (int i = 0; i < 3; ++i) {
    a.qs[i] = strides[i]; a.ks[i] = strides[3 + i]; a.vs[i] = strides[6 + i]; a.os[i] = strides[9 + i];
  }
  for (int i = 0; i < 4; ++i) { a.ms[i] = strides[12 + i]; a.bs[i] = strides[16 + i]; }
  a.scale = scale;
  if (a.B * a.H * a.Q * a.Dv == 0) return XFH_OK;
  XFH_REQUIRE(q && out && (a.K == 0 || (k && v)), "dot_product_attention: null tensor");
  // bf16 with head dims <= 64, a batch-shared bias and a per-(batch entry, key) mask (the
  // single-track and diffusion shapes) run on the triangle-attention kernel given a
  // workspace of xfh_dot_product_attention_workspace_size bytes; the rest, or a call
  // without workspace, on the general kernel.
  if (workspace && mha_supported(a, dtype)) return mha(a, workspace, workspace_bytes, as_stream(stream));
  if (bias && (bias_dtype == XFH_BIAS_PACKED || bias_dtype == XFH_BIAS_PACKED_BF16))
    return fail(XFH_EUNSUPPORTED, "dot_product_attention: a packed bias needs the pipelined kernel "
                                  "(bf16, head dim <= 64, workspace given)");
  return attention(a, dtype, as_stream(stream));
}

int64_t xfh_attention_max_keys(void) { return grid_attention_max_n(); }

int xfh_attention_bias_pack(const void *bias, int dtype, const int64_t *shape, const int64_t *strides,
                            void *packed, void *stream) {
  XFH_REQUIRE(shape && strides, "attention_bias_pack: null shape/strides");
  XFH_REQUIRE(float_dtype(dtype), "attention_bias_pack: dtype must be f32/bf16");
  for (int i = 0; i < 4; ++i) XFH_REQUIRE(shape[i] >= 0, "attention_bias_pack: negative size");
  XFH_REQUIRE(shape[3] <= grid_attention_max_n(), "attention_bias_pack: more keys than the attention kernel takes");
  if (shape[0] * shape[1] * shape[2] * shape[3] == 0) return XFH_OK;
  XFH_REQUIRE(bias && packed, "attention_bias_pack: null tensor");
  return attention_bias_pack(bias, dtype, shape, strides, packed, as_stream(stream));
}

int xfh_attention_operands_size(int64_t B, int64_t T, int64_t H, int64_t Dh, int64_t *sizes) {
  XFH_REQUIRE(sizes && B >= 0 && H >= 0, "attention_operands_size: bad arguments");
  int dp = 0;
  int64_t tpad = 0;
  XFH_TRY(attention_operands_dims(T, Dh, &dp, &tpad));
  sizes[0] = dp;
  sizes[1] = tpad;
  sizes[2] = B * H * T * dp;
  sizes[3] = B * H * tpad * dp;
  sizes[4] = B * H * dp * tpad;
  return XFH_OK;
}

int xfh_attention_project(const void *x, int64_t ldx, const void *w, const float *bias, int64_t B, int64_t T,
                          int64_t K, int64_t H, int64_t Dh, float qscale, void *q, void *k, void *vt, void *gate,
                          void *stream) {
  XFH_REQUIRE(B >= 0 && H > 0 && K > 0 && ldx >= K, "attention_project: bad sizes");
  int dp = 0;
  int64_t tpad = 0;
  XFH_TRY(attention_operands_dims(T, Dh, &dp, &tpad));
  const int64_t c = H * Dh, n = (gate ? 4 : 3) * c, m = B * T;
  XFH_REQUIRE(m < (int64_t(1) << 31) && n < (int64_t(1) << 31) && K < (int64_t(1) << 31),
              "attention_project: sizes must fit in 32 bits");
  if (m == 0) return XFH_OK;
  XFH_REQUIRE(x && w && q && k && vt, "attention_project: null tensor");
  auto al8 = [](const void *p) { return reinterpret_cast<uintptr_t>(p) % 8 == 0; };
  XFH_REQUIRE(al8(q) && al8(k) && al8(vt) && (!gate || al8(gate)), "attention_project: outputs must be 8-byte aligned");
  GemmArgs g = gemm_args(x, ldx, w, K, q, n, m, n, K);
  g.bias = bias;
  g.attn.q = static_cast<bf16 *>(q);
  g.attn.k = static_cast<bf16 *>(k);
  g.attn.vt = static_cast<bf16 *>(vt);
  g.attn.gate = static_cast<bf16 *>(gate);
  g.attn.T = int(T); g.attn.Tpad = int(tpad); g.attn.H = int(H); g.attn.Dh = int(Dh); g.attn.Dp = dp;
  g.attn.qscale = qscale;
  if (!gemm_ring_supported(g, XFH_BF16))
    return fail(XFH_EUNSUPPORTED, "attention_project: needs K % 32 == 0, ldx % 8 == 0 and 16-byte aligned x and w");
  return gemm_ring(g, 1, XFH_BF16, false, as_stream(stream));
}

int xfh_attention_mask_words(const void *mask, int mask_dtype, int64_t mask_stride, int64_t rows, int64_t T,
                             uint64_t *words, void *stream) {
  XFH_REQUIRE(rows >= 0 && T >= 0 && mask_stride >= 0, "attention_mask_words: bad sizes");
  XFH_REQUIRE(!mask || mask_dtype_ok(mask_dtype), "attention_mask_words: bad mask dtype");
  if (rows * T == 0) return XFH_OK;
  XFH_REQUIRE(words, "attention_mask_words: null words");
  return attention_mask_words(mask, mask_dtype, mask_stride, rows, T, words, as_stream(stream));
}

int xfh_attention_operands(const void *q, const void *k, const void *vt, const uint64_t *words, int words_shared,
                           const void *bias, int bias_dtype, const void *gate, void *out, int64_t B, int64_t T,
                           int64_t H, int64_t Dh, void *stream) {
  XFH_REQUIRE(B >= 0 && H > 0, "attention_operands: bad sizes");
  XFH_REQUIRE(bias_dtype == XFH_BIAS_PACKED || bias_dtype == XFH_BIAS_PACKED_BF16,
              "attention_operands: the bias must be packed (XFH_BIAS_PACKED or XFH_BIAS_PACKED_BF16)");
  if (B == 0) return XFH_OK;
  XFH_REQUIRE(q && k && vt && words && bias && out, "attention_operands: null tensor (the bias is required)");
  XFH_REQUIRE(reinterpret_cast<uintptr_t>(out) % 8 == 0 && (!gate || reinterpret_cast<uintptr_t>(gate) % 8 == 0),
              "attention_operands: out and gate must be 8-byte aligned");
  return attention_operands(static_cast<const bf16 *>(q), static_cast<const bf16 *>(k),
                            static_cast<const bf16 *>(vt), words, words_shared != 0, bias,
                            bias_dtype == XFH_BIAS_PACKED_BF16, static_cast<const bf16 *>(gate),
                            static_cast<bf16 *>(out), B, T, H, Dh, as_stream(stream));
}

int xfh_pair_attention_bias(const void *pair, int pair_dtype, int64_t n, int64_t c, const float *ln_w,
                            const float *ln_b, float eps, const void *w, int w_dtype, int64_t heads,
                            void *packed, int out_dtype, void *stream) {
  XFH_REQUIRE(float_dtype(pair_dtype), "pair_attention_bias: pair dtype must be f32/bf16");
  XFH_REQUIRE(float_dtype(out_dtype), "pair_attention_bias: out dtype must be f32/bf16");
  XFH_REQUIRE(w_dtype == XFH_BF16, "pair_attention_bias: the weight must be bf16");
  XFH_REQUIRE(c == 128, "pair_attention_bias: 128 pair channels");
  XFH_REQUIRE(heads > 0 && heads <= pair_bias_max_heads(), "pair_attention_bias: 1..384 heads");
  XFH_REQUIRE(n >= 0 && n <= grid_attention_max_n(), "pair_attention_bias: more keys than the attention kernel takes");
  XFH_REQUIRE(eps >= 0.f, "pair_attention_bias: eps must be nonnegative");
  if (n == 0) return XFH_OK;
  XFH_REQUIRE(pair && w && packed, "pair_attention_bias: null tensor");
  PairBiasArgs a;
  a.pair = pair; a.ln_w = ln_w; a.ln_b = ln_b; a.eps = eps;
  a.w = static_cast<const bf16 *>(w); a.packed = packed; a.packed_bf16 = out_dtype == XFH_BF16;
  a.n = int(n); a.npad = int(align_up(n, 64)); a.heads = int(heads);
  return pair_bias(a, pair_dtype, as_stream(stream));
}

int64_t xfh_triangle_multiplication_workspace_size(int64_t n, int64_t c, int dtype) {
  if (n < 0 || c < 0 || !float_dtype(dtype)) return -1;
  Carver cv(nullptr, 0);
  TriMulPlan p;
  return trimul_carve(cv, p, n, c, dtype, XFH_F32) + 256;
}

int xfh_triangle_multiplication(const void *pair, int pair_dtype, const void *mask, int mask_dtype,
                                int64_t n, int64_t c, int outgoing, const float *left_w,
                                const float *left_b, float left_eps, const void *proj_w,
                                const void *gate_w, const float *center_w, const float *center_b,
                                float center_eps, const void *out_w, const void *gating_w, int dtype,
                                void *out, int out_dtype, int accumulate, void *workspace,
                                int64_t workspace_bytes, void *stream) {
  XFH_REQUIRE(n >= 0 && c > 0, "triangle_multiplication: bad size");
  XFH_REQUIRE(float_dtype(pair_dtype) && float_dtype(dtype) && float_dtype(out_dtype),
              "triangle_multiplication: dtypes must be f32/bf16");
  XFH_REQUIRE(!mask || mask_dtype_ok(mask_dtype), "triangle_multiplication: bad mask dtype");
  XFH_REQUIRE(left_eps >= 0.f && center_eps >= 0.f, "triangle_multiplication: eps must be nonnegative");
  if (n == 0) return XFH_OK;
  XFH_REQUIRE(n * n < (int64_t(1) << 31), "triangle_multiplication: n*n must fit in 32 bits");
  XFH_REQUIRE(pair && out && proj_w && gate_w && out_w && gating_w, "triangle_multiplication: null tensor");
  Carver cv(workspace, workspace_bytes);
  TriMulPlan p;
  const int64_t need = trimul_carve(cv, p, n, c, dtype, out_dtype);
  if (!workspace || need > workspace_bytes)
    return fail(XFH_EWORKSPACE, "triangle_multiplication: workspace too small (need " +
                                    std::to_string(need) + " bytes)");
  hipStream_t s = as_stream(stream);
  const int64_t plane = n * n;
  if (trimul_fast_path(c, dtype)) {
    TriProjectArgs pa;
    pa.pair = pair; pa.mask = mask; pa.mask_dtype = mask_dtype;
    pa.ln_w = left_w; pa.ln_b = left_b; pa.eps = left_eps;
    pa.w_proj = static_cast<const bf16 *>(proj_w); pa.w_gate = static_cast<const bf16 *>(gate_w);
    pa.left = static_cast<bf16 *>(p.left); pa.right = static_cast<bf16 *>(p.right);
    pa.n = int(n); pa.ld = int(contraction_ld(n)); pa.outgoing = outgoing;
    XFH_TRY(trimul_project(pa, pair_dtype, s));
    ContractionArgs ca;
    ca.left = static_cast<const bf16 *>(p.left);
    ca.right = static_cast<const bf16 *>(p.right);
    ca.out = static_cast<bf16 *>(p.contracted);
    ca.n = int(n); ca.ld = int(contraction_ld(n)); ca.channels = int(c);
    XFH_TRY(contraction(ca, s));
    TriOutputArgs oa;
    oa.pair = pair; oa.contracted = static_cast<const bf16 *>(p.contracted);
    oa.ln_in_w = left_w; oa.ln_in_b = left_b; oa.eps_in = left_eps;
    oa.ln_c_w = center_w; oa.ln_c_b = center_b; oa.eps_c = center_eps;
    oa.w_gating = static_cast<const bf16 *>(gating_w); oa.w_out = static_cast<const bf16 *>(out_w);
    oa.out = out; oa.accumulate = accumulate; oa.n = int(n);
    return trimul_output(oa, pair_dtype, out_dtype, s);
  }
  XFH_TRY(layer_norm_rows(pair, pair_dtype, plane, c, left_w, left_b, left_eps, p.normed, dtype, s));
  GemmArgs g = gemm_args(p.normed, c, proj_w, c, p.proj, 2 * c, plane, 2 * c, c);
  XFH_TRY(gemm_nt(g, 1, dtype, dtype, false, s));
  g = gemm_args(p.normed, c, gate_w, c, p.gate, 2 * c, plane, 2 * c, c);
  XFH_TRY(gemm_nt(g, 1, dtype, dtype, false, s));
  XFH_TRY(trimul_gate(p.proj, p.gate, dtype, mask, mask_dtype, n, c, outgoing, p.left, p.right, s));
  // Per-channel contraction: contracted[k] = left[k] right[k]^T, batch = c.
  g = gemm_args(p.left, n, p.right, n, p.contracted, n, n, n, n);
  g.sA = plane; g.sB = plane; g.sC = plane;
  XFH_TRY(gemm_nt(g, c, dtype, dtype, false, s));
  XFH_TRY(layer_norm_planes(p.contracted, dtype, plane, int(c), center_w, center_b, center_eps,
                            p.centered, dtype, s));
  g = gemm_args(p.normed, c, gating_w, c, p.gating, c, plane, c, c);
  XFH_TRY(gemm_nt(g, 1, dtype, out_dtype, false, s));
  g = gemm_args(p.centered, c, out_w, c, out, c, plane, c, c);
  g.aux = p.gating; g.ldaux = c;
  g.epi = accumulate ? XFH_EPI_MUL_SIGMOID_AUX_ACCUMULATE : XFH_EPI_MUL_SIGMOID_AUX;
  return gemm_nt(g, 1, dtype, out_dtype, false, s);
}

int64_t xfh_grid_self_attention_workspace_size(int64_t n, int64_t c, int64_t heads, int dtype) {
  if (n < 0 || c < 0 || heads <= 0 || !float_dtype(dtype)) return -1;
  Carver cv(nullptr, 0);
  GridPlan p;
  return grid_carve(cv, p, n, c, heads, dtype) + 256;
}

int xfh_grid_self_attention(const void *pair, int pair_dtype, const void *mask, int mask_dtype,
                            int64_t n, int64_t c, int64_t heads, int transpose, const float *norm_w,
                            const float *norm_b, float eps, const void *bias_w, const void *q_w,
                            const void *k_w, const void *v_w, const void *gating_w,
                            const void *out_w, int dtype, void *out, int out_dtype, int accumulate,
                            void *workspace, int64_t workspace_bytes, void *stream) {
  XFH_REQUIRE(n >= 0 && c > 0 && heads > 0 && c % heads == 0, "grid_self_attention: bad size");
  XFH_REQUIRE(c / heads <= 64, "grid_self_attention: head dim must be <= 64");
  XFH_REQUIRE(float_dtype(pair_dtype) && float_dtype(dtype) && float_dtype(out_dtype),
              "grid_self_attention: dtypes must be f32/bf16");
  XFH_REQUIRE(!mask || mask_dtype_ok(mask_dtype), "grid_self_attention: bad mask dtype");
  if (n == 0) return XFH_OK;
  XFH_REQUIRE(n * n < (int64_t(1) << 31), "grid_self_attention: n*n must fit in 32 bits");
  XFH_REQUIRE(pair && out && bias_w && q_w && k_w && v_w && gating_w && out_w,
              "grid_self_attention: null tensor");
  Carver cv(workspace, workspace_bytes);
  GridPlan p;
  const int64_t need = grid_carve(cv, p, n, c, heads, dtype);
  if (!workspace || need > workspace_bytes)
    return fail(XFH_EWORKSPACE, "grid_self_attention: workspace too small (need " +
                                    std::to_string(need) + " bytes)");
  hipStream_t s = as_stream(stream);
  const int64_t plane = n * n, es = dsize(dtype), dh = c / heads;
  // Batch row b, position t of the (optionally transposed) grid lives at pair row
  // b*n + t (starting node) or t*n + b (ending node); the output keeps pair rows.
  const int64_t row_b = transpose ? 1 : n, row_t = transpose ? n : 1;
  if (grid_fast_path(n, c, heads, dtype)) {
    const int64_t npad = grid_attention_pad(n);
    GridProjectArgs pa;
    pa.pair = pair; pa.n = int(n); pa.heads = int(heads); pa.transpose = transpose;
    pa.ln_w = norm_w; pa.ln_b = norm_b; pa.eps = eps;
    pa.wq = static_cast<const bf16 *>(q_w); pa.wk = static_cast<const bf16 *>(k_w);
    pa.wv = static_cast<const bf16 *>(v_w); pa.wb = static_cast<const bf16 *>(bias_w);
    pa.mask = mask; pa.mask_dtype = mask_dtype; pa.maskbits = p.maskbits;
    pa.qscale = kLog2e / std::sqrt(float(dh));
    pa.q = static_cast<bf16 *>(p.qh); pa.k = static_cast<bf16 *>(p.kh); pa.vt = static_cast<bf16 *>(p.vt);
    pa.bias = p.bias_t; pa.npad = int(npad);
    XFH_TRY(grid_project(pa, pair_dtype, s));
    GridAttentionArgs ga;
    ga.q = static_cast<const bf16 *>(p.qh);
    ga.k = static_cast<const bf16 *>(p.kh);
    ga.vt = static_cast<const bf16 *>(p.vt);
    ga.bias = p.bias_t;
    ga.maskbits = p.maskbits;
    ga.out = static_cast<bf16 *>(p.attn);
    ga.osb = row_b * c;
    ga.ost = row_t * c;
    ga.ohs = dh;
    ga.B = int(n); ga.H = int(heads); ga.Nq = int(n); ga.N = int(n);
    ga.Npad = int(npad);
    ga.Nblk = ga.Npad / 64;
    ga.mbs = ga.Nblk;
    ga.Dv = int(dh);
    XFH_TRY(grid_attention(ga, s));
    GridOutputArgs oa;
    oa.pair = pair; oa.attn = static_cast<const bf16 *>(p.attn);
    oa.ln_w = norm_w; oa.ln_b = norm_b; oa.eps = eps;
    oa.w_gating = static_cast<const bf16 *>(gating_w); oa.w_out = static_cast<const bf16 *>(out_w);
    oa.out = out; oa.accumulate = accumulate; oa.n = int(n);
    return grid_output(oa, pair_dtype, out_dtype, s);
  }
  XFH_TRY(layer_norm_rows(pair, pair_dtype, plane, c, norm_w, norm_b, eps, p.normed, dtype, s));
  GemmArgs g = gemm_args(p.normed, c, bias_w, c, p.bias, heads, plane, heads, c);
  XFH_TRY(gemm_nt(g, 1, dtype, dtype, false, s));
  // [q | k | v] = LN(z) [Wq; Wk; Wv]^T in one GEMM: the normalised pair is read once for the
  // three projections (each output column is the same dot product as in a GEMM of its own).
  const void *wsrc[4] = {q_w, k_w, v_w, nullptr};
  const int64_t wrows[4] = {c, c, c, 0};
  if (stack_rows(p.wcat, wsrc, wrows, c, int(es), s) == XFH_OK) {
    g = gemm_args(p.normed, c, p.wcat, c, p.qkv, 3 * c, plane, 3 * c, c);
    XFH_TRY(gemm_nt(g, 1, dtype, dtype, false, s));
  } else {                                           // weights not 16-byte stackable
    for (int i = 0; i < 3; ++i) {
      g = gemm_args(p.normed, c, wsrc[i], c, static_cast<char *>(p.qkv) + i * c * es, 3 * c, plane, c, c);
      XFH_TRY(gemm_nt(g, 1, dtype, dtype, false, s));
    }
  }
  AttentionArgs a;
  std::memset(&a, 0, sizeof(a));
  a.q = p.qkv;
  a.k = static_cast<char *>(p.qkv) + c * es;
  a.v = static_cast<char *>(p.qkv) + 2 * c * es;
  a.o = p.attn;
  a.out_dtype = dtype;
  a.B = n; a.H = heads; a.Q = n; a.K = n; a.D = dh; a.Dv = dh;
  const int64_t qkv_ld = 3 * c;
  a.qs[0] = a.ks[0] = a.vs[0] = row_b * qkv_ld;
  a.qs[1] = a.ks[1] = a.vs[1] = dh;
  a.qs[2] = a.ks[2] = a.vs[2] = row_t * qkv_ld;
  a.os[0] = row_b * c; a.os[1] = dh; a.os[2] = row_t * c;
  a.mask = mask; a.mask_dtype = mask_dtype;
  a.ms[0] = n; a.ms[1] = 0; a.ms[2] = 0; a.ms[3] = 1;
  a.bias = p.bias; a.bias_dtype = dtype;
  a.bs[0] = 0; a.bs[1] = 1; a.bs[2] = n * heads; a.bs[3] = heads;
  a.scale = 1.0f / std::sqrt(float(dh));
  // bf16: the pipelined attention kernel on operands repacked from the projections: whole
  // projection rows through LDS (qkv_repack) where the width allows, else mha_prepare's
  // strided reads; the per-query kernel of attention.hip keeps fp32 and the shapes neither takes.
  bool done = false;
  if (p.mha_ws && dtype == XFH_BF16) {
    const int64_t npad = align_up(n, 64), dp = dh <= 16 ? 16 : dh <= 32 ? 32 : 64;
    Carver mc(p.mha_ws, p.mha_bytes);
    bf16 *oq = static_cast<bf16 *>(mc.take(n * heads * n * dp * 2));
    bf16 *ok = static_cast<bf16 *>(mc.take(n * heads * npad * dp * 2));
    bf16 *ovt = static_cast<bf16 *>(mc.take(n * heads * dp * npad * 2));
    float *obias = static_cast<float *>(mc.take(heads * n * npad * 4));
    uint64_t *owords = static_cast<uint64_t *>(mc.take(n * (npad / 64) * 8));
    if (mc.used <= p.mha_bytes &&
        qkv_repack(static_cast<const bf16 *>(p.qkv), qkv_ld, n, n, heads, dh, transpose, kLog2e * a.scale, oq, ok,
                   ovt, s) == XFH_OK) {
      const int64_t shape[4] = {1, heads, n, n}, strides[4] = {0, 1, n * heads, heads};
      XFH_TRY(attention_bias_pack(p.bias, dtype, shape, strides, obias, s));
      XFH_TRY(attention_mask_words(mask, mask_dtype, n, n, n, owords, s));
      GridAttentionArgs ga;
      ga.q = oq; ga.k = ok; ga.vt = ovt; ga.bias = obias; ga.maskbits = owords;
      ga.out = static_cast<bf16 *>(p.attn);
      ga.osb = row_b * c; ga.ost = row_t * c; ga.ohs = dh;
      ga.B = int(n); ga.H = int(heads); ga.Nq = int(n); ga.N = int(n);
      ga.Npad = int(npad); ga.Nblk = int(npad / 64); ga.mbs = ga.Nblk; ga.Dv = int(dh);
      XFH_TRY(mha_attention(ga, int(dp), s));
      done = true;
    }
  }
  if (!done) {
    if (p.mha_ws && mha_supported(a, dtype)) XFH_TRY(mha(a, p.mha_ws, p.mha_bytes, s));
    else XFH_TRY(attention(a, dtype, s));
  }
  // attn <- sigmoid(LN(z) Wgate^T) * attn, in place.
  g = gemm_args(p.normed, c, gating_w, c, p.attn, c, plane, c, c);
  g.epi = XFH_EPI_SIGMOID_MUL_AUX; g.aux = p.attn; g.ldaux = c;
  XFH_TRY(gemm_nt(g, 1, dtype, dtype, false, s));
  g = gemm_args(p.attn, c, out_w, c, out, c, plane, c, c);
  g.epi = accumulate ? XFH_EPI_ACCUMULATE : XFH_EPI_STORE;
  return gemm_nt(g, 1, dtype, out_dtype, false, s);
}

int64_t xfh_transition_workspace_size(int64_t rows, int64_t c, int64_t f, int dtype) {
  if (rows < 0 || c < 0 || f < 0 || !float_dtype(dtype)) return -1;
  const int64_t es = dsize(dtype);
  return align_up(rows * c * es, 256) + align_up(rows * f * es, 256) + 256;
}

int xfh_transition(const void *x, int x_dtype, int64_t rows, int64_t c, int64_t f,
                   const float *norm_w, const float *norm_b, float eps, const void *w1_packed,
                   const void *w2, int dtype, void *out, int out_dtype, int accumulate,
                   void *workspace, int64_t workspace_bytes, void *stream) {
  XFH_REQUIRE(rows >= 0 && c > 0 && f > 0, "transition: bad size");
  XFH_REQUIRE(rows < (int64_t(1) << 31), "transition: rows must fit in 32 bits");
  XFH_REQUIRE(float_dtype(x_dtype) && float_dtype(dtype) && float_dtype(out_dtype),
              "transition: dtypes must be f32/bf16");
  if (rows == 0) return XFH_OK;
  XFH_REQUIRE(x && out && w1_packed && w2, "transition: null tensor");
  if (dtype == XFH_BF16 && c == 128 && f == 512) {
    TransitionArgs ta;
    ta.x = x; ta.rows = rows; ta.ln_w = norm_w; ta.ln_b = norm_b; ta.eps = eps;
    ta.w1 = static_cast<const bf16 *>(w1_packed); ta.w2 = static_cast<const bf16 *>(w2);
    ta.out = out; ta.accumulate = accumulate;
    return transition_fused(ta, x_dtype, out_dtype, as_stream(stream));
  }
  Carver cv(workspace, workspace_bytes);
  const int64_t es = dsize(dtype);
  void *normed = cv.take(rows * c * es);
  void *hidden = cv.take(rows * f * es);
  if (!workspace || cv.used > workspace_bytes)
    return fail(XFH_EWORKSPACE, "transition: workspace too small (need " + std::to_string(cv.used) + " bytes)");
  hipStream_t s = as_stream(stream);
  XFH_TRY(layer_norm_rows(x, x_dtype, rows, c, norm_w, norm_b, eps, normed, dtype, s));
  GemmArgs g = gemm_args(normed, c, w1_packed, c, hidden, f, rows, xfh_glu_packed_rows(f), c);
  g.glu_f = int(f);
  XFH_TRY(gemm_nt(g, 1, dtype, dtype, true, s));
  g = gemm_args(hidden, f, w2, f, out, c, rows, c, f);
  g.epi = accumulate ? XFH_EPI_ACCUMULATE : XFH_EPI_STORE;
  return gemm_nt(g, 1, dtype, out_dtype, false, s);
}

int xfh_transition_pair_bias(void *pair, int64_t n, int64_t c, int64_t f, const float *norm_w,
                             const float *norm_b, float eps, const void *w1_packed, const void *w2,
                             const float *bias_ln_w, const float *bias_ln_b, float bias_eps,
                             const void *bias_w, int64_t heads, float *packed, void *stream) {
  XFH_REQUIRE(n >= 0, "transition_pair_bias: bad size");
  XFH_REQUIRE(c == 128 && f == 512, "transition_pair_bias: 128 pair channels and 512 hidden");
  XFH_REQUIRE(heads > 0 && heads <= 16, "transition_pair_bias: 1..16 heads");
  XFH_REQUIRE(n <= grid_attention_max_n(), "transition_pair_bias: more keys than the attention kernel takes");
  XFH_REQUIRE(eps >= 0.f && bias_eps >= 0.f, "transition_pair_bias: eps must be nonnegative");
  if (n == 0) return XFH_OK;
  XFH_REQUIRE(pair && w1_packed && w2 && bias_w && packed, "transition_pair_bias: null tensor");
  XFH_REQUIRE(reinterpret_cast<uintptr_t>(packed) % 16 == 0, "transition_pair_bias: packed must be 16-byte aligned");
  TransitionArgs ta;
  ta.x = pair; ta.rows = n * n; ta.ln_w = norm_w; ta.ln_b = norm_b; ta.eps = eps;
  ta.w1 = static_cast<const bf16 *>(w1_packed); ta.w2 = static_cast<const bf16 *>(w2);
  ta.out = pair; ta.accumulate = 1;
  TransitionBias tb;
  tb.ln_w = bias_ln_w; tb.ln_b = bias_ln_b; tb.eps = bias_eps; tb.w = static_cast<const bf16 *>(bias_w);
  tb.packed = packed; tb.n = int(n); tb.npad = int(align_up(n, 64)); tb.heads = int(heads);
  return transition_pair_bias(ta, tb, as_stream(stream));
}

}  // extern "C"
