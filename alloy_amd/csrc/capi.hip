// C ABI entry points: argument validation, status codes, dispatch to launchers.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <string>

#include "../../include/alloy_amd.h"
#include "launch.h"
#include "moe.h"

namespace {

thread_local std::string g_err;

alloy_status fail(alloy_status s, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
alloy_status fail(alloy_status s, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return s;
}

alloy_status hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return ALLOY_OK;
  return fail(ALLOY_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

struct FmtInfo {
  const char* name;
  int qk;           // K must be a multiple of this
  int bb;           // bytes per block (GGUF wire) or 0
  int w_align;      // required alignment of the main buffer
};

const FmtInfo kFmt[] = {
    {"q8_0", 32, 34, 4},  {"q5_0", 32, 22, 4},  {"q4_k", 256, 144, 16}, {"q6_k", 256, 210, 4},
    {"mlx_q4", 32, 0, 16}, {"q8_0_split", 32, 0, 16}, {"q5_0_split", 32, 0, 16},
};

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// Validates the weight buffers of `fmt` and fills QArgs.
alloy_status make_args(int fmt, const void* w, const void* aux, const void* scales,
                       const void* biases, int32_t gs, int64_t K, QArgs& a) {
  if (fmt < 0 || fmt > 6) return fail(ALLOY_E_ARG, "unknown format code %d", fmt);
  const FmtInfo& fi = kFmt[fmt];
  if (K <= 0 || K > (1 << 30)) return fail(ALLOY_E_SHAPE, "%s: K=%lld out of range", fi.name, (long long)K);
  if (K % fi.qk) return fail(ALLOY_E_SHAPE, "%s: K=%lld not divisible by %d", fi.name, (long long)K, fi.qk);
  if (!w) return fail(ALLOY_E_ARG, "%s: null weight pointer", fi.name);
  if (!aligned(w, fi.w_align)) return fail(ALLOY_E_ALIGN, "%s: weight buffer not %d-byte aligned", fi.name, fi.w_align);
  a = QArgs{};
  a.w = (const uint8_t*)w;
  a.aux = (const uint8_t*)aux;
  a.s = (const uint16_t*)scales;
  a.b = (const uint16_t*)biases;
  a.K = (int32_t)K;
  a.gs = 32;
  switch (fmt) {
    case alloy::F_Q8_0: case alloy::F_Q5_0: case alloy::F_Q4_K: case alloy::F_Q6_K:
      a.rb = (K / fi.qk) * fi.bb;
      break;
    case alloy::F_MLX:
      if (!scales || !biases) return fail(ALLOY_E_ARG, "mlx_q4: scales and biases are required");
      if (gs <= 0 || K % gs) return fail(ALLOY_E_SHAPE, "mlx_q4: group size %d does not divide K=%lld", gs, (long long)K);
      if (gs % 32) return fail(ALLOY_E_UNSUPPORTED, "mlx_q4: group size %d unsupported (must be a multiple of 32)", gs);
      if (!aligned(scales, 2) || !aligned(biases, 2)) return fail(ALLOY_E_ALIGN, "mlx_q4: scales/biases not 2-byte aligned");
      a.gs = gs;
      a.rb = K / 2;
      break;
    case alloy::F_Q8_0S:
      if (!scales) return fail(ALLOY_E_ARG, "q8_0: scales are required");
      if (!aligned(scales, 2)) return fail(ALLOY_E_ALIGN, "q8_0: scales not 2-byte aligned");
      a.rb = K;
      break;
    case alloy::F_Q5_0S:
      if (!scales || !aux) return fail(ALLOY_E_ARG, "q5_0: qhigh and scales are required");
      if (!aligned(aux, 16)) return fail(ALLOY_E_ALIGN, "q5_0: qhigh not 16-byte aligned");
      if (!aligned(scales, 2)) return fail(ALLOY_E_ALIGN, "q5_0: scales not 2-byte aligned");
      a.rb = K / 2;
      break;
  }
  return ALLOY_OK;
}

alloy_status check_dtype(alloy_dtype d, const char* what) {
  if (d != ALLOY_DT_F32 && d != ALLOY_DT_F16) return fail(ALLOY_E_DTYPE, "%s: unsupported dtype code %d", what, (int)d);
  return ALLOY_OK;
}

}  // namespace

extern "C" {

const char* alloy_last_error(void) { return g_err.c_str(); }
const char* alloy_version(void) { return "alloy_amd 0.1.0 (gfx950)"; }

int64_t alloy_gemm_workspace_bytes(alloy_format fmt, int64_t M, int64_t N, int64_t K) {
  if (M < 2 || M > 65535LL * 128 || N <= 0 || K <= 0) return 0;
  if (M <= 16) return alloy::gemv_workspace_bytes((int)fmt, M, N, K);
  return alloy::gemm_workspace_bytes((int)fmt, M, N, K);
}

alloy_status alloy_qmm(alloy_format fmt, const void* w, const void* aux, const void* scales,
                       const void* biases, int32_t group_size, const void* x, alloy_dtype x_dtype,
                       void* y, alloy_dtype y_dtype, int64_t M, int64_t N, int64_t K,
                       alloy_path path, int64_t opts, void* stream) {
  return alloy_qmm_ws(fmt, w, aux, scales, biases, group_size, x, x_dtype, y, y_dtype, M, N, K, path, opts, nullptr,
                      0, stream);
}

alloy_status alloy_qmm_ws(alloy_format fmt, const void* w, const void* aux, const void* scales,
                          const void* biases, int32_t group_size, const void* x, alloy_dtype x_dtype,
                          void* y, alloy_dtype y_dtype, int64_t M, int64_t N, int64_t K,
                          alloy_path path, int64_t opts, void* ws, int64_t ws_bytes, void* stream) {
  QArgs a;
  alloy_status s = make_args((int)fmt, w, aux, scales, biases, group_size, K, a);
  if (s != ALLOY_OK) return s;
  if ((s = check_dtype(x_dtype, "activations")) != ALLOY_OK) return s;
  if ((s = check_dtype(y_dtype, "output")) != ALLOY_OK) return s;
  if (M < 0 || N < 0) return fail(ALLOY_E_SHAPE, "negative M=%lld or N=%lld", (long long)M, (long long)N);
  if (N > (int64_t)1 << 31) return fail(ALLOY_E_SHAPE, "N=%lld too large", (long long)N);
  if (M == 0 || N == 0) return ALLOY_OK;
  if (!x || !y) return fail(ALLOY_E_ARG, "null activation or output pointer");
  if (!aligned(x, 16)) return fail(ALLOY_E_ALIGN, "activations not 16-byte aligned");
  if (!aligned(y, y_dtype == ALLOY_DT_F32 ? 4 : 2)) return fail(ALLOY_E_ALIGN, "output misaligned");
  alloy::Opts o;
  o.lanes_per_row = (int)(opts & 0xFFF);
  o.grid_cap = (int)((opts >> 12) & 0xFFFF);
  o.row_groups = (int)((opts >> 28) & 0xF);
  o.depth = (int)((opts >> 32) & 0xF);
  o.variant = (int)((opts >> 36) & 0xF);
  o.splits = (int)((opts >> 40) & 0xF);
  if (o.lanes_per_row && (o.lanes_per_row % 16 || o.lanes_per_row > 256))
    return fail(ALLOY_E_ARG, "lanes_per_row %d must be a multiple of 16 in [16, 256]", o.lanes_per_row);
  int p = (int)path;
  if (p == ALLOY_PATH_AUTO) p = (M == 1 && K <= alloy::max_k_dot2((int)fmt)) ? alloy::P_GEMV : (M <= 16 ? alloy::P_GEMV_MFMA : alloy::P_GEMM);
  const bool xf = x_dtype == ALLOY_DT_F32, yf = y_dtype == ALLOY_DT_F32;
  hipStream_t st = (hipStream_t)stream;
  switch (p) {
    case alloy::P_GEMV:
      if (K > alloy::max_k_dot2((int)fmt)) return fail(ALLOY_E_UNSUPPORTED, "v_dot2 GEMV: K=%lld exceeds %lld", (long long)K, (long long)alloy::max_k_dot2((int)fmt));
      if (M > 65535) return fail(ALLOY_E_SHAPE, "v_dot2 GEMV: M=%lld too large", (long long)M);
      return hip_status(alloy::launch_gemv_dot2((int)fmt, a, x, xf, y, yf, M, N, o, st), "gemv_dot2 launch");
    case alloy::P_GEMV_MFMA:
      if (M > 65535 * 16) return fail(ALLOY_E_SHAPE, "MFMA GEMV: M=%lld too large", (long long)M);
      if (ws_bytes < 0 || (ws_bytes > 0 && !ws)) return fail(ALLOY_E_ARG, "bad workspace (%lld bytes)", (long long)ws_bytes);
      return hip_status(alloy::launch_gemv_mfma((int)fmt, a, x, xf, y, yf, M, N, o, st, ws, ws_bytes), "gemv_mfma launch");
    case alloy::P_GEMM:
      if (M > 65535LL * 128) return fail(ALLOY_E_SHAPE, "GEMM: M=%lld too large", (long long)M);
      if (ws_bytes < 0 || (ws_bytes > 0 && !ws)) return fail(ALLOY_E_ARG, "bad workspace (%lld bytes)", (long long)ws_bytes);
      return hip_status(alloy::launch_gemm((int)fmt, a, x, xf, y, yf, M, N, o, ws, ws_bytes, st), "gemm launch");
    default:
      return fail(ALLOY_E_ARG, "unknown path code %d", (int)path);
  }
}

alloy_status alloy_gguf_q4_k_mm(const void* x, alloy_dtype xd, const void* blocks, void* y,
                                alloy_dtype yd, int64_t M, int64_t N, int64_t K, void* stream) {
  return alloy_qmm(ALLOY_FMT_Q4_K, blocks, nullptr, nullptr, nullptr, 0, x, xd, y, yd, M, N, K,
                   ALLOY_PATH_AUTO, 0, stream);
}

alloy_status alloy_gguf_q6_k_mm(const void* x, alloy_dtype xd, const void* packed, void* y,
                                alloy_dtype yd, int64_t M, int64_t N, int64_t K, void* stream) {
  return alloy_qmm(ALLOY_FMT_Q6_K, packed, nullptr, nullptr, nullptr, 0, x, xd, y, yd, M, N, K,
                   ALLOY_PATH_AUTO, 0, stream);
}

alloy_status alloy_gguf_q8_0_mm(const void* x, alloy_dtype xd, const void* qweight,
                                const void* scales, void* y, alloy_dtype yd, int64_t M, int64_t N,
                                int64_t K, void* stream) {
  return alloy_qmm(ALLOY_FMT_Q8_0_SPLIT, qweight, nullptr, scales, nullptr, 0, x, xd, y, yd, M, N,
                   K, ALLOY_PATH_AUTO, 0, stream);
}

alloy_status alloy_gguf_q5_0_mm(const void* x, alloy_dtype xd, const void* qweight,
                                const void* qhigh, const void* scales, void* y, alloy_dtype yd,
                                int64_t M, int64_t N, int64_t K, void* stream) {
  return alloy_qmm(ALLOY_FMT_Q5_0_SPLIT, qweight, qhigh, scales, nullptr, 0, x, xd, y, yd, M, N, K,
                   ALLOY_PATH_AUTO, 0, stream);
}

alloy_status alloy_gguf_q8_0_blocks_mm(const void* x, alloy_dtype xd, const void* blocks, void* y,
                                       alloy_dtype yd, int64_t M, int64_t N, int64_t K,
                                       void* stream) {
  return alloy_qmm(ALLOY_FMT_Q8_0, blocks, nullptr, nullptr, nullptr, 0, x, xd, y, yd, M, N, K,
                   ALLOY_PATH_AUTO, 0, stream);
}

alloy_status alloy_gguf_q5_0_blocks_mm(const void* x, alloy_dtype xd, const void* blocks, void* y,
                                       alloy_dtype yd, int64_t M, int64_t N, int64_t K,
                                       void* stream) {
  return alloy_qmm(ALLOY_FMT_Q5_0, blocks, nullptr, nullptr, nullptr, 0, x, xd, y, yd, M, N, K,
                   ALLOY_PATH_AUTO, 0, stream);
}

alloy_status alloy_mlx_q4_mm(const void* x, alloy_dtype xd, const void* qweight,
                             const void* scales, const void* biases, int32_t gs, void* y,
                             alloy_dtype yd, int64_t M, int64_t N, int64_t K, void* stream) {
  return alloy_qmm(ALLOY_FMT_MLX_Q4, qweight, nullptr, scales, biases, gs, x, xd, y, yd, M, N, K,
                   ALLOY_PATH_AUTO, 0, stream);
}

alloy_status alloy_dequant(alloy_format fmt, const void* w, const void* aux, const void* scales,
                           const void* biases, int32_t gs, void* out, alloy_dtype od, int64_t row0,
                           int64_t nrows, int64_t N, int64_t K, void* stream) {
  QArgs a;
  alloy_status s = make_args((int)fmt, w, aux, scales, biases, gs, K, a);
  if (s != ALLOY_OK) return s;
  if ((s = check_dtype(od, "output")) != ALLOY_OK) return s;
  if (row0 < 0 || nrows < 0 || row0 + nrows > N)
    return fail(ALLOY_E_SHAPE, "rows [%lld, %lld) outside [0, %lld)", (long long)row0, (long long)(row0 + nrows), (long long)N);
  if (nrows == 0) return ALLOY_OK;
  if (!out || !aligned(out, 16)) return fail(ALLOY_E_ALIGN, "output null or not 16-byte aligned");
  return hip_status(alloy::launch_dequant((int)fmt, a, out, od == ALLOY_DT_F16, row0, nrows, (hipStream_t)stream),
                    "dequant launch");
}

alloy_status alloy_moe_router_topk(const float* logits, int32_t* idx, float* weights, int64_t T,
                                   int32_t E, int32_t top_k, void* stream) {
  if (T < 0) return fail(ALLOY_E_SHAPE, "negative T");
  if (E <= 0 || E > alloy::kMoeMaxExperts) return fail(ALLOY_E_UNSUPPORTED, "num_experts %d outside [1, %d]", E, alloy::kMoeMaxExperts);
  if (top_k <= 0 || top_k > E || top_k > alloy::kMoeMaxTopK) return fail(ALLOY_E_SHAPE, "top_k %d invalid for %d experts", top_k, E);
  if (T == 0) return ALLOY_OK;
  if (!logits || !idx || !weights) return fail(ALLOY_E_ARG, "null pointer");
  return hip_status(alloy::launch_router(logits, idx, weights, T, E, top_k, (hipStream_t)stream), "router launch");
}

size_t alloy_moe_workspace_bytes(int64_t T, int32_t E, int32_t top_k, int64_t H, int64_t I) {
  if (T < 0 || E <= 0 || top_k <= 0 || H <= 0 || I <= 0) return 0;
  return alloy::moe_layout(T, E, top_k, H, I).total;
}

alloy_status alloy_mlx_moe_routed(const void* hidden, const float* logits, const void* gu_q,
                                  const void* gu_s, const void* gu_b, const void* dn_q,
                                  const void* dn_s, const void* dn_b, int32_t gs, int32_t E,
                                  int32_t top_k, int64_t T, int64_t H, int64_t I, void* ws,
                                  size_t ws_bytes, float* y, void* stream) {
  if (T < 0) return fail(ALLOY_E_SHAPE, "negative T");
  if (E <= 0 || E > alloy::kMoeMaxExperts) return fail(ALLOY_E_UNSUPPORTED, "num_experts %d outside [1, %d]", E, alloy::kMoeMaxExperts);
  if (top_k <= 0 || top_k > E || top_k > alloy::kMoeMaxTopK) return fail(ALLOY_E_SHAPE, "top_k %d invalid for %d experts", top_k, E);
  if (T * top_k > alloy::kMoeMaxRoutes) return fail(ALLOY_E_UNSUPPORTED, "T*top_k=%lld exceeds %d", (long long)(T * top_k), alloy::kMoeMaxRoutes);
  if (H <= 0 || I <= 0) return fail(ALLOY_E_SHAPE, "H and I must be positive");
  if (gs <= 0 || H % gs || I % gs) return fail(ALLOY_E_SHAPE, "group size %d must divide H=%lld and I=%lld", gs, (long long)H, (long long)I);
  if (gs % 32) return fail(ALLOY_E_UNSUPPORTED, "group size %d unsupported (must be a multiple of 32)", gs);
  if (T == 0) return ALLOY_OK;
  if (!hidden || !logits || !gu_q || !gu_s || !gu_b || !dn_q || !dn_s || !dn_b || !y || !ws)
    return fail(ALLOY_E_ARG, "null pointer");
  if (!aligned(hidden, 16) || !aligned(gu_q, 16) || !aligned(dn_q, 16) || !aligned(ws, 256))
    return fail(ALLOY_E_ALIGN, "hidden/qweights must be 16-byte and workspace 256-byte aligned");
  const alloy::MoeLayout L = alloy::moe_layout(T, E, top_k, H, I);
  if (ws_bytes < L.total) return fail(ALLOY_E_SHAPE, "workspace %zu bytes < required %zu", ws_bytes, L.total);
  alloy::MoeArgs m{};
  m.x = (const f16*)hidden;
  m.logits = logits;
  m.gu = QArgs{(const uint8_t*)gu_q, nullptr, (const uint16_t*)gu_s, (const uint16_t*)gu_b, H / 2, gs, (int32_t)H};
  m.dn = QArgs{(const uint8_t*)dn_q, nullptr, (const uint16_t*)dn_s, (const uint16_t*)dn_b, I / 2, gs, (int32_t)I};
  m.E = E; m.top_k = top_k; m.T = T; m.H = H; m.I = I;
  m.ws = (uint8_t*)ws;
  m.y = y;
  return hip_status(alloy::launch_mlx_moe(m, L, (hipStream_t)stream), "moe launch");
}

alloy_status alloy_embedding(alloy_format fmt, const void* w, const void* aux, const void* scales,
                             const void* biases, int32_t group_size, const void* ids, int32_t ids_int64,
                             int64_t n_ids, int64_t N, int64_t K, float* out, void* stream) {
  QArgs a;
  alloy_status s = make_args((int)fmt, w, aux, scales, biases, group_size, K, a);
  if (s != ALLOY_OK) return s;
  if (n_ids < 0 || N < 0) return fail(ALLOY_E_SHAPE, "negative n_ids=%lld or N=%lld", (long long)n_ids, (long long)N);
  if (n_ids == 0) return ALLOY_OK;
  if (!ids || !out) return fail(ALLOY_E_ARG, "null ids or output pointer");
  if (!aligned(ids, ids_int64 ? 8 : 4)) return fail(ALLOY_E_ALIGN, "ids misaligned");
  if (!aligned(out, 16)) return fail(ALLOY_E_ALIGN, "output not 16-byte aligned");
  return hip_status(alloy::launch_embedding((int)fmt, a, ids, ids_int64 != 0, n_ids, N, out, (hipStream_t)stream),
                    "embedding launch");
}

alloy_status alloy_qmm_batched(alloy_format fmt, int32_t n, const void* const* w, const void* const* aux,
                               const void* const* scales, const void* const* biases, const int64_t* N,
                               int32_t group_size, const void* x, alloy_dtype x_dtype, void* const* y,
                               alloy_dtype y_dtype, int64_t M, int64_t K, void* stream) {
  if (n < 0) return fail(ALLOY_E_ARG, "negative matrix count %d", n);
  if (n == 0) return ALLOY_OK;
  if (!w || !N || !y) return fail(ALLOY_E_ARG, "null pointer table");
  alloy_status s;
  if ((s = check_dtype(x_dtype, "activations")) != ALLOY_OK) return s;
  if ((s = check_dtype(y_dtype, "output")) != ALLOY_OK) return s;
  if (M < 0 || K <= 0) return fail(ALLOY_E_SHAPE, "bad M=%lld or K=%lld", (long long)M, (long long)K);
  const bool xf = x_dtype == ALLOY_DT_F32, yf = y_dtype == ALLOY_DT_F32;
  // one launch per group of up to kMaxBatch matrices (M = 1, wave-row kernel);
  // otherwise (or for a shape that kernel does not take) one alloy_qmm per matrix
  auto single = [&](int i) -> alloy_status {
    return alloy_qmm(fmt, w[i], aux ? aux[i] : nullptr, scales ? scales[i] : nullptr, biases ? biases[i] : nullptr,
                     group_size, x, x_dtype, y[i], y_dtype, M, N[i], K, ALLOY_PATH_AUTO, 0, stream);
  };
  alloy::WaveBatch b{};
  int which[alloy::kMaxBatch];
  auto flush = [&]() -> alloy_status {
    if (b.n == 0) return ALLOY_OK;
    const hipError_t e = alloy::launch_gemv_batched((int)fmt, b, x, xf, yf, alloy::Opts{}, (hipStream_t)stream);
    const int cnt = b.n;
    b.n = 0;
    if (e == hipSuccess) return ALLOY_OK;
    if (e != hipErrorNotSupported) return hip_status(e, "batched gemv launch");
    (void)hipGetLastError();
    for (int k = 0; k < cnt; ++k) {
      const alloy_status r = single(which[k]);
      if (r != ALLOY_OK) return r;
    }
    return ALLOY_OK;
  };
  const bool one_launch = M == 1 && !xf && K <= alloy::max_k_dot2((int)fmt);
  for (int i = 0; i < n; ++i) {
    if (N[i] < 0 || N[i] >= ((int64_t)1 << 31)) return fail(ALLOY_E_SHAPE, "bad N=%lld of matrix %d", (long long)N[i], i);
    if (N[i] == 0 || M == 0) continue;         // (an empty matrix may have no buffer at all)
    QArgs a;
    if ((s = make_args((int)fmt, w[i], aux ? aux[i] : nullptr, scales ? scales[i] : nullptr,
                       biases ? biases[i] : nullptr, group_size, K, a)) != ALLOY_OK) return s;
    if (!x || !y[i]) return fail(ALLOY_E_ARG, "null activation or output pointer");
    if (!aligned(x, 16)) return fail(ALLOY_E_ALIGN, "activations not 16-byte aligned");
    if (!aligned(y[i], yf ? 4 : 2)) return fail(ALLOY_E_ALIGN, "output %d misaligned", i);
    if (!one_launch) {
      if ((s = single(i)) != ALLOY_OK) return s;
      continue;
    }
    which[b.n] = i;
    b.a[b.n] = a;
    b.y[b.n] = y[i];
    b.ldy[b.n] = N[i];
    b.N[b.n] = (int)N[i];
    if (++b.n == alloy::kMaxBatch && (s = flush()) != ALLOY_OK) return s;
  }
  return flush();
}

size_t alloy_glu_workspace_bytes(alloy_format fmt, int64_t M, int64_t N, int64_t K, int32_t group_size,
                                 alloy_dtype x_dtype) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  if (alloy::glu_fused_supported((int)fmt, M, N, K, x_dtype == ALLOY_DT_F32, group_size)) return 0;
  return 2 * (((size_t)M * (size_t)N * 4 + 255) & ~(size_t)255);
}

alloy_status alloy_qmm_glu(alloy_format fmt, alloy_act act, const void* gw, const void* gaux, const void* gsc,
                           const void* gbi, const void* uw, const void* uaux, const void* usc, const void* ubi,
                           int32_t group_size, const void* x, alloy_dtype x_dtype, void* y, alloy_dtype y_dtype,
                           int64_t M, int64_t N, int64_t K, void* ws, size_t ws_bytes, void* stream) {
  if (act != ALLOY_ACT_SILU && act != ALLOY_ACT_GELU_TANH) return fail(ALLOY_E_ARG, "unknown activation code %d", (int)act);
  QArgs g, u;
  alloy_status s = make_args((int)fmt, gw, gaux, gsc, gbi, group_size, K, g);
  if (s != ALLOY_OK) return s;
  if ((s = make_args((int)fmt, uw, uaux, usc, ubi, group_size, K, u)) != ALLOY_OK) return s;
  if ((s = check_dtype(x_dtype, "activations")) != ALLOY_OK) return s;
  if ((s = check_dtype(y_dtype, "output")) != ALLOY_OK) return s;
  if (M < 0 || N < 0) return fail(ALLOY_E_SHAPE, "negative M=%lld or N=%lld", (long long)M, (long long)N);
  if (N > (int64_t)1 << 31) return fail(ALLOY_E_SHAPE, "N=%lld too large", (long long)N);
  if (M == 0 || N == 0) return ALLOY_OK;
  if (!x || !y) return fail(ALLOY_E_ARG, "null activation or output pointer");
  if (!aligned(x, 16)) return fail(ALLOY_E_ALIGN, "activations not 16-byte aligned");
  if (!aligned(y, y_dtype == ALLOY_DT_F32 ? 4 : 2)) return fail(ALLOY_E_ALIGN, "output misaligned");
  const bool xf = x_dtype == ALLOY_DT_F32, yf = y_dtype == ALLOY_DT_F32;
  hipStream_t st = (hipStream_t)stream;
  alloy::Opts o;
  if (alloy::glu_fused_supported((int)fmt, M, N, K, xf, group_size))
    return hip_status(alloy::launch_glu_fused((int)fmt, (int)act, g, u, x, xf, y, yf, M, N, o, st), "fused glu launch");
  const size_t need = alloy_glu_workspace_bytes(fmt, M, N, K, group_size, x_dtype);
  if (!ws || ws_bytes < need) return fail(ALLOY_E_SHAPE, "workspace %zu bytes < required %zu", ws_bytes, need);
  if (!aligned(ws, 256)) return fail(ALLOY_E_ALIGN, "workspace not 256-byte aligned");
  float* gf = (float*)ws;
  float* uf = (float*)((uint8_t*)ws + need / 2);
  s = alloy_qmm(fmt, gw, gaux, gsc, gbi, group_size, x, x_dtype, gf, ALLOY_DT_F32, M, N, K, ALLOY_PATH_AUTO, 0, stream);
  if (s != ALLOY_OK) return s;
  s = alloy_qmm(fmt, uw, uaux, usc, ubi, group_size, x, x_dtype, uf, ALLOY_DT_F32, M, N, K, ALLOY_PATH_AUTO, 0, stream);
  if (s != ALLOY_OK) return s;
  return hip_status(alloy::launch_glu_combine((int)act, gf, uf, y, yf, M * N, st), "glu combine launch");
}

alloy_status alloy_gguf_q4_k_silu(const void* x, alloy_dtype xd, const void* gate_blocks, const void* up_blocks,
                                  void* y, alloy_dtype yd, int64_t M, int64_t N, int64_t K, void* ws,
                                  size_t ws_bytes, void* stream) {
  return alloy_qmm_glu(ALLOY_FMT_Q4_K, ALLOY_ACT_SILU, gate_blocks, nullptr, nullptr, nullptr, up_blocks, nullptr,
                       nullptr, nullptr, 0, x, xd, y, yd, M, N, K, ws, ws_bytes, stream);
}

alloy_status alloy_gguf_q4_k_gelu(const void* x, alloy_dtype xd, const void* gate_blocks, const void* up_blocks,
                                  void* y, alloy_dtype yd, int64_t M, int64_t N, int64_t K, void* ws,
                                  size_t ws_bytes, void* stream) {
  return alloy_qmm_glu(ALLOY_FMT_Q4_K, ALLOY_ACT_GELU_TANH, gate_blocks, nullptr, nullptr, nullptr, up_blocks,
                       nullptr, nullptr, nullptr, 0, x, xd, y, yd, M, N, K, ws, ws_bytes, stream);
}

alloy_status alloy_mlx_q4_silu(const void* x, alloy_dtype xd, const void* gate_qweight, const void* gate_scales,
                               const void* gate_biases, const void* up_qweight, const void* up_scales,
                               const void* up_biases, int32_t gs, void* y, alloy_dtype yd, int64_t M, int64_t N,
                               int64_t K, void* ws, size_t ws_bytes, void* stream) {
  return alloy_qmm_glu(ALLOY_FMT_MLX_Q4, ALLOY_ACT_SILU, gate_qweight, nullptr, gate_scales, gate_biases, up_qweight,
                       nullptr, up_scales, up_biases, gs, x, xd, y, yd, M, N, K, ws, ws_bytes, stream);
}

alloy_status alloy_gguf_q8_0_silu(const void* x, alloy_dtype xd, const void* gate_qweight, const void* gate_scales,
                                  const void* up_qweight, const void* up_scales, void* y, alloy_dtype yd, int64_t M,
                                  int64_t N, int64_t K, void* ws, size_t ws_bytes, void* stream) {
  return alloy_qmm_glu(ALLOY_FMT_Q8_0_SPLIT, ALLOY_ACT_SILU, gate_qweight, nullptr, gate_scales, nullptr, up_qweight,
                       nullptr, up_scales, nullptr, 0, x, xd, y, yd, M, N, K, ws, ws_bytes, stream);
}

alloy_status alloy_gguf_moe_routed(const void* hidden, const float* logits, const void* gate_up_blocks,
                                   const void* down_qweight, int32_t E, int32_t top_k, int64_t T, int64_t H,
                                   int64_t I, void* ws, size_t ws_bytes, float* y, void* stream) {
  if (T < 0) return fail(ALLOY_E_SHAPE, "negative T");
  if (E <= 0 || E > alloy::kMoeMaxExperts) return fail(ALLOY_E_UNSUPPORTED, "num_experts %d outside [1, %d]", E, alloy::kMoeMaxExperts);
  if (top_k <= 0 || top_k > E || top_k > alloy::kMoeMaxTopK) return fail(ALLOY_E_SHAPE, "top_k %d invalid for %d experts", top_k, E);
  if (T * top_k > alloy::kMoeMaxRoutes) return fail(ALLOY_E_UNSUPPORTED, "T*top_k=%lld exceeds %d", (long long)(T * top_k), alloy::kMoeMaxRoutes);
  if (H <= 0 || I <= 0 || H % 256 || I % 256)
    return fail(ALLOY_E_SHAPE, "hidden %lld and moe_intermediate %lld must be positive multiples of 256", (long long)H, (long long)I);
  const alloy::MoeLayout L = alloy::moe_layout(T, E, top_k, H, I);
  if (!alloy::gguf_moe_supported(T, H, I, L))
    return fail(ALLOY_E_UNSUPPORTED, "gguf_moe_routed: H=%lld I=%lld T=%lld beyond the supported sizes (H, I <= 4096)",
                (long long)H, (long long)I, (long long)T);
  if (T == 0) return ALLOY_OK;
  if (!hidden || !logits || !gate_up_blocks || !down_qweight || !y || !ws) return fail(ALLOY_E_ARG, "null pointer");
  if (!aligned(hidden, 16) || !aligned(gate_up_blocks, 16) || !aligned(down_qweight, 2) || !aligned(ws, 256))
    return fail(ALLOY_E_ALIGN, "hidden/gate_up_blocks must be 16-byte, down_qweight 2-byte and workspace 256-byte aligned");
  if (ws_bytes < L.total) return fail(ALLOY_E_SHAPE, "workspace %zu bytes < required %zu", ws_bytes, L.total);
  alloy::MoeArgs m{};
  m.x = (const f16*)hidden;
  m.logits = logits;
  m.gu = QArgs{(const uint8_t*)gate_up_blocks, nullptr, nullptr, nullptr, H / 256 * 144, 32, (int32_t)H};
  m.dn = QArgs{(const uint8_t*)down_qweight, nullptr, nullptr, nullptr, I / 256 * 210, 32, (int32_t)I};
  m.E = E; m.top_k = top_k; m.T = T; m.H = H; m.I = I;
  m.ws = (uint8_t*)ws;
  m.y = y;
  return hip_status(alloy::launch_gguf_moe(m, L, (hipStream_t)stream), "gguf moe launch");
}

// ------------------------------------------------------------------ allocation-free MoE
// The workspace of alloy_gguf_moe_routed_noalloc: a file-scope device array (each GPU
// the library runs on holds its own copy until the process ends).  Host code never
// passes `scratch` itself to a kernel (in host code it names a host-side stand-in);
// it uses the device address hipGetSymbolAddress returns, resolved once per device
// with that device current.  Every call on one GPU shares the array: calls that
// overlap (other streams) race and must be serialized by the caller.  The MoE
// kernels need no zeroed workspace (every region is written before it is read).
}  // extern "C"

namespace {
constexpr size_t kMoeScratchBytes = ALLOY_MOE_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) uint8_t scratch[kMoeScratchBytes];
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];

// device address of this GPU's scratch array (device `dev` current), nullptr on failure
void* scratch_ptr(int dev) {
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (p) return p;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
  g_scratch[dev].store(p, std::memory_order_release);
  return p;
}
}  // namespace

extern "C" {

alloy_status alloy_gguf_moe_routed_noalloc(const void* hidden, const float* logits, const void* gate_up_blocks,
                                           const void* down_qweight, int32_t E, int32_t top_k, int64_t T,
                                           int64_t H, int64_t I, float* y, void* stream) {
  if (T < 0 || E <= 0 || top_k <= 0 || H <= 0 || I <= 0)
    return alloy_gguf_moe_routed(hidden, logits, gate_up_blocks, down_qweight, E, top_k, T, H, I, nullptr, 0, y,
                                 stream);   // the argument errors of the workspace entry point
  if (E <= alloy::kMoeMaxExperts && top_k <= E && top_k <= alloy::kMoeMaxTopK && T * top_k <= alloy::kMoeMaxRoutes) {
    const size_t need = alloy::moe_layout(T, E, top_k, H, I).total;
    if (need > kMoeScratchBytes)
      return fail(ALLOY_E_UNSUPPORTED,
                  "gguf_moe_routed_noalloc: T=%lld needs %zu workspace bytes, beyond the %zu-byte static scratch",
                  (long long)T, need, kMoeScratchBytes);
  }
  if (T == 0) return alloy_gguf_moe_routed(hidden, logits, gate_up_blocks, down_qweight, E, top_k, T, H, I, nullptr,
                                           0, y, stream);
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(ALLOY_E_HIP, "gguf_moe_routed_noalloc: no current device (or device index %d >= %d)", dev, kMaxDevices);
  void* ws = scratch_ptr(dev);
  if (!ws) return fail(ALLOY_E_HIP, "gguf_moe_routed_noalloc: hipGetSymbolAddress of the scratch array failed");
  return alloy_gguf_moe_routed(hidden, logits, gate_up_blocks, down_qweight, E, top_k, T, H, I, ws, kMoeScratchBytes,
                               y, stream);
}

}  // extern "C"
