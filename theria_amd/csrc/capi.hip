// C ABI of libtheria_sdpa.so (declared in include/theria_sdpa.h): argument validation, launch
// sequencing and error reporting. No device memory is allocated here.
#include <atomic>
#include <cmath>
#include <cstdio>
#include <mutex>
#include <string>

#include "../../include/theria_sdpa.h"
#include "sdpa_params.hpp"

#define THERIA_API extern "C" __attribute__((visibility("default")))

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

struct Checker {
  std::string err;
  bool vec = true;
  int vec_elems = 8;
  bool q_rows = true;  // the query-side tensors hold at least one element (B*H*T > 0)
  bool k_rows = true;  // the key-side tensors hold at least one element (B*H*M > 0)
  explicit Checker(const theria::Shape& s)
      : vec_elems(s.dtype == THERIA_DTYPE_F32 ? 4 : 8),
        q_rows((int64_t)s.B * s.H * s.T > 0),
        k_rows((int64_t)s.B * s.H * s.M > 0) {}
  void need(bool ok, const char* msg) {
    if (!ok && err.empty()) err = msg;
  }
  // A tensor with no elements needs no storage: it is only required when its rows exist.
  void qview(const theria_tensor_t* t, const char* name, bool required) { view(t, name, required && q_rows); }
  void kview(const theria_tensor_t* t, const char* name, bool required) { view(t, name, required && k_rows); }
  void view(const theria_tensor_t* t, const char* name, bool required) {
    if (!t || !t->data) {
      if (required && err.empty()) err = std::string(name) + " is required";
      return;
    }
    if (t->stride_b < 0 || t->stride_h < 0 || t->stride_row < 0) {
      if (err.empty()) err = std::string(name) + " has a negative stride";
      return;
    }
    if (reinterpret_cast<uintptr_t>(t->data) % 16 != 0) vec = false;
    if (t->stride_b % vec_elems || t->stride_h % vec_elems || t->stride_row % vec_elems) vec = false;
  }
};

bool shape_from(const theria_sdpa_problem_t* p, theria::Shape& s, std::string& err) {
  if (!p) {
    err = "problem descriptor is NULL";
    return false;
  }
  if (p->dtype < THERIA_DTYPE_F32 || p->dtype > THERIA_DTYPE_BF16) {
    err = "Unsupported dtype (expected float32, float16 or bfloat16)";
    return false;
  }
  if (p->batch < 0 || p->heads < 0 || p->tq < 0 || p->tk < 0) {
    err = "negative batch, heads, tq or tk";
    return false;
  }
  if (p->head_dim < 1 || p->head_dim > 128) {
    err = "head_dim must be in [1, 128]";
    return false;
  }
  if (!(std::isfinite(p->scale) && p->scale > 0.f)) {
    err = "scale must be finite and positive";
    return false;
  }
  s.B = p->batch;
  s.H = p->heads;
  s.T = p->tq;
  s.M = p->tk;
  s.D = p->head_dim;
  s.scale = p->scale;
  s.causal = p->causal != 0;
  s.dtype = p->dtype;
  s.dp = p->head_dim <= 32 ? 32 : (p->head_dim <= 64 ? 64 : 128);
  s.vec = true;
  s.unpaired = false;
  return true;
}

theria::View cv(const theria_tensor_t* t) {
  if (!t || !t->data) return theria::View{nullptr, 0, 0, 0};
  return theria::View{t->data, t->stride_b, t->stride_h, t->stride_row};
}
theria::MutView mv(const theria_tensor_t* t) {
  if (!t || !t->data) return theria::MutView{nullptr, 0, 0, 0};
  return theria::MutView{t->data, t->stride_b, t->stride_h, t->stride_row};
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return THERIA_OK;
  return fail(THERIA_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

bool empty_problem(const theria::Shape& s) { return s.B == 0 || s.H == 0 || s.T == 0; }

}  // namespace

namespace theria {

// Compute units of the current device. The per-device cache is written with the same value by any
// thread that fills it, so concurrent first calls are harmless.
int device_cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < 64) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  if (dev < 64) cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

}  // namespace theria

// Static row workspace of theria_sdpa_bwd_bwd_noalloc: kScratchFloats floats (20 MiB) on every device the
// library runs on, held until the process ends. Its name is only a host-side stand-in; the device address is
// looked up once per device (with that device current) and kept in g_scratch_ptr. The kernels overwrite
// every element they later read (r, t, the row term and the row statistics), so nothing is cleared; two calls that
// overlap on one device race on it.
constexpr int64_t kWsRows = 5;  // row workspace: kWsRows * batch * heads * tq floats
constexpr int64_t kScratchFloats = kWsRows << 20;
static __device__ __align__(256) float scratch[kScratchFloats];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

int scratch_on_current_device(float** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, "theria_sdpa_bwd_bwd_noalloc (hipGetDevice)");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(THERIA_ERR_CONTRACT, "theria_sdpa_bwd_bwd_noalloc: device index beyond " + std::to_string(kMaxDevices));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_status(e, "theria_sdpa_bwd_bwd_noalloc (hipGetSymbolAddress)");
    g_scratch_ptr[dev] = static_cast<float*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return THERIA_OK;
}
}  // namespace

THERIA_API int theria_abi_version(void) { return THERIA_SDPA_ABI_VERSION; }

THERIA_API const char* theria_last_error(void) { return g_last_error.c_str(); }

THERIA_API int theria_sdpa_fwd(const theria_sdpa_problem_t* p, const theria_tensor_t* q, const theria_tensor_t* k,
                               const theria_tensor_t* v, const theria_tensor_t* o, int32_t o_is_f32, float* lse,
                               float* row_max, float* row_sum, void* stream) {
  theria::Shape s;
  std::string err;
  if (!shape_from(p, s, err)) return fail(THERIA_ERR_CONTRACT, err);
  Checker c(s);
  c.qview(q, "q", true);
  c.kview(k, "k", true);
  c.kview(v, "v", true);
  c.qview(o, "o", true);
  c.need(lse != nullptr || !c.q_rows, "lse is required");
  if (o_is_f32 && o && (o->stride_b % 4 || o->stride_h % 4 || o->stride_row % 4)) c.vec = false;
  if (!c.err.empty()) return fail(THERIA_ERR_CONTRACT, c.err);
  s.vec = c.vec;
  if (empty_problem(s)) return THERIA_OK;
  theria::FwdParams fp{};
  fp.s = s;
  fp.q = cv(q);
  fp.k = cv(k);
  fp.v = cv(v);
  fp.o = mv(o);
  fp.o_f32 = o_is_f32 != 0;
  fp.lse = lse;
  fp.row_max = row_max;
  fp.row_sum = row_sum;
  return hip_status(theria::launch_fwd(fp, (hipStream_t)stream), "theria_sdpa_fwd");
}

// The dQ kernel; row_term (theria::RowTerm) says how it obtains the row term it writes to (or reads from) delta.
static int run_dq(const theria::Shape& s, const theria_tensor_t* q, const theria_tensor_t* k,
                  const theria_tensor_t* v, const theria_tensor_t* o, bool o_f32, int row_term,
                  const theria_tensor_t* dout, const float* lse, float* delta,
                  const theria_tensor_t* dq, hipStream_t st, const char* what, float* lse_out = nullptr,
                  float* l2_out = nullptr) {
  theria::DqParams dp{};
  dp.s = s;
  dp.q = cv(q);
  dp.k = cv(k);
  dp.v = cv(v);
  dp.dout = cv(dout);
  dp.o = cv(o);
  dp.o_f32 = o_f32;
  dp.row_term = row_term;
  dp.lse = lse;
  dp.delta = delta;
  dp.dq = mv(dq);
  dp.lse_out = lse_out;
  dp.l2_out = l2_out;
  return hip_status(theria::launch_bwd_dq(dp, st), what);
}

static int run_dkdv(const theria::Shape& s, const theria_tensor_t* q, const theria_tensor_t* k,
                    const theria_tensor_t* v, const theria_tensor_t* dout, const float* lse,
                    const float* delta, const theria_tensor_t* dk, const theria_tensor_t* dv, bool dv_only,
                    hipStream_t st) {
  theria::DkdvParams kp{};
  kp.s = s;
  kp.q = cv(q);
  kp.k = cv(k);
  kp.v = cv(v);
  kp.dout = cv(dout);
  kp.lse = lse;
  kp.delta = delta;
  kp.dk = mv(dk);
  kp.dv = mv(dv);
  kp.dv_only = dv_only;
  return hip_status(theria::launch_bwd_dkdv(kp, st), "theria_sdpa_bwd_dkdv");
}

THERIA_API int theria_sdpa_bwd_dq(const theria_sdpa_problem_t* p, const theria_tensor_t* q, const theria_tensor_t* k,
                                  const theria_tensor_t* v, const theria_tensor_t* o, int32_t o_is_f32,
                                  const theria_tensor_t* dout, const float* lse, float* delta,
                                  const theria_tensor_t* dq, void* stream) {
  theria::Shape s;
  std::string err;
  if (!shape_from(p, s, err)) return fail(THERIA_ERR_CONTRACT, err);
  Checker c(s);
  c.qview(q, "q", true);
  c.kview(k, "k", true);
  c.kview(v, "v", true);
  c.qview(o, "o", false);
  c.qview(dout, "dout", true);
  c.qview(dq, "dq", false);
  c.need(lse != nullptr || !c.q_rows, "lse is required");
  c.need(delta != nullptr || !c.q_rows, "delta is required");
  if (o_is_f32 && o && (o->stride_b % 4 || o->stride_h % 4 || o->stride_row % 4)) c.vec = false;
  if (!c.err.empty()) return fail(THERIA_ERR_CONTRACT, c.err);
  s.vec = c.vec;
  if (!c.q_rows) return THERIA_OK;
  const int rt = (o && o->data) ? theria::kRowFromO : theria::kRowGiven;
  return run_dq(s, q, k, v, o, o_is_f32 != 0, rt, dout, lse, delta, dq, (hipStream_t)stream,
                "theria_sdpa_bwd_dq");
}

THERIA_API int theria_sdpa_bwd_dkdv(const theria_sdpa_problem_t* p, const theria_tensor_t* q,
                                    const theria_tensor_t* k, const theria_tensor_t* v,
                                    const theria_tensor_t* dout, const float* lse,
                                    const float* delta, const theria_tensor_t* dk, const theria_tensor_t* dv,
                                    void* stream) {
  theria::Shape s;
  std::string err;
  if (!shape_from(p, s, err)) return fail(THERIA_ERR_CONTRACT, err);
  Checker c(s);
  c.qview(q, "q", true);
  c.kview(k, "k", true);
  c.kview(v, "v", true);
  c.qview(dout, "dout", true);
  c.kview(dk, "dk", false);
  c.kview(dv, "dv", true);
  c.need(lse != nullptr || !c.q_rows, "lse is required");
  c.need(delta != nullptr || !c.q_rows, "delta is required");
  if (!c.err.empty()) return fail(THERIA_ERR_CONTRACT, c.err);
  s.vec = c.vec;
  if (!c.k_rows) return THERIA_OK;
  return run_dkdv(s, q, k, v, dout, lse, delta, dk, dv, false, (hipStream_t)stream);
}

THERIA_API int theria_sdpa_bwd(const theria_sdpa_problem_t* p, const theria_tensor_t* q, const theria_tensor_t* k,
                               const theria_tensor_t* v, const theria_tensor_t* o, int32_t o_is_f32,
                               const theria_tensor_t* dout, const float* lse,
                               float* delta_out, const theria_tensor_t* dq, const theria_tensor_t* dk,
                               const theria_tensor_t* dv, void* stream) {
  theria::Shape s;
  std::string err;
  if (!shape_from(p, s, err)) return fail(THERIA_ERR_CONTRACT, err);
  Checker c(s);
  c.qview(q, "q", true);
  c.kview(k, "k", true);
  c.kview(v, "v", true);
  c.qview(o, "o", true);
  c.qview(dout, "dout", true);
  c.qview(dq, "dq", false);
  c.kview(dk, "dk", false);
  c.kview(dv, "dv", true);
  c.need(lse != nullptr || !c.q_rows, "lse is required");
  c.need(delta_out != nullptr || !c.q_rows, "delta_out is required");
  if (o_is_f32 && o && (o->stride_b % 4 || o->stride_h % 4 || o->stride_row % 4)) c.vec = false;
  if (!c.err.empty()) return fail(THERIA_ERR_CONTRACT, c.err);
  s.vec = c.vec;
  const hipStream_t st = (hipStream_t)stream;
  if (c.q_rows) {
    int rc = run_dq(s, q, k, v, o, o_is_f32 != 0, theria::kRowFromO, dout, lse, delta_out, dq, st,
                    "theria_sdpa_bwd (dq)");
    if (rc != THERIA_OK) return rc;
  }
  if (!c.k_rows) return THERIA_OK;
  return run_dkdv(s, q, k, v, dout, lse, delta_out, dk, dv, false, st);
}

THERIA_API int theria_sdpa_bwd_from_stats(const theria_sdpa_problem_t* p, const theria_tensor_t* q,
                                          const theria_tensor_t* k, const theria_tensor_t* v,
                                          const theria_tensor_t* dout, const float* lse,
                                          float* delta_out, const theria_tensor_t* dq, const theria_tensor_t* dk,
                                          const theria_tensor_t* dv, int32_t normalize, void* stream) {
  theria::Shape s;
  std::string err;
  if (!shape_from(p, s, err)) return fail(THERIA_ERR_CONTRACT, err);
  const bool dv_only = !(v && v->data) && (int64_t)s.B * s.H * s.M > 0;
  Checker c(s);
  c.qview(q, "q", true);
  c.kview(k, "k", true);
  c.kview(v, "v", false);
  c.qview(dout, "dout", true);
  c.qview(dq, "dq", false);
  c.kview(dk, "dk", false);
  c.kview(dv, "dv", true);
  c.need(lse != nullptr || !c.q_rows, "lse is required");
  c.need(dv_only || delta_out != nullptr || !c.q_rows, "delta_out is required");
  c.need(!dv_only || !((dq && dq->data) || (dk && dk->data)), "dq and dk need v");
  if (!c.err.empty()) return fail(THERIA_ERR_CONTRACT, c.err);
  s.vec = c.vec;
  const hipStream_t st = (hipStream_t)stream;
  if (!dv_only && c.q_rows) {
    // the dQ kernel forms the row term from P(lse) and dP in a first pass over the keys (and dQ when asked)
    const int rt = normalize ? theria::kRowNormalized : theria::kRowFrozen;
    const int rc = run_dq(s, q, k, v, nullptr, false, rt, dout, lse, delta_out, dq, st,
                          "theria_sdpa_bwd_from_stats (dq)");
    if (rc != THERIA_OK) return rc;
  }
  if (!c.k_rows) return THERIA_OK;
  return run_dkdv(s, q, k, v, dout, lse, delta_out, dk, dv, dv_only, st);
}

THERIA_API int theria_sdpa_jvp(const theria_sdpa_problem_t* p, const theria_tensor_t* q, const theria_tensor_t* k,
                               const theria_tensor_t* v, const theria_tensor_t* o, const float* lse,
                               const theria_tensor_t* tq, const theria_tensor_t* tk, const theria_tensor_t* tv,
                               const theria_tensor_t* tout, int32_t normalize, void* stream) {
  theria::Shape s;
  std::string err;
  if (!shape_from(p, s, err)) return fail(THERIA_ERR_CONTRACT, err);
  Checker c(s);
  c.qview(q, "q", true);
  c.kview(k, "k", true);
  c.kview(v, "v", true);
  c.qview(o, "o", false);
  c.qview(tq, "tq", false);
  c.kview(tk, "tk", false);
  c.kview(tv, "tv", false);
  c.qview(tout, "tout", true);
  c.need(lse != nullptr || !c.q_rows, "lse is required");
  if (!c.err.empty()) return fail(THERIA_ERR_CONTRACT, c.err);
  s.vec = c.vec;
  if (empty_problem(s)) return THERIA_OK;
  theria::JvpParams jp{};
  jp.s = s;
  jp.q = cv(q);
  jp.k = cv(k);
  jp.v = cv(v);
  jp.o = cv(o);
  jp.tq = cv(tq);
  jp.tk = cv(tk);
  jp.tv = cv(tv);
  jp.lse = lse;
  jp.tout = mv(tout);
  jp.normalize = normalize != 0;
  // The frozen-stats form rebuilds O from the P it is given; a saved O belongs to the exact stats.
  if (!jp.normalize) jp.o = theria::View{nullptr, 0, 0, 0};
  return hip_status(theria::launch_jvp(jp, (hipStream_t)stream), "theria_sdpa_jvp");
}

// The double backward with its row workspace either given (row_ws) or, for the allocation-free entry point
// (noalloc), the calling device's static scratch array.
static int run_bwd_bwd(const theria_sdpa_problem_t* p, const theria_tensor_t* q, const theria_tensor_t* k,
                       const theria_tensor_t* v, const theria_tensor_t* o, const theria_tensor_t* dout,
                       const float* lse, const float* delta, const theria_tensor_t* gq, const theria_tensor_t* gk,
                       const theria_tensor_t* gv, const theria_tensor_t* out_gq, const theria_tensor_t* out_gk,
                       const theria_tensor_t* out_gv, const theria_tensor_t* out_gdout, float* row_ws, bool noalloc,
                       void* stream) {
  theria::Shape s;
  std::string err;
  if (!shape_from(p, s, err)) return fail(THERIA_ERR_CONTRACT, err);
  Checker c(s);
  c.qview(q, "q", true);
  c.kview(k, "k", true);
  c.kview(v, "v", true);
  c.qview(o, "o", false);
  c.qview(dout, "dout", true);
  c.qview(gq, "gq", false);
  c.kview(gk, "gk", false);
  c.kview(gv, "gv", false);
  c.qview(out_gq, "out_gq", true);
  c.kview(out_gk, "out_gk", true);
  c.kview(out_gv, "out_gv", true);
  c.qview(out_gdout, "out_gdout", true);
  c.need(lse != nullptr || !c.q_rows, "lse is required");
  // the row term is recomputed (below); delta is not read
  (void)delta;
  c.need(noalloc || row_ws != nullptr || !c.q_rows, "row_ws is required");
  if (!c.err.empty()) return fail(THERIA_ERR_CONTRACT, c.err);
  s.vec = c.vec;
  if (s.B == 0 || s.H == 0) return THERIA_OK;
  const hipStream_t st = (hipStream_t)stream;
  const int64_t nrows = (int64_t)s.B * s.H * s.T;
  if (noalloc) {
    if (kWsRows * nrows > kScratchFloats)
      return fail(THERIA_ERR_CONTRACT, "theria_sdpa_bwd_bwd_noalloc: 5 * batch * heads * tq = " +
                                           std::to_string(kWsRows * nrows) + " floats exceeds the static scratch of " +
                                           std::to_string(kScratchFloats) + " (use theria_sdpa_bwd_bwd with row_ws)");
    const int rc = scratch_on_current_device(&row_ws);
    if (rc != THERIA_OK) return rc;
  }
  theria::BwdBwdParams bp{};
  bp.s = s;
  bp.q = cv(q);
  bp.k = cv(k);
  bp.v = cv(v);
  bp.dout = cv(dout);
  bp.gq = cv(gq);
  bp.gk = cv(gk);
  bp.gv = cv(gv);
  bp.lse = lse;
  bp.row_l2 = nullptr;
  bp.r_row = row_ws;
  bp.t_row = row_ws + nrows;
  if (s.dtype == THERIA_DTYPE_F32 && s.T > 0) {
    // float32: a pass over the keys forms each row's own statistics from its float32 scores, m2 = max_j fl(S c),
    // L2 = log2 sum_j exp2(fl(S c) - m2) (c = scale log2 e), and the row term z = sum_j P dP / sum_j P with dP
    // formed from zero. The row and column kernels rebuild P = exp2((fl(S c) - m2) - L2) and dP the same way,
    // so on a row whose probability sits on one key that key's P is exactly 2^-L2 and dP - z, Gam - r, E1 - t
    // are differences of consistently rounded values. P from the forward's lse instead carries the rounding
    // of lse and of S against it (~2e-6 relative at |lse| ~ 30), which those differences amplify: G_Q, G_K, G_V
    // then miss 1e-5 on such rows.
    float* z = row_ws + 2 * nrows;
    float* m2 = row_ws + 3 * nrows;
    float* l2 = row_ws + 4 * nrows;
    const int rc = run_dq(s, q, k, v, nullptr, false, theria::kRowOwnStats, dout, lse, z, nullptr, st,
                          "theria_sdpa_bwd_bwd (row statistics)", m2, l2);
    if (rc != THERIA_OK) return rc;
    bp.delta = z;
    bp.lse = m2;
    bp.row_l2 = l2;
  }
  const bool rows_make_terms = s.dtype != THERIA_DTYPE_F32 && s.T > 0 && theria::bwdbwd_rows_make_row_terms(bp);
  if (rows_make_terms) {
    // 16-bit inputs at head dims up to 64 (LDS-DMA tiles): the key-split row kernel forms the row term and the exact
    // normaliser itself in its first pass (from the forward's lse) and writes them for the column kernel; that
    // pass also forms G_dO, so no JVP launch follows.
    bp.lse_fwd = lse;
    bp.out_gdo = mv(out_gdout);
    bp.z_out = row_ws + 2 * nrows;
    bp.lse_out = row_ws + 3 * nrows;
    bp.delta = bp.z_out;
    bp.lse = bp.lse_out;
  } else if (s.dtype != THERIA_DTYPE_F32 && s.T > 0) {
    // 16-bit inputs: a 16-bit forward's lse comes from rounded probabilities, so P rebuilt from it sums to one
    // only within ~2^-9, and on peaked rows the second-order terms (Gam - r, dP - z, E1 - t) are differences
    // that such a scale error does not cancel from. The row-term pass of the dQ kernel forms the exact
    // normaliser: lse + ln(sum_j P_ij) for the row and column kernels, and z = sum_j P_ij dP_ij / sum_j P_ij in
    // float32 instead of dO . O with the 16-bit O.
    float* rt_delta = row_ws + 2 * nrows;
    float* lse_c = row_ws + 3 * nrows;
    const int rc = run_dq(s, q, k, v, nullptr, false, theria::kRowNormalized, dout, lse, rt_delta, nullptr, st,
                          "theria_sdpa_bwd_bwd (row term)", lse_c);
    if (rc != THERIA_OK) return rc;
    bp.delta = rt_delta;
    bp.lse = lse_c;
  }
  bp.out_gq = mv(out_gq);
  bp.out_gk = mv(out_gk);
  bp.out_gv = mv(out_gv);
  if (s.T > 0) {
    int rc = hip_status(theria::launch_bwdbwd_rows(bp, st), "theria_sdpa_bwd_bwd (rows)");
    if (rc != THERIA_OK) return rc;
  }
  int rc = hip_status(theria::launch_bwdbwd_cols(bp, st), "theria_sdpa_bwd_bwd (cols)");
  if (rc != THERIA_OK || s.T == 0 || rows_make_terms) return rc;
  theria::JvpParams jp{};
  jp.s = s;
  jp.q = cv(q);
  jp.k = cv(k);
  jp.v = cv(v);
  jp.o = cv(o);
  jp.tq = cv(gq);
  jp.tk = cv(gk);
  jp.tv = cv(gv);
  jp.lse = lse;
  jp.tout = mv(out_gdout);
  jp.normalize = true;  // lse is the operator's own: G_dO is the JVP of the exact softmax
  return hip_status(theria::launch_jvp(jp, st), "theria_sdpa_bwd_bwd (dout)");
}

THERIA_API int theria_sdpa_bwd_bwd(const theria_sdpa_problem_t* p, const theria_tensor_t* q, const theria_tensor_t* k,
                                   const theria_tensor_t* v, const theria_tensor_t* o, const theria_tensor_t* dout,
                                   const float* lse, const float* delta, const theria_tensor_t* gq,
                                   const theria_tensor_t* gk, const theria_tensor_t* gv, const theria_tensor_t* out_gq,
                                   const theria_tensor_t* out_gk, const theria_tensor_t* out_gv,
                                   const theria_tensor_t* out_gdout, float* row_ws, void* stream) {
  return run_bwd_bwd(p, q, k, v, o, dout, lse, delta, gq, gk, gv, out_gq, out_gk, out_gv, out_gdout, row_ws, false,
                     stream);
}

THERIA_API int theria_sdpa_bwd_bwd_noalloc(const theria_sdpa_problem_t* p, const theria_tensor_t* q,
                                           const theria_tensor_t* k, const theria_tensor_t* v, const theria_tensor_t* o,
                                           const theria_tensor_t* dout, const float* lse, const float* delta,
                                           const theria_tensor_t* gq, const theria_tensor_t* gk,
                                           const theria_tensor_t* gv, const theria_tensor_t* out_gq,
                                           const theria_tensor_t* out_gk, const theria_tensor_t* out_gv,
                                           const theria_tensor_t* out_gdout, void* stream) {
  return run_bwd_bwd(p, q, k, v, o, dout, lse, delta, gq, gk, gv, out_gq, out_gk, out_gv, out_gdout, nullptr, true,
                     stream);
}

THERIA_API int theria_debug_tile_counts(uint64_t* counts, int32_t reset) {
  if (!counts) return fail(THERIA_ERR_CONTRACT, "theria_debug_tile_counts: counts is NULL");
#ifdef THERIA_TILE_COUNT
  unsigned long long f = 0, q = 0, kv = 0;
  hipError_t e = theria::tile_counts_fwd(&f, reset != 0);
  if (e == hipSuccess) e = theria::tile_counts_bwd(&q, &kv, reset != 0);
  if (e != hipSuccess) return hip_status(e, "theria_debug_tile_counts");
  counts[0] = f;
  counts[1] = q;
  counts[2] = kv;
  return THERIA_OK;
#else
  counts[0] = counts[1] = counts[2] = 0;
  return fail(THERIA_ERR_CONTRACT, "theria_debug_tile_counts: this library was built without tile counters "
                                   "(libtheria_sdpa_tiles.so has them)");
#endif
}

THERIA_API int theria_debug_atomic_probe(float* buf, int64_t n, int32_t reps, int32_t atomic, void* stream) {
  if (!buf || n < 128 * 64 || reps <= 0)
    return fail(THERIA_ERR_CONTRACT, "theria_debug_atomic_probe: needs a buffer of at least 8192 floats and reps > 0");
#ifdef THERIA_TILE_COUNT
  return hip_status(theria::launch_atomic_probe(buf, n, reps, atomic != 0, (hipStream_t)stream),
                    "theria_debug_atomic_probe");
#else
  (void)stream;
  return fail(THERIA_ERR_CONTRACT, "theria_debug_atomic_probe: this library was built without the measurement "
                                   "kernels (libtheria_sdpa_tiles.so has them)");
#endif
}

// Partial-fusion score kernels: the problem's v-related fields are unused; causal must be 0.
static int run_scores(const theria_sdpa_problem_t* p, const theria_tensor_t* q, const theria_tensor_t* k, void* out,
                      bool out_f32, bool softmax, void* stream, const char* what) {
  theria::Shape s;
  std::string err;
  if (!shape_from(p, s, err)) return fail(THERIA_ERR_CONTRACT, err);
  if (s.causal) return fail(THERIA_ERR_CONTRACT, std::string(what) + ": the score kernels have no causal mask");
  Checker c(s);
  c.qview(q, "q", true);
  c.kview(k, "k", true);
  c.need(out != nullptr || !c.q_rows || !c.k_rows, "out is required");
  if (!c.err.empty()) return fail(THERIA_ERR_CONTRACT, c.err);
  s.vec = c.vec;
  if (empty_problem(s) || s.M == 0) return THERIA_OK;
  theria::ScoresParams sp{};
  sp.s = s;
  sp.q = cv(q);
  sp.k = cv(k);
  sp.out = out;
  sp.out_f32 = out_f32;
  sp.softmax = softmax;
  return hip_status(theria::launch_scores(sp, (hipStream_t)stream), what);
}

THERIA_API int theria_qk_scores(const theria_sdpa_problem_t* p, const theria_tensor_t* q, const theria_tensor_t* k,
                                void* out, int32_t out_f32, void* stream) {
  return run_scores(p, q, k, out, out_f32 != 0 || (p && p->dtype == THERIA_DTYPE_F32), false, stream, "theria_qk_scores");
}

THERIA_API int theria_qk_softmax(const theria_sdpa_problem_t* p, const theria_tensor_t* q, const theria_tensor_t* k,
                                 float* probs, void* stream) {
  return run_scores(p, q, k, probs, true, true, stream, "theria_qk_softmax");
}
