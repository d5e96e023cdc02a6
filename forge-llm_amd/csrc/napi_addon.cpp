// forge_napi.node — thin N-API (v8) binding of the C ABI in include/forge_hip.h
// for the JavaScript host (forge-llm_amd/src).  No compute happens here: every
// function converts arguments, calls one fg_* entry point, and turns a
// non-zero status into a thrown JS Error carrying fg_last_error().
//
// Device buffers are N-API externals wrapping {ptr, bytes}.  free(handle)
// returns the memory to the library's caching allocator immediately; a handle
// that is garbage-collected without free() is returned by its finalizer.
#define NAPI_VERSION 8
#include <node_api.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "forge_hip.h"

namespace {

// Externals carry a tag so that a handle of one kind is never read as another.
constexpr uint32_t kBufTag = 0x46474246u;   // device buffer
constexpr uint32_t kPlanTag = 0x4647504cu;  // Adam plan

struct DevBuf {
  uint32_t tag;
  void* ptr;
  size_t bytes;
  bool owned;  // false for views into another buffer
  bool freed;
};

struct PlanBox {
  uint32_t tag;
  fg_adam_plan* plan;
};

bool g_inited = false;

void buf_finalize(napi_env, void* data, void*) {
  DevBuf* b = static_cast<DevBuf*>(data);
  if (b->owned && !b->freed && g_inited) fg_free(b->ptr);
  delete b;
}

// A plan that is garbage-collected returns its table to the allocator (in
// stream order: steps already queued still read it).
void plan_finalize(napi_env, void* data, void*) {
  PlanBox* p = static_cast<PlanBox*>(data);
  if (p->plan && g_inited) fg_adam_plan_destroy(p->plan);
  delete p;
}

napi_value throw_err(napi_env env, const char* what) {
  napi_throw_error(env, "FORGE_HIP", what);
  return nullptr;
}

napi_value check(napi_env env, int rc, const char* fn) {
  if (rc != 0) {
    std::string m = std::string(fn) + ": " + fg_last_error();
    napi_throw_error(env, rc == FG_ERR_ARG ? "FORGE_ARG" : rc == FG_ERR_OOM ? "FORGE_OOM" : "FORGE_HIP", m.c_str());
  }
  return nullptr;
}

napi_value undef(napi_env env) {
  napi_value u;
  napi_get_undefined(env, &u);
  return u;
}

struct Args {
  napi_env env;
  size_t argc = 24;
  napi_value argv[24];
  bool ok = true;
  Args(napi_env e, napi_callback_info info, size_t need) : env(e) {
    napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr);
    if (argc < need) {
      ok = false;
      throw_err(env, "missing arguments");
    }
  }
  bool is_nullish(size_t i) {
    napi_valuetype t;
    napi_typeof(env, argv[i], &t);
    return t == napi_null || t == napi_undefined;
  }
  DevBuf* buf(size_t i) {
    if (is_nullish(i)) return nullptr;
    void* d = nullptr;
    if (napi_get_value_external(env, argv[i], &d) != napi_ok || !d) {
      ok = false;
      throw_err(env, "expected a device buffer handle");
      return nullptr;
    }
    DevBuf* b = static_cast<DevBuf*>(d);
    if (b->tag != kBufTag) {
      ok = false;
      throw_err(env, "expected a device buffer handle");
      return nullptr;
    }
    if (b->freed) {
      ok = false;
      throw_err(env, "device buffer used after free");
      return nullptr;
    }
    return b;
  }
  fg_adam_plan* plan(size_t i) {
    void* d = nullptr;
    if (napi_get_value_external(env, argv[i], &d) != napi_ok || !d ||
        static_cast<PlanBox*>(d)->tag != kPlanTag) {
      ok = false;
      throw_err(env, "expected an Adam plan handle");
      return nullptr;
    }
    return static_cast<PlanBox*>(d)->plan;
  }
  void* ptr(size_t i) {
    DevBuf* b = buf(i);
    return b ? b->ptr : nullptr;
  }
  float* f(size_t i) { return static_cast<float*>(ptr(i)); }
  int32_t* i32p(size_t i) { return static_cast<int32_t*>(ptr(i)); }
  double* dp(size_t i) { return static_cast<double*>(ptr(i)); }
  int32_t i32(size_t i) {
    int32_t v = 0;
    if (napi_get_value_int32(env, argv[i], &v) != napi_ok) ok = false;
    return v;
  }
  int64_t i64(size_t i) {
    double v = 0;
    if (napi_get_value_double(env, argv[i], &v) != napi_ok) ok = false;
    return (int64_t)v;
  }
  double f64(size_t i) {
    double v = 0;
    if (napi_get_value_double(env, argv[i], &v) != napi_ok) ok = false;
    return v;
  }
  bool typed(size_t i, void** data, size_t* bytes) {
    napi_typedarray_type t;
    size_t len = 0, off = 0;
    napi_value ab;
    void* d = nullptr;
    if (napi_get_typedarray_info(env, argv[i], &t, &len, &d, &ab, &off) != napi_ok) {
      ok = false;
      throw_err(env, "expected a TypedArray");
      return false;
    }
    size_t el = 1;
    switch (t) {
      case napi_int16_array: case napi_uint16_array: el = 2; break;
      case napi_int32_array: case napi_uint32_array: case napi_float32_array: el = 4; break;
      case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: el = 8; break;
      default: el = 1;
    }
    *data = d;
    *bytes = len * el;
    return true;
  }
};

napi_value make_buf(napi_env env, void* p, size_t bytes, bool owned) {
  DevBuf* b = new DevBuf{kBufTag, p, bytes, owned, false};
  napi_value ext;
  if (napi_create_external(env, b, buf_finalize, nullptr, &ext) != napi_ok) {
    if (owned) fg_free(p);
    delete b;
    return throw_err(env, "napi_create_external failed");
  }
  return ext;
}

napi_value num(napi_env env, double v) {
  napi_value r;
  napi_create_double(env, v, &r);
  return r;
}

#define FN(name) napi_value name(napi_env env, napi_callback_info info)
#define CALL(expr, fname)                         \
  do {                                            \
    if (!a.ok) return nullptr;                    \
    int rc_ = (expr);                             \
    if (rc_) return check(env, rc_, fname);       \
    return undef(env);                            \
  } while (0)

// ── runtime ──────────────────────────────────────────────────────────────
FN(js_device_count) {
  int n = 0;
  fg_device_count(&n);
  return num(env, n);
}
FN(js_init) {
  Args a(env, info, 1);
  if (!a.ok) return nullptr;
  int rc = fg_init(a.i32(0));
  if (rc) return check(env, rc, "fg_init");
  g_inited = true;
  return undef(env);
}
FN(js_alloc) {
  Args a(env, info, 1);
  if (!a.ok) return nullptr;
  size_t bytes = (size_t)a.i64(0);
  void* p = nullptr;
  int rc = fg_malloc(&p, bytes);
  if (rc) return check(env, rc, "fg_malloc");
  return make_buf(env, p, bytes, true);
}
FN(js_view) {  // view(handle, byteOffset, bytes): non-owning sub-buffer
  Args a(env, info, 3);
  DevBuf* b = a.buf(0);
  if (!a.ok || !b) return nullptr;
  size_t off = (size_t)a.i64(1), bytes = (size_t)a.i64(2);
  if (off + bytes > b->bytes) return throw_err(env, "view exceeds its buffer");
  return make_buf(env, static_cast<char*>(b->ptr) + off, bytes, false);
}
FN(js_free) {
  Args a(env, info, 1);
  DevBuf* b = a.buf(0);
  if (!a.ok || !b) return nullptr;
  b->freed = true;
  if (b->owned) {
    int rc = fg_free(b->ptr);
    if (rc) return check(env, rc, "fg_free");
  }
  return undef(env);
}
FN(js_bytes) {
  Args a(env, info, 1);
  DevBuf* b = a.buf(0);
  if (!a.ok || !b) return nullptr;
  return num(env, (double)b->bytes);
}
FN(js_h2d) {  // h2d(handle, typedArray[, byteOffset])
  Args a(env, info, 2);
  DevBuf* b = a.buf(0);
  void* host;
  size_t bytes;
  if (!a.ok || !b || !a.typed(1, &host, &bytes)) return nullptr;
  size_t off = a.argc > 2 ? (size_t)a.i64(2) : 0;
  if (off + bytes > b->bytes) return throw_err(env, "h2d: source larger than the device buffer");
  CALL(fg_h2d(static_cast<char*>(b->ptr) + off, host, bytes), "fg_h2d");
}
FN(js_d2h) {  // d2h(handle, typedArray[, byteOffset])
  Args a(env, info, 2);
  DevBuf* b = a.buf(0);
  void* host;
  size_t bytes;
  if (!a.ok || !b || !a.typed(1, &host, &bytes)) return nullptr;
  size_t off = a.argc > 2 ? (size_t)a.i64(2) : 0;
  if (off + bytes > b->bytes) return throw_err(env, "d2h: destination larger than the device buffer");
  CALL(fg_d2h(host, static_cast<char*>(b->ptr) + off, bytes), "fg_d2h");
}
FN(js_d2d) {
  Args a(env, info, 3);
  CALL(fg_d2d(a.ptr(0), a.ptr(1), (size_t)a.i64(2)), "fg_d2d");
}
FN(js_zero) {  // zero(handle[, bytes])
  Args a(env, info, 1);
  DevBuf* b = a.buf(0);
  if (!a.ok || !b) return nullptr;
  size_t bytes = a.argc > 1 ? (size_t)a.i64(1) : b->bytes;
  CALL(fg_zero(b->ptr, bytes), "fg_zero");
}
FN(js_sync) {
  Args a(env, info, 0);
  CALL(fg_sync(), "fg_sync");
}
FN(js_read_async) {  // readAsync(handle, bytes) -> ticket
  Args a(env, info, 2);
  void* p = a.ptr(0);
  if (!a.ok) return nullptr;
  int ticket = -1;
  int rc = fg_read_async(p, (size_t)a.i64(1), &ticket);
  if (rc) return check(env, rc, "fg_read_async");
  return num(env, ticket);
}
FN(js_read_wait) {  // readWait(ticket, typedArray) -> bool (false: stale ticket)
  Args a(env, info, 2);
  void* host;
  size_t bytes;
  int32_t t = a.i32(0);
  if (!a.ok || !a.typed(1, &host, &bytes)) return nullptr;
  int rc = fg_read_wait(t, host, bytes);
  napi_value r;
  napi_get_boolean(env, rc == 0, &r);
  return r;
}
FN(js_mem_stats) {
  size_t inuse = 0, cached = 0;
  fg_mem_stats(&inuse, &cached);
  napi_value arr;
  napi_create_array_with_length(env, 2, &arr);
  napi_set_element(env, arr, 0, num(env, (double)inuse));
  napi_set_element(env, arr, 1, num(env, (double)cached));
  return arr;
}
FN(js_empty_cache) {
  Args a(env, info, 0);
  CALL(fg_empty_cache(), "fg_empty_cache");
}
void ev_finalize(napi_env, void* data, void*) {
  if (g_inited) fg_event_destroy(data);
}
FN(js_event_create) {
  void* ev = nullptr;
  int rc = fg_event_create(&ev);
  if (rc) return check(env, rc, "fg_event_create");
  napi_value ext;
  napi_create_external(env, ev, ev_finalize, nullptr, &ext);
  return ext;
}
FN(js_event_record) {
  Args a(env, info, 1);
  void* ev = nullptr;
  napi_get_value_external(env, a.argv[0], &ev);
  CALL(fg_event_record(ev), "fg_event_record");
}
FN(js_event_elapsed) {
  Args a(env, info, 2);
  void *e0 = nullptr, *e1 = nullptr;
  napi_get_value_external(env, a.argv[0], &e0);
  napi_get_value_external(env, a.argv[1], &e1);
  float ms = 0;
  int rc = fg_event_elapsed_ms(e0, e1, &ms);
  if (rc) return check(env, rc, "fg_event_elapsed_ms");
  return num(env, ms);
}
FN(js_kprof_enable) {
  Args a(env, info, 1);
  CALL(fg_kprof_enable(a.i32(0)), "fg_kprof_enable");
}
FN(js_kprof_reset) {
  Args a(env, info, 0);
  CALL(fg_kprof_reset(), "fg_kprof_reset");
}
FN(js_kprof_report) {
  std::vector<char> buf(1 << 20);
  int rc = fg_kprof_report(buf.data(), buf.size());
  if (rc) return check(env, rc, "fg_kprof_report");
  napi_value s;
  napi_create_string_utf8(env, buf.data(), NAPI_AUTO_LENGTH, &s);
  return s;
}

// ── ops ──────────────────────────────────────────────────────────────────
// The GEMM ops take the operand-maxima buffers of the *_p entry points as
// optional trailing arguments (xpA, xpB[, xpC], have).
FN(js_matmulT_fwd) {  // matmulTFwd(Y, X, W, M, K, N[, xpX, xpW, have])
  Args a(env, info, 6);
  if (a.argc >= 9)
    CALL(fg_matmulT_fwd_p(a.f(0), a.f(1), a.f(2), a.i32(3), a.i32(4), a.i32(5), a.f(6), a.f(7), a.i32(8)),
         "fg_matmulT_fwd");
  CALL(fg_matmulT_fwd(a.f(0), a.f(1), a.f(2), a.i32(3), a.i32(4), a.i32(5)), "fg_matmulT_fwd");
}
FN(js_matmulT_bwd_x) {  // matmulTBwdX(gX, gY, W, M, K, N, beta[, xpG, xpW, have])
  Args a(env, info, 7);
  if (a.argc >= 10)
    CALL(fg_matmulT_bwd_x_p(a.f(0), a.f(1), a.f(2), a.i32(3), a.i32(4), a.i32(5), a.i32(6), a.f(7), a.f(8),
                            a.i32(9)),
         "fg_matmulT_bwd_x");
  CALL(fg_matmulT_bwd_x(a.f(0), a.f(1), a.f(2), a.i32(3), a.i32(4), a.i32(5), a.i32(6)), "fg_matmulT_bwd_x");
}
FN(js_matmulT_fwd_swiglu) {  // matmulTFwdSwiglu(O, GU, X, Wgu, M, K, H[, xpX, xpW, have])
  Args a(env, info, 7);
  if (a.argc >= 10)
    CALL(fg_matmulT_fwd_swiglu_p(a.f(0), a.f(1), a.f(2), a.f(3), a.i32(4), a.i32(5), a.i32(6), a.f(7), a.f(8),
                                 a.i32(9)),
         "fg_matmulT_fwd_swiglu");
  CALL(fg_matmulT_fwd_swiglu(a.f(0), a.f(1), a.f(2), a.f(3), a.i32(4), a.i32(5), a.i32(6)), "fg_matmulT_fwd_swiglu");
}
FN(js_matmulT_bwd_x_pieces) {  // matmulTBwdXPieces(M, K, N) -> K pieces of fg_matmulT_bwd_x
  Args a(env, info, 3);
  if (!a.ok) return nullptr;
  const int p = fg_matmulT_bwd_x_pieces(a.i32(0), a.i32(1), a.i32(2));
  if (p < 0) return check(env, p, "fg_matmulT_bwd_x_pieces");
  return num(env, p);
}
FN(js_matmulT_bwd_x_halves) {  // matmulTBwdXHalves(gXhalves, gY, W, M, K, N[, xpG, xpW, have])
  Args a(env, info, 6);
  if (a.argc >= 9)
    CALL(fg_matmulT_bwd_x_halves_p(a.f(0), a.f(1), a.f(2), a.i32(3), a.i32(4), a.i32(5), a.f(6), a.f(7), a.i32(8)),
         "fg_matmulT_bwd_x_halves");
  CALL(fg_matmulT_bwd_x_halves(a.f(0), a.f(1), a.f(2), a.i32(3), a.i32(4), a.i32(5)), "fg_matmulT_bwd_x_halves");
}
FN(js_matmulT_bwd_w) {  // matmulTBwdW(gW, gY, X, M, K, N, beta[, xpG, xpX, have])
  Args a(env, info, 7);
  if (a.argc >= 10)
    CALL(fg_matmulT_bwd_w_p(a.f(0), a.f(1), a.f(2), a.i32(3), a.i32(4), a.i32(5), a.i32(6), a.f(7), a.f(8),
                            a.i32(9)),
         "fg_matmulT_bwd_w");
  CALL(fg_matmulT_bwd_w(a.f(0), a.f(1), a.f(2), a.i32(3), a.i32(4), a.i32(5), a.i32(6)), "fg_matmulT_bwd_w");
}
FN(js_matmulT_bwd) {  // matmulTBwd(gX, bx, gW, bw, gY, X, W, M, K, N[, xpG, xpX, xpW, have])
  Args a(env, info, 10);
  if (a.argc >= 14)
    CALL(fg_matmulT_bwd_p(a.f(0), a.i32(1), a.f(2), a.i32(3), a.f(4), a.f(5), a.f(6), a.i32(7), a.i32(8), a.i32(9),
                          a.f(10), a.f(11), a.f(12), a.i32(13)),
         "fg_matmulT_bwd");
  CALL(fg_matmulT_bwd(a.f(0), a.i32(1), a.f(2), a.i32(3), a.f(4), a.f(5), a.f(6), a.i32(7), a.i32(8), a.i32(9)),
       "fg_matmulT_bwd");
}
FN(js_matmulT_fwd_resid) {  // matmulTFwdResid(Y, R, X, W, M, K, N[, xpX, xpW, have])
  Args a(env, info, 7);
  if (a.argc >= 10)
    CALL(fg_matmulT_fwd_resid_p(a.f(0), a.f(1), a.f(2), a.f(3), a.i32(4), a.i32(5), a.i32(6), a.f(7), a.f(8),
                                a.i32(9)),
         "fg_matmulT_fwd_resid");
  CALL(fg_matmulT_fwd_resid(a.f(0), a.f(1), a.f(2), a.f(3), a.i32(4), a.i32(5), a.i32(6)), "fg_matmulT_fwd_resid");
}
FN(js_matmulT_fwd_rope) {  // matmulTFwdRope(Y, X, W, M, K, N, cos, sin, npos, nH, nKV, dH, pos0, posStride[, xpX, xpW, have])
  Args a(env, info, 14);
  if (a.argc >= 17)
    CALL(fg_matmulT_fwd_rope_p(a.f(0), a.f(1), a.f(2), a.i32(3), a.i32(4), a.i32(5), a.dp(6), a.dp(7), a.i32(8),
                               a.i32(9), a.i32(10), a.i32(11), a.i32(12), a.i32(13), a.f(14), a.f(15), a.i32(16)),
         "fg_matmulT_fwd_rope");
  CALL(fg_matmulT_fwd_rope(a.f(0), a.f(1), a.f(2), a.i32(3), a.i32(4), a.i32(5), a.dp(6), a.dp(7), a.i32(8),
                           a.i32(9), a.i32(10), a.i32(11), a.i32(12), a.i32(13)),
       "fg_matmulT_fwd_rope");
}
FN(js_attn_fwd_qkv) {  // attnFwdQkv(O, lse, qkv, B, T, nH, nKV, dH[, xpQkv])
  Args a(env, info, 8);
  CALL(fg_attn_fwd_qkv_p(a.f(0), a.f(1), a.f(2), a.i32(3), a.i32(4), a.i32(5), a.i32(6), a.i32(7),
                         a.argc >= 9 ? a.f(8) : nullptr),
       "fg_attn_fwd_qkv");
}
FN(js_attn_bwd_qkv) {  // attnBwdQkv(gqkv, dO, qkv, O, lse, B, T, nH, nKV, dH, cos, sin, npos, pos0, posStride[, xpQkv])
  Args a(env, info, 15);
  CALL(fg_attn_bwd_qkv_p(a.f(0), a.f(1), a.f(2), a.f(3), a.f(4), a.i32(5), a.i32(6), a.i32(7), a.i32(8), a.i32(9),
                         a.dp(10), a.dp(11), a.i32(12), a.i32(13), a.i32(14), a.argc >= 16 ? a.f(15) : nullptr),
       "fg_attn_bwd_qkv");
}
FN(js_attn_fwd) {
  Args a(env, info, 10);
  CALL(fg_attn_fwd(a.f(0), a.f(1), a.f(2), a.f(3), a.f(4), a.i32(5), a.i32(6), a.i32(7), a.i32(8), a.i32(9)),
       "fg_attn_fwd");
}
FN(js_attn_bwd) {
  Args a(env, info, 17);
  CALL(fg_attn_bwd(a.f(0), a.i32(1), a.f(2), a.i32(3), a.f(4), a.i32(5), a.f(6), a.f(7), a.f(8), a.f(9), a.f(10),
                   a.f(11), a.i32(12), a.i32(13), a.i32(14), a.i32(15), a.i32(16)),
       "fg_attn_bwd");
}
FN(js_ce_fwd) {
  Args a(env, info, 6);
  CALL(fg_ce_fwd(a.f(0), a.f(1), a.f(2), a.i32p(3), a.i32(4), a.i32(5)), "fg_ce_fwd");
}
FN(js_ce_fwd_bwd) {  // ceFwdBwd(loss, lse, dlogits, logits, targets, rows, V[, xpGrad])
  Args a(env, info, 7);
  CALL(fg_ce_fwd_bwd_p(a.f(0), a.f(1), a.f(2), a.f(3), a.i32p(4), a.i32(5), a.i32(6), a.argc >= 8 ? a.f(7) : nullptr),
       "fg_ce_fwd_bwd");
}
FN(js_ce_bwd) {  // ceBwd(dlogits, logits, lse, targets, gloss, rows, V, beta[, xpGrad])
  Args a(env, info, 8);
  CALL(fg_ce_bwd_p(a.f(0), a.f(1), a.f(2), a.i32p(3), a.f(4), a.i32(5), a.i32(6), a.i32(7),
                   a.argc >= 9 ? a.f(8) : nullptr),
       "fg_ce_bwd");
}
FN(js_rmsnorm_fwd) {
  Args a(env, info, 7);
  CALL(fg_rmsnorm_fwd(a.f(0), a.f(1), a.f(2), a.f(3), a.i32(4), a.i32(5), a.f64(6)), "fg_rmsnorm_fwd");
}
FN(js_rmsnorm_bwd_from) {  // rmsnormBwdFrom(gX, gXin|null, gw|null, beta_w, g, X, w, inv, T, D)
  Args a(env, info, 10);
  CALL(fg_rmsnorm_bwd_from(a.f(0), a.f(1), a.f(2), a.i32(3), a.f(4), a.f(5), a.f(6), a.f(7), a.i32(8), a.i32(9)),
       "fg_rmsnorm_bwd_from");
}
FN(js_rmsnorm_bwd_from_halves) {  // rmsnormBwdFromHalves(gX, gXin|null, gw|null, beta_w, gHalves, X, w, inv, T, D)
  Args a(env, info, 10);
  CALL(fg_rmsnorm_bwd_from_halves(a.f(0), a.f(1), a.f(2), a.i32(3), a.f(4), a.f(5), a.f(6), a.f(7), a.i32(8),
                                  a.i32(9)),
       "fg_rmsnorm_bwd_from_halves");
}
FN(js_rmsnorm_bwd_parts) {  // rmsnormBwdParts(T, D) -> rows of the deferred form's partial matrix (0: none)
  Args a(env, info, 2);
  if (!a.ok) return nullptr;
  const int p = fg_rmsnorm_bwd_parts(a.i32(0), a.i32(1));
  if (p < 0) return check(env, p, "fg_rmsnorm_bwd_parts");
  return num(env, p);
}
FN(js_rmsnorm_bwd_partial) {  // rmsnormBwdPartial(gX, gXin|null, partial, g, gHalves(0/1), X, w, inv, T, D)
  Args a(env, info, 10);
  CALL(fg_rmsnorm_bwd_partial(a.f(0), a.f(1), a.f(2), a.f(3), a.i32(4), a.f(5), a.f(6), a.f(7), a.i32(8), a.i32(9)),
       "fg_rmsnorm_bwd_partial");
}
// colsumGrouped([[out, partial, rows, n, beta], ...])
FN(js_colsum_grouped) {
  Args a(env, info, 1);
  if (!a.ok) return nullptr;
  uint32_t len = 0;
  if (napi_get_array_length(env, a.argv[0], &len) != napi_ok) return throw_err(env, "colsumGrouped: expected an array");
  std::vector<fg_colsum_job> jobs(len);
  for (uint32_t i = 0; i < len; ++i) {
    napi_value row;
    napi_get_element(env, a.argv[0], i, &row);
    napi_value el[5];
    for (uint32_t k = 0; k < 5; ++k) napi_get_element(env, row, k, &el[k]);
    void* ptrs[2];
    for (int k = 0; k < 2; ++k) {
      void* d = nullptr;
      if (napi_get_value_external(env, el[k], &d) != napi_ok || !d || static_cast<DevBuf*>(d)->tag != kBufTag)
        return throw_err(env, "colsumGrouped: bad handle");
      DevBuf* b = static_cast<DevBuf*>(d);
      if (b->freed) return throw_err(env, "colsumGrouped: buffer used after free");
      ptrs[k] = b->ptr;
    }
    int32_t v[3];
    for (int k = 0; k < 3; ++k) napi_get_value_int32(env, el[2 + k], &v[k]);
    jobs[i].out = static_cast<float*>(ptrs[0]);
    jobs[i].partial = static_cast<const float*>(ptrs[1]);
    jobs[i].rows = v[0]; jobs[i].n = v[1]; jobs[i].beta = v[2];
  }
  CALL(fg_colsum_grouped(jobs.data(), (int)len), "fg_colsum_grouped");
}
// matmulTBwdWGrouped([[gW, gY, X, M, K, N, beta[, xpG, xpX]], ...])
FN(js_matmulT_bwd_w_grouped) {
  Args a(env, info, 1);
  if (!a.ok) return nullptr;
  uint32_t len = 0;
  if (napi_get_array_length(env, a.argv[0], &len) != napi_ok) return throw_err(env, "matmulTBwdWGrouped: expected an array");
  std::vector<fg_wgrad_job> jobs(len);
  for (uint32_t i = 0; i < len; ++i) {
    napi_value row;
    napi_get_element(env, a.argv[0], i, &row);
    uint32_t rl = 0;
    napi_get_array_length(env, row, &rl);
    napi_value el[9];
    for (uint32_t k = 0; k < 9; ++k) {
      if (k < rl) napi_get_element(env, row, k, &el[k]);
      else napi_get_null(env, &el[k]);
    }
    void* ptrs[3];
    for (int k = 0; k < 3; ++k) {
      void* d = nullptr;
      if (napi_get_value_external(env, el[k], &d) != napi_ok || !d || static_cast<DevBuf*>(d)->tag != kBufTag)
        return throw_err(env, "matmulTBwdWGrouped: bad handle");
      DevBuf* b = static_cast<DevBuf*>(d);
      if (b->freed) return throw_err(env, "matmulTBwdWGrouped: buffer used after free");
      ptrs[k] = b->ptr;
    }
    int32_t v[4];
    for (int k = 0; k < 4; ++k) napi_get_value_int32(env, el[3 + k], &v[k]);
    jobs[i].gW = static_cast<float*>(ptrs[0]);
    jobs[i].gY = static_cast<const float*>(ptrs[1]);
    jobs[i].X = static_cast<const float*>(ptrs[2]);
    jobs[i].M = v[0]; jobs[i].K = v[1]; jobs[i].N = v[2]; jobs[i].beta = v[3];
    // optional operand maxima (as filled by the *_p forms), null: computed
    const float* xp[2] = {nullptr, nullptr};
    for (int k = 0; k < 2; ++k) {
      napi_valuetype ty;
      napi_typeof(env, el[7 + k], &ty);
      if (ty == napi_null || ty == napi_undefined) continue;
      void* d = nullptr;
      if (napi_get_value_external(env, el[7 + k], &d) != napi_ok || !d || static_cast<DevBuf*>(d)->tag != kBufTag)
        return throw_err(env, "matmulTBwdWGrouped: bad maxima handle");
      DevBuf* b = static_cast<DevBuf*>(d);
      if (b->freed) return throw_err(env, "matmulTBwdWGrouped: buffer used after free");
      xp[k] = static_cast<const float*>(b->ptr);
    }
    jobs[i].xp_gy = xp[0];
    jobs[i].xp_x = xp[1];
  }
  CALL(fg_matmulT_bwd_w_grouped(jobs.data(), (int)len), "fg_matmulT_bwd_w_grouped");
}
FN(js_rmsnorm_bwd) {
  Args a(env, info, 10);
  CALL(fg_rmsnorm_bwd(a.f(0), a.i32(1), a.f(2), a.i32(3), a.f(4), a.f(5), a.f(6), a.f(7), a.i32(8), a.i32(9)),
       "fg_rmsnorm_bwd");
}
FN(js_rope_table) {  // ropeTable(cosF64, sinF64, npos, dHead, theta) — host
  Args a(env, info, 5);
  void *c, *s;
  size_t cb, sb;
  if (!a.ok || !a.typed(0, &c, &cb) || !a.typed(1, &s, &sb)) return nullptr;
  int npos = a.i32(2), dh = a.i32(3);
  if ((size_t)npos * (dh / 2) * 8 > cb || (size_t)npos * (dh / 2) * 8 > sb) return throw_err(env, "ropeTable: arrays too small");
  CALL(fg_rope_table(static_cast<double*>(c), static_cast<double*>(s), npos, dh, a.f64(4)), "fg_rope_table");
}
FN(js_rope_fwd) {
  Args a(env, info, 10);
  CALL(fg_rope_fwd(a.f(0), a.f(1), a.dp(2), a.dp(3), a.i32(4), a.i32(5), a.i32(6), a.i32(7), a.i32(8), a.i32(9)),
       "fg_rope_fwd");
}
FN(js_rope_bwd) {
  Args a(env, info, 11);
  CALL(fg_rope_bwd(a.f(0), a.f(1), a.dp(2), a.dp(3), a.i32(4), a.i32(5), a.i32(6), a.i32(7), a.i32(8), a.i32(9),
                   a.i32(10)),
       "fg_rope_bwd");
}
FN(js_qkv_rope_fwd) {
  Args a(env, info, 13);
  CALL(fg_qkv_rope_fwd(a.f(0), a.f(1), a.f(2), a.f(3), a.dp(4), a.dp(5), a.i32(6), a.i32(7), a.i32(8), a.i32(9),
                       a.i32(10), a.i32(11), a.i32(12)),
       "fg_qkv_rope_fwd");
}
FN(js_qkv_rope_bwd) {
  Args a(env, info, 14);
  CALL(fg_qkv_rope_bwd(a.f(0), a.f(1), a.f(2), a.f(3), a.dp(4), a.dp(5), a.i32(6), a.i32(7), a.i32(8), a.i32(9),
                       a.i32(10), a.i32(11), a.i32(12), a.i32(13)),
       "fg_qkv_rope_bwd");
}
FN(js_swiglu_gu_fwd) {
  Args a(env, info, 4);
  CALL(fg_swiglu_gu_fwd(a.f(0), a.f(1), a.i32(2), a.i32(3)), "fg_swiglu_gu_fwd");
}
FN(js_swiglu_gu_bwd) {
  Args a(env, info, 6);
  if (a.argc >= 7)
    CALL(fg_swiglu_gu_bwd_p(a.f(0), a.i32(1), a.f(2), a.f(3), a.i32(4), a.i32(5), a.f(6)), "fg_swiglu_gu_bwd_p");
  CALL(fg_swiglu_gu_bwd(a.f(0), a.i32(1), a.f(2), a.f(3), a.i32(4), a.i32(5)), "fg_swiglu_gu_bwd");
}
FN(js_swiglu_fwd) {
  Args a(env, info, 4);
  CALL(fg_swiglu_fwd(a.f(0), a.f(1), a.f(2), a.i64(3)), "fg_swiglu_fwd");
}
FN(js_swiglu_bwd) {
  Args a(env, info, 8);
  CALL(fg_swiglu_bwd(a.f(0), a.i32(1), a.f(2), a.i32(3), a.f(4), a.f(5), a.f(6), a.i64(7)), "fg_swiglu_bwd");
}
FN(js_embed_fwd) {
  Args a(env, info, 6);
  CALL(fg_embed_fwd(a.f(0), a.f(1), a.i32p(2), a.i32(3), a.i32(4), a.i32(5)), "fg_embed_fwd");
}
FN(js_embed_plan) {  // embedPlan(idsInt32, V, perm, segStart, segId) -> nseg  (host)
  Args a(env, info, 5);
  void *ids, *perm, *ss, *sid;
  size_t ib, pb, sb, db;
  if (!a.ok || !a.typed(0, &ids, &ib) || !a.typed(2, &perm, &pb) || !a.typed(3, &ss, &sb) || !a.typed(4, &sid, &db))
    return nullptr;
  int T = (int)(ib / 4);
  if (pb < ib || sb < ib + 4 || db < ib) return throw_err(env, "embedPlan: output arrays too small");
  int nseg = 0;
  int rc = fg_embed_plan(static_cast<int32_t*>(ids), T, a.i32(1), static_cast<int32_t*>(perm),
                         static_cast<int32_t*>(ss), static_cast<int32_t*>(sid), &nseg);
  if (rc) return check(env, rc, "fg_embed_plan");
  return num(env, nseg);
}
FN(js_embed_bwd) {
  Args a(env, info, 7);
  CALL(fg_embed_bwd(a.f(0), a.f(1), a.i32p(2), a.i32p(3), a.i32p(4), a.i32(5), a.i32(6)), "fg_embed_bwd");
}
FN(js_slice_fwd) {
  Args a(env, info, 6);
  CALL(fg_slice_cols_fwd(a.f(0), a.f(1), a.i32(2), a.i32(3), a.i32(4), a.i32(5)), "fg_slice_cols_fwd");
}
FN(js_slice_bwd) {
  Args a(env, info, 6);
  CALL(fg_slice_cols_bwd(a.f(0), a.f(1), a.i32(2), a.i32(3), a.i32(4), a.i32(5)), "fg_slice_cols_bwd");
}
FN(js_add_fwd) {
  Args a(env, info, 4);
  CALL(fg_add_fwd(a.f(0), a.f(1), a.f(2), a.i64(3)), "fg_add_fwd");
}
FN(js_accum) {
  Args a(env, info, 4);
  CALL(fg_accum(a.f(0), a.f(1), a.i64(2), a.i32(3)), "fg_accum");
}
FN(js_wsum_fwd) {
  Args a(env, info, 4);
  CALL(fg_weighted_sum_fwd(a.f(0), a.f(1), a.f(2), a.i64(3)), "fg_weighted_sum_fwd");
}
FN(js_wsum_bwd) {
  Args a(env, info, 5);
  CALL(fg_weighted_sum_bwd(a.f(0), a.f(1), a.f(2), a.i64(3), a.i32(4)), "fg_weighted_sum_bwd");
}
FN(js_vec_mul_fwd) {
  Args a(env, info, 5);
  CALL(fg_vec_mul_fwd(a.f(0), a.f(1), a.f(2), a.i64(3), a.i64(4)), "fg_vec_mul_fwd");
}
FN(js_vec_mul_bwd) {
  Args a(env, info, 9);
  CALL(fg_vec_mul_bwd(a.f(0), a.i32(1), a.f(2), a.i32(3), a.f(4), a.f(5), a.f(6), a.i64(7), a.i64(8)),
       "fg_vec_mul_bwd");
}
FN(js_vec_silu_fwd) {
  Args a(env, info, 4);
  CALL(fg_vec_silu_fwd(a.f(0), a.f(1), a.f(2), a.i64(3)), "fg_vec_silu_fwd");
}
FN(js_vec_silu_bwd) {
  Args a(env, info, 6);
  CALL(fg_vec_silu_bwd(a.f(0), a.i32(1), a.f(2), a.f(3), a.f(4), a.i64(5)), "fg_vec_silu_bwd");
}
FN(js_vec_dot_fwd) {
  Args a(env, info, 4);
  CALL(fg_vec_dot_fwd(a.f(0), a.f(1), a.f(2), a.i64(3)), "fg_vec_dot_fwd");
}
FN(js_vec_dot_bwd) {
  Args a(env, info, 8);
  CALL(fg_vec_dot_bwd(a.f(0), a.i32(1), a.f(2), a.i32(3), a.f(4), a.f(5), a.f(6), a.i64(7)), "fg_vec_dot_bwd");
}
FN(js_vec_scale_fwd) {
  Args a(env, info, 4);
  CALL(fg_vec_scale_fwd(a.f(0), a.f(1), a.f64(2), a.i64(3)), "fg_vec_scale_fwd");
}
FN(js_vec_scale_bwd) {
  Args a(env, info, 5);
  CALL(fg_vec_scale_bwd(a.f(0), a.i32(1), a.f(2), a.f64(3), a.i64(4)), "fg_vec_scale_bwd");
}
FN(js_vec_rope_fwd) {
  Args a(env, info, 6);
  CALL(fg_vec_rope_fwd(a.f(0), a.f(1), a.dp(2), a.dp(3), a.i64(4), a.i32(5)), "fg_vec_rope_fwd");
}
FN(js_vec_rope_bwd) {
  Args a(env, info, 7);
  CALL(fg_vec_rope_bwd(a.f(0), a.i32(1), a.f(2), a.dp(3), a.dp(4), a.i64(5), a.i32(6)), "fg_vec_rope_bwd");
}
FN(js_vec_softmax_fwd) {
  Args a(env, info, 4);
  CALL(fg_vec_softmax_fwd(a.f(0), a.f(1), a.f(2), a.i64(3)), "fg_vec_softmax_fwd");
}
FN(js_vec_softmax_bwd) {
  Args a(env, info, 5);
  CALL(fg_vec_softmax_bwd(a.f(0), a.i32(1), a.f(2), a.f(3), a.i64(4)), "fg_vec_softmax_bwd");
}
FN(js_row_attention) {
  Args a(env, info, 12);
  CALL(fg_row_attention(a.f(0), a.f(1), a.f(2), a.f(3), a.i32(4), a.i32(5), a.f64(6), a.i32(7), a.i32(8), a.i32(9),
                        a.i32(10), a.f(11)),
       "fg_row_attention");
}
FN(js_row_rmsnorm) {
  Args a(env, info, 5);
  CALL(fg_row_rmsnorm(a.f(0), a.f(1), a.f(2), a.i32(3), a.f64(4)), "fg_row_rmsnorm");
}
// [[p, g, m, v, n], ...] -> tensor list (false: an exception is pending)
bool adam_list(napi_env env, napi_value arr, std::vector<fg_adam_tensor>& ts) {
  uint32_t len = 0;
  if (napi_get_array_length(env, arr, &len) != napi_ok) {
    throw_err(env, "adamStep: expected an array");
    return false;
  }
  ts.resize(len);
  for (uint32_t i = 0; i < len; ++i) {
    napi_value row;
    napi_get_element(env, arr, i, &row);
    napi_value el[5];
    for (uint32_t k = 0; k < 5; ++k) napi_get_element(env, row, k, &el[k]);
    void* ptrs[4];
    for (int k = 0; k < 4; ++k) {
      void* d = nullptr;
      if (napi_get_value_external(env, el[k], &d) != napi_ok || !d) {
        throw_err(env, "adamStep: bad handle");
        return false;
      }
      DevBuf* b = static_cast<DevBuf*>(d);
      if (b->tag != kBufTag) {
        throw_err(env, "adamStep: bad handle");
        return false;
      }
      if (b->freed) {
        throw_err(env, "adamStep: buffer used after free");
        return false;
      }
      ptrs[k] = b->ptr;
    }
    double n = 0;
    napi_get_value_double(env, el[4], &n);
    ts[i].p = static_cast<float*>(ptrs[0]);
    ts[i].g = static_cast<const float*>(ptrs[1]);
    ts[i].m = static_cast<float*>(ptrs[2]);
    ts[i].v = static_cast<float*>(ptrs[3]);
    ts[i].n = (int64_t)n;
  }
  return true;
}
// adamStep([[p, g, m, v, n], ...], lr_t, b1, b2, eps, wd, clip, bc1, bc2, stats|null)
FN(js_adam_step) {
  Args a(env, info, 10);
  if (!a.ok) return nullptr;
  std::vector<fg_adam_tensor> ts;
  if (!adam_list(env, a.argv[0], ts)) return nullptr;
  CALL(fg_adam_step(ts.data(), (int)ts.size(), a.f64(1), a.f64(2), a.f64(3), a.f64(4), a.f64(5), a.f64(6), a.f64(7),
                    a.f64(8), a.dp(9)),
       "fg_adam_step");
}
// adamStepSched([[p, g, m, v, n], ...], sched, b1, b2, eps, wd, clip, stats|null)
FN(js_adam_step_sched) {
  Args a(env, info, 8);
  if (!a.ok) return nullptr;
  std::vector<fg_adam_tensor> ts;
  if (!adam_list(env, a.argv[0], ts)) return nullptr;
  CALL(fg_adam_step_sched(ts.data(), (int)ts.size(), a.dp(1), a.f64(2), a.f64(3), a.f64(4), a.f64(5), a.f64(6),
                          a.dp(7)),
       "fg_adam_step_sched");
}
// adamPlanCreate([[p, g, m, v, n], ...]) -> plan handle (its own device table)
FN(js_adam_plan_create) {
  Args a(env, info, 1);
  if (!a.ok) return nullptr;
  std::vector<fg_adam_tensor> ts;
  if (!adam_list(env, a.argv[0], ts)) return nullptr;
  fg_adam_plan* pl = nullptr;
  int rc = fg_adam_plan_create(ts.data(), (int)ts.size(), &pl);
  if (rc) return check(env, rc, "fg_adam_plan_create");
  PlanBox* box = new PlanBox{kPlanTag, pl};
  napi_value ext;
  if (napi_create_external(env, box, plan_finalize, nullptr, &ext) != napi_ok) {
    fg_adam_plan_destroy(pl);
    delete box;
    return throw_err(env, "napi_create_external failed");
  }
  return ext;
}
// adamPlanMatches(plan, [[p, g, m, v, n], ...]) -> bool
FN(js_adam_plan_matches) {
  Args a(env, info, 2);
  if (!a.ok) return nullptr;
  fg_adam_plan* pl = a.plan(0);
  if (!a.ok) return nullptr;
  std::vector<fg_adam_tensor> ts;
  if (!adam_list(env, a.argv[1], ts)) return nullptr;
  int match = 0;
  int rc = fg_adam_plan_matches(pl, ts.data(), (int)ts.size(), &match);
  if (rc) return check(env, rc, "fg_adam_plan_matches");
  napi_value r;
  napi_get_boolean(env, match != 0, &r);
  return r;
}
// adamStepPlan(plan, lr_t, b1, b2, eps, wd, clip, bc1, bc2, stats|null)
FN(js_adam_step_plan) {
  Args a(env, info, 10);
  if (!a.ok) return nullptr;
  fg_adam_plan* pl = a.plan(0);
  CALL(fg_adam_step_plan(pl, a.f64(1), a.f64(2), a.f64(3), a.f64(4), a.f64(5), a.f64(6), a.f64(7), a.f64(8),
                         a.dp(9)),
       "fg_adam_step_plan");
}
// adamStepSchedPlan(plan, sched, b1, b2, eps, wd, clip, stats|null)
FN(js_adam_step_sched_plan) {
  Args a(env, info, 8);
  if (!a.ok) return nullptr;
  fg_adam_plan* pl = a.plan(0);
  CALL(fg_adam_step_sched_plan(pl, a.dp(1), a.f64(2), a.f64(3), a.f64(4), a.f64(5), a.f64(6), a.dp(7)),
       "fg_adam_step_sched_plan");
}
// ── device-resident loop ────────────────────────────────────────────────
FN(js_batch_gather) {  // batchGather(ids, targets, data, n, starts, B, T, V)
  Args a(env, info, 8);
  CALL(fg_batch_gather(a.i32p(0), a.i32p(1), a.i32p(2), a.i64(3), a.i32p(4), a.i32(5), a.i32(6), a.i32(7)),
       "fg_batch_gather");
}
FN(js_embed_keys_len) {
  Args a(env, info, 1);
  if (!a.ok) return nullptr;
  int64_t n = 0;
  int rc = fg_embed_keys_len(a.i32(0), &n);
  if (rc) return check(env, rc, "fg_embed_keys_len");
  return num(env, (double)n);
}
FN(js_embed_sort_keys) {  // embedSortKeys(keys, len, ids, T, V)
  Args a(env, info, 5);
  CALL(fg_embed_sort_keys(static_cast<uint64_t*>(a.ptr(0)), a.i64(1), a.i32p(2), a.i32(3), a.i32(4)),
       "fg_embed_sort_keys");
}
FN(js_embed_bwd_sorted) {  // embedBwdSorted(gW, g, keys, T, V, D, beta)
  Args a(env, info, 7);
  CALL(fg_embed_bwd_sorted(a.f(0), a.f(1), static_cast<const uint64_t*>(a.ptr(2)), a.i32(3), a.i32(4), a.i32(5),
                           a.i32(6)),
       "fg_embed_bwd_sorted");
}
FN(js_fill_f32) {  // fillF32(handle, value, n)
  Args a(env, info, 3);
  CALL(fg_fill_f32(a.f(0), (float)a.f64(1), a.i64(2)), "fg_fill_f32");
}
// Graph handles are externals without a finalizer action: fg_graph_destroy
// must be called explicitly (it synchronises the stream).
FN(js_graph_begin) {
  Args a(env, info, 0);
  CALL(fg_graph_begin(), "fg_graph_begin");
}
FN(js_graph_end) {
  Args a(env, info, 0);
  if (!a.ok) return nullptr;
  void* g = nullptr;
  int rc = fg_graph_end(&g);
  if (rc) return check(env, rc, "fg_graph_end");
  napi_value ext;
  napi_create_external(env, g, nullptr, nullptr, &ext);
  return ext;
}
FN(js_graph_launch) {
  Args a(env, info, 1);
  if (!a.ok) return nullptr;
  void* g = nullptr;
  if (napi_get_value_external(env, a.argv[0], &g) != napi_ok || !g) return throw_err(env, "graphLaunch: bad handle");
  CALL(fg_graph_launch(g), "fg_graph_launch");
}
FN(js_graph_destroy) {
  Args a(env, info, 1);
  if (!a.ok) return nullptr;
  void* g = nullptr;
  if (napi_get_value_external(env, a.argv[0], &g) != napi_ok || !g) return throw_err(env, "graphDestroy: bad handle");
  CALL(fg_graph_destroy(g), "fg_graph_destroy");
}
FN(js_graph_abort) {
  Args a(env, info, 0);
  CALL(fg_graph_abort(), "fg_graph_abort");
}

// ── decode ──────────────────────────────────────────────────────────────
struct DecodeHolder {
  fg_decode_model m;
  std::vector<fg_decode_layer> layers;
};
void decode_finalize(napi_env, void* data, void*) { delete static_cast<DecodeHolder*>(data); }

bool get_prop(napi_env env, napi_value obj, const char* k, napi_value* out) {
  bool has = false;
  if (napi_has_named_property(env, obj, k, &has) != napi_ok || !has) {
    std::string m = std::string("decodeModel: missing field ") + k;
    throw_err(env, m.c_str());
    return false;
  }
  return napi_get_named_property(env, obj, k, out) == napi_ok;
}
bool prop_ptr(napi_env env, napi_value obj, const char* k, void** p) {
  napi_value v;
  if (!get_prop(env, obj, k, &v)) return false;
  void* d = nullptr;
  if (napi_get_value_external(env, v, &d) != napi_ok || !d || static_cast<DevBuf*>(d)->tag != kBufTag ||
      static_cast<DevBuf*>(d)->freed) {
    std::string m = std::string("decodeModel: field ") + k + " is not a live device buffer";
    throw_err(env, m.c_str());
    return false;
  }
  *p = static_cast<DevBuf*>(d)->ptr;
  return true;
}
bool prop_num(napi_env env, napi_value obj, const char* k, double* x) {
  napi_value v;
  if (!get_prop(env, obj, k, &v)) return false;
  return napi_get_value_double(env, v, x) == napi_ok;
}
// An optional integer field (the ggml type of a weight; absent = 0, f32).
int prop_type(napi_env env, napi_value obj, const char* k) {
  bool has = false;
  if (napi_has_named_property(env, obj, k, &has) != napi_ok || !has) return 0;
  napi_value v;
  int32_t t = 0;
  if (napi_get_named_property(env, obj, k, &v) != napi_ok || napi_get_value_int32(env, v, &t) != napi_ok) return 0;
  return t;
}

// decodeModel({dim, hidden, nLayers, nHeads, nKvHeads, vocab, maxSeq, normEps,
//              tok_emb, ln_f, wcls, rope_cos, rope_sin, x, q, h, attn_part,
//              emb_type?, cls_type?,
//              layers: [{ln1, wqkv, wo, ln2, gate, up, down, *_type?}, ...]}) -> handle
FN(js_decode_model) {
  Args a(env, info, 1);
  if (!a.ok) return nullptr;
  napi_value o = a.argv[0];
  DecodeHolder* hd = new DecodeHolder();
  fg_decode_model& m = hd->m;
  double d[8];
  const char* nums[8] = {"dim", "hidden", "nLayers", "nHeads", "nKvHeads", "vocab", "maxSeq", "normEps"};
  void* p[9];
  const char* ptrs[9] = {"tok_emb", "ln_f", "wcls", "rope_cos", "rope_sin", "x", "q", "h", "attn_part"};
  bool ok = true;
  for (int i = 0; i < 8 && ok; ++i) ok = prop_num(env, o, nums[i], &d[i]);
  for (int i = 0; i < 9 && ok; ++i) ok = prop_ptr(env, o, ptrs[i], &p[i]);
  napi_value layers;
  uint32_t nl = 0;
  if (ok) ok = get_prop(env, o, "layers", &layers) && napi_get_array_length(env, layers, &nl) == napi_ok;
  const char* lk[7] = {"ln1", "wqkv", "wo", "ln2", "gate", "up", "down"};
  for (uint32_t l = 0; l < nl && ok; ++l) {
    napi_value lo;
    napi_get_element(env, layers, l, &lo);
    void* q[7];
    for (int i = 0; i < 7 && ok; ++i) ok = prop_ptr(env, lo, lk[i], &q[i]);
    if (ok) {
      fg_decode_layer y;
      y.ln1 = (const float*)q[0]; y.wqkv = q[1]; y.wo = q[2];
      y.ln2 = (const float*)q[3]; y.gate = q[4]; y.up = q[5];
      y.down = q[6];
      y.wqkv_type = prop_type(env, lo, "wqkv_type"); y.wo_type = prop_type(env, lo, "wo_type");
      y.gate_type = prop_type(env, lo, "gate_type"); y.up_type = prop_type(env, lo, "up_type");
      y.down_type = prop_type(env, lo, "down_type");
      hd->layers.push_back(y);
    }
  }
  if (!ok) {
    delete hd;
    return nullptr;
  }
  m.dim = (int)d[0]; m.hidden = (int)d[1]; m.nLayers = (int)d[2]; m.nHeads = (int)d[3];
  m.nKvHeads = (int)d[4]; m.vocab = (int)d[5]; m.maxSeq = (int)d[6]; m.normEps = d[7];
  if ((uint32_t)m.nLayers != nl) {
    delete hd;
    return throw_err(env, "decodeModel: layers.length != nLayers");
  }
  m.emb_type = prop_type(env, o, "emb_type");
  m.cls_type = prop_type(env, o, "cls_type");
  m.tok_emb = p[0]; m.ln_f = (const float*)p[1]; m.wcls = p[2];
  m.rope_cos = (const float*)p[3]; m.rope_sin = (const float*)p[4];
  m.x = (float*)p[5]; m.q = (float*)p[6]; m.h = (float*)p[7]; m.attn_part = (double*)p[8];
  m.layers = hd->layers.data();
  napi_value ext;
  if (napi_create_external(env, hd, decode_finalize, nullptr, &ext) != napi_ok) {
    delete hd;
    return throw_err(env, "napi_create_external failed");
  }
  return ext;
}
// ── quantized weights ───────────────────────────────────────────────────
FN(js_qrow_bytes) {  // qrowBytes(type, n) -> bytes
  Args a(env, info, 2);
  if (!a.ok) return nullptr;
  int64_t b = 0;
  int rc = fg_qrow_bytes(a.i32(0), a.i64(1), &b);
  if (rc) return check(env, rc, "fg_qrow_bytes");
  return num(env, (double)b);
}
FN(js_qmatvec) {  // qmatvec(type, y, W, x, N, K)
  Args a(env, info, 6);
  if (!a.ok) return nullptr;
  CALL(fg_qmatvec(a.i32(0), a.f(1), a.ptr(2), a.f(3), a.i32(4), a.i32(5)), "fg_qmatvec");
}
FN(js_qmatvec_f64) {  // qmatvecF64(type, y, W, x, N, K)
  Args a(env, info, 6);
  if (!a.ok) return nullptr;
  CALL(fg_qmatvec_f64(a.i32(0), a.dp(1), a.ptr(2), a.f(3), a.i32(4), a.i32(5)), "fg_qmatvec_f64");
}
FN(js_silu_mul) {  // siluMul(h, g, u, n)
  Args a(env, info, 4);
  if (!a.ok) return nullptr;
  CALL(fg_silu_mul(a.f(0), a.f(1), a.f(2), a.i64(3)), "fg_silu_mul");
}
FN(js_dequantize) {  // dequantize(type, out, q, n)
  Args a(env, info, 4);
  if (!a.ok) return nullptr;
  CALL(fg_dequantize(a.i32(0), a.f(1), a.ptr(2), a.i64(3)), "fg_dequantize");
}
FN(js_quantize) {  // quantize(type, out, x, n)
  Args a(env, info, 4);
  if (!a.ok) return nullptr;
  CALL(fg_quantize(a.i32(0), a.ptr(1), a.f(2), a.i64(3)), "fg_quantize");
}
FN(js_decode_part_len) {  // decodePartLen(nHeads, dHead, maxSeq) -> doubles
  Args a(env, info, 3);
  if (!a.ok) return nullptr;
  int64_t n = 0;
  int rc = fg_decode_part_len(a.i32(0), a.i32(1), a.i32(2), &n);
  if (rc) return check(env, rc, "fg_decode_part_len");
  return num(env, (double)n);
}
FN(js_decode_step) {  // decodeStep(model, kcache, vcache, state, logits)
  Args a(env, info, 5);
  if (!a.ok) return nullptr;
  void* d = nullptr;
  if (napi_get_value_external(env, a.argv[0], &d) != napi_ok || !d) return throw_err(env, "decodeStep: bad model");
  CALL(fg_decode_step(&static_cast<DecodeHolder*>(d)->m, a.f(1), a.f(2), a.i32p(3), a.f(4)), "fg_decode_step");
}

napi_value Init(napi_env env, napi_value exports) {
  struct {
    const char* name;
    napi_callback cb;
  } fns[] = {
      {"deviceCount", js_device_count}, {"init", js_init}, {"alloc", js_alloc}, {"view", js_view},
      {"free", js_free}, {"bytes", js_bytes}, {"h2d", js_h2d}, {"d2h", js_d2h}, {"d2d", js_d2d},
      {"zero", js_zero}, {"sync", js_sync}, {"readAsync", js_read_async}, {"readWait", js_read_wait},
      {"memStats", js_mem_stats}, {"emptyCache", js_empty_cache}, {"eventCreate", js_event_create},
      {"eventRecord", js_event_record}, {"eventElapsed", js_event_elapsed}, {"kprofEnable", js_kprof_enable},
      {"kprofReset", js_kprof_reset}, {"kprofReport", js_kprof_report},
      {"matmulTFwd", js_matmulT_fwd}, {"matmulTBwdX", js_matmulT_bwd_x}, {"matmulTBwdW", js_matmulT_bwd_w},
      {"matmulTFwdSwiglu", js_matmulT_fwd_swiglu}, {"matmulTBwdXPieces", js_matmulT_bwd_x_pieces}, {"matmulTBwdXHalves", js_matmulT_bwd_x_halves},
      {"rmsnormBwdFromHalves", js_rmsnorm_bwd_from_halves}, {"rmsnormBwdParts", js_rmsnorm_bwd_parts},
      {"rmsnormBwdPartial", js_rmsnorm_bwd_partial}, {"colsumGrouped", js_colsum_grouped},
      {"matmulTFwdResid", js_matmulT_fwd_resid}, {"matmulTBwd", js_matmulT_bwd}, {"qkvRopeFwd", js_qkv_rope_fwd}, {"qkvRopeBwd", js_qkv_rope_bwd},
      {"attnFwd", js_attn_fwd}, {"attnBwd", js_attn_bwd}, {"matmulTFwdRope", js_matmulT_fwd_rope},
      {"attnFwdQkv", js_attn_fwd_qkv}, {"attnBwdQkv", js_attn_bwd_qkv}, {"ceFwd", js_ce_fwd}, {"ceBwd", js_ce_bwd}, {"ceFwdBwd", js_ce_fwd_bwd},
      {"rmsnormFwd", js_rmsnorm_fwd}, {"rmsnormBwd", js_rmsnorm_bwd}, {"rmsnormBwdFrom", js_rmsnorm_bwd_from},
      {"matmulTBwdWGrouped", js_matmulT_bwd_w_grouped}, {"ropeTable", js_rope_table},
      {"ropeFwd", js_rope_fwd}, {"ropeBwd", js_rope_bwd}, {"swigluFwd", js_swiglu_fwd},
      {"swigluBwd", js_swiglu_bwd}, {"swigluGuFwd", js_swiglu_gu_fwd},
      {"swigluGuBwd", js_swiglu_gu_bwd}, {"embedFwd", js_embed_fwd}, {"embedPlan", js_embed_plan},
      {"embedBwd", js_embed_bwd}, {"sliceColsFwd", js_slice_fwd}, {"sliceColsBwd", js_slice_bwd},
      {"addFwd", js_add_fwd}, {"accum", js_accum}, {"weightedSumFwd", js_wsum_fwd},
      {"weightedSumBwd", js_wsum_bwd}, {"vecMulFwd", js_vec_mul_fwd}, {"vecMulBwd", js_vec_mul_bwd},
      {"vecSiluFwd", js_vec_silu_fwd}, {"vecSiluBwd", js_vec_silu_bwd}, {"vecDotFwd", js_vec_dot_fwd},
      {"vecDotBwd", js_vec_dot_bwd}, {"vecScaleFwd", js_vec_scale_fwd}, {"vecScaleBwd", js_vec_scale_bwd},
      {"vecRopeFwd", js_vec_rope_fwd}, {"vecRopeBwd", js_vec_rope_bwd}, {"vecSoftmaxFwd", js_vec_softmax_fwd},
      {"vecSoftmaxBwd", js_vec_softmax_bwd}, {"rowAttention", js_row_attention}, {"rowRmsnorm", js_row_rmsnorm}, {"adamStep", js_adam_step},
      {"adamStepSched", js_adam_step_sched}, {"adamPlanCreate", js_adam_plan_create},
      {"adamPlanMatches", js_adam_plan_matches}, {"adamStepPlan", js_adam_step_plan},
      {"adamStepSchedPlan", js_adam_step_sched_plan}, {"batchGather", js_batch_gather}, {"embedKeysLen", js_embed_keys_len},
      {"embedSortKeys", js_embed_sort_keys}, {"embedBwdSorted", js_embed_bwd_sorted}, {"fillF32", js_fill_f32},
      {"graphBegin", js_graph_begin}, {"graphEnd", js_graph_end}, {"graphLaunch", js_graph_launch},
      {"graphDestroy", js_graph_destroy}, {"graphAbort", js_graph_abort}, {"decodeModel", js_decode_model},
      {"qrowBytes", js_qrow_bytes}, {"qmatvec", js_qmatvec}, {"qmatvecF64", js_qmatvec_f64}, {"siluMul", js_silu_mul}, {"dequantize", js_dequantize}, {"quantize", js_quantize},
      {"decodeStep", js_decode_step}, {"decodePartLen", js_decode_part_len},
  };
  for (auto& f : fns) {
    napi_value fn;
    napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.cb, nullptr, &fn);
    napi_set_named_property(env, exports, f.name, fn);
  }
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Init)
