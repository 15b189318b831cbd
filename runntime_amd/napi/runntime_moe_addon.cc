// N-API binding of libmoe.so: the native half of a ruNNtime Executor that
// runs the MoE ops on HIP (include/runntime_moe.h).
//
// The reference's host is TypeScript in Node; its ops record `pending`
// nodes that an Executor dispatches (src/core/graph/evalCore.ts:14-31,
// registry src/core/gpu/dispatch/registry.ts:74-146). hipExecutor.ts, next
// to this file, is that Executor: it calls the functions below with device
// pointers as BigInt and sizes as numbers, one C-ABI call each. Errors come
// back as the reference's RunntimeError shape (src/core/error.ts:3-50): an
// Error named 'RunntimeError' whose `code` is the status name.
//
// Build: g++ -shared -fPIC -I<node headers> -Iinclude this file
//        -Lrunntime_amd -lmoe (runntime_amd/build.py does it).
#define NAPI_VERSION 6
#include <node_api.h>

#include <stdint.h>
#include <string.h>

#include <string>
#include <vector>

#include "../../include/runntime_moe.h"

namespace {

const char *const CODES[] = {"OK", "INVALID_ARGUMENT", "EXECUTION_FAILED", "NOT_INITIALIZED",
                             "RESOURCE_DISPOSED"};

// Throws a RunntimeError {name, code, message}; returns nullptr for the
// caller to return.
napi_value throw_error(napi_env env, const char *code, const std::string &msg) {
  napi_value c, m, err, name;
  napi_create_string_utf8(env, code, NAPI_AUTO_LENGTH, &c);
  napi_create_string_utf8(env, msg.c_str(), msg.size(), &m);
  napi_create_error(env, c, m, &err);
  napi_create_string_utf8(env, "RunntimeError", NAPI_AUTO_LENGTH, &name);
  napi_set_named_property(env, err, "name", name);
  napi_throw(env, err);
  return nullptr;
}

napi_value throw_status(napi_env env, int rc) {
  const char *code = rc > 0 && rc < 5 ? CODES[rc] : "EXECUTION_FAILED";
  return throw_error(env, code, moe_last_error());
}

// Argument readers. A bad JS type throws INVALID_ARGUMENT and sets `ok`
// false; every reader is a no-op once `ok` is false.
struct Args {
  napi_env env;
  std::vector<napi_value> v;
  bool ok = true;
  std::string what;

  Args(napi_env e, napi_callback_info info, size_t n) : env(e), v(n) {
    size_t argc = n;
    napi_get_cb_info(env, info, &argc, v.data(), nullptr, nullptr);
    if (argc < n) fail("expected " + std::to_string(n) + " arguments, got " + std::to_string(argc));
  }
  void fail(const std::string &m) {
    if (ok) what = m;
    ok = false;
  }
  napi_valuetype type(size_t i) {
    napi_valuetype t = napi_undefined;
    napi_typeof(env, v[i], &t);
    return t;
  }
  // A device (or host) pointer: BigInt, a non-negative integer Number, or
  // null / undefined / 0n for NULL.
  void *ptr(size_t i) {
    if (!ok) return nullptr;
    const napi_valuetype t = type(i);
    if (t == napi_null || t == napi_undefined) return nullptr;
    if (t == napi_bigint) {
      uint64_t u = 0;
      bool lossless = false;
      napi_get_value_bigint_uint64(env, v[i], &u, &lossless);
      if (!lossless) fail("argument " + std::to_string(i) + ": pointer out of range");
      return (void *)(uintptr_t)u;
    }
    if (t == napi_number) {
      double d = 0;
      napi_get_value_double(env, v[i], &d);
      if (d < 0 || d != (double)(uint64_t)d) fail("argument " + std::to_string(i) + ": not a pointer");
      return (void *)(uintptr_t)(uint64_t)d;
    }
    fail("argument " + std::to_string(i) + ": expected a BigInt pointer");
    return nullptr;
  }
  int64_t i64(size_t i) {
    if (!ok) return 0;
    if (type(i) == napi_bigint) {
      int64_t x = 0;
      bool lossless = false;
      napi_get_value_bigint_int64(env, v[i], &x, &lossless);
      if (!lossless) {
        fail("argument " + std::to_string(i) + ": integer out of int64 range");
        return 0;
      }
      return x;
    }
    double d = 0;
    if (napi_get_value_double(env, v[i], &d) != napi_ok || d != (double)(int64_t)d) {
      fail("argument " + std::to_string(i) + ": expected an integer");
      return 0;
    }
    return (int64_t)d;
  }
  int i32(size_t i) {
    const int64_t x = i64(i);
    if (ok && (x < INT32_MIN || x > INT32_MAX)) fail("argument " + std::to_string(i) + ": out of int32 range");
    return (int)x;
  }
  float f32(size_t i) {
    double d = 0;
    if (ok && napi_get_value_double(env, v[i], &d) != napi_ok) fail("argument " + std::to_string(i) + ": expected a number");
    return (float)d;
  }
  std::string str(size_t i) {
    if (!ok) return "";
    size_t n = 0;
    if (napi_get_value_string_utf8(env, v[i], nullptr, 0, &n) != napi_ok) {
      fail("argument " + std::to_string(i) + ": expected a string");
      return "";
    }
    std::string s(n, '\0');
    napi_get_value_string_utf8(env, v[i], &s[0], n + 1, &n);
    return s;
  }
  // Host bytes of an ArrayBuffer or typed array (for uploads / readbacks).
  void *bytes(size_t i, size_t *len) {
    *len = 0;
    if (!ok) return nullptr;
    bool is = false;
    void *data = nullptr;
    napi_is_typedarray(env, v[i], &is);
    if (is) {
      napi_typedarray_type tt;
      size_t n = 0, off = 0;
      napi_value ab;
      napi_get_typedarray_info(env, v[i], &tt, &n, &data, &ab, &off);
      static const size_t el[] = {1, 1, 1, 2, 2, 4, 4, 4, 8, 8, 8};
      *len = n * (tt <= napi_biguint64_array ? el[tt] : 1);
      return data;
    }
    napi_is_arraybuffer(env, v[i], &is);
    if (is) {
      napi_get_arraybuffer_info(env, v[i], &data, len);
      return data;
    }
    fail("argument " + std::to_string(i) + ": expected an ArrayBuffer or typed array");
    return nullptr;
  }
  // moe_value_desc from a ValueMeta-like object {elems, dtype, dims?}
  // (src/core/graph/value.ts:17-24).
  moe_value_desc meta(size_t i) {
    moe_value_desc d{};
    if (!ok) return d;
    if (type(i) != napi_object) {
      fail("argument " + std::to_string(i) + ": expected a ValueMeta {elems, dtype, dims?}");
      return d;
    }
    // elems and every dim must be non-negative integers, rank at most 4: a
    // malformed meta must not reach the shape checks as another, valid-looking
    // shape.
    auto whole = [&](napi_value y, int64_t *out) {
      double dv = 0;
      if (napi_get_value_double(env, y, &dv) != napi_ok || !(dv >= 0) || dv > 9.0e15 ||
          dv != (double)(int64_t)dv)
        return false;
      *out = (int64_t)dv;
      return true;
    };
    napi_value x;
    napi_get_named_property(env, v[i], "elems", &x);
    if (!whole(x, &d.elems)) {
      fail("argument " + std::to_string(i) + ": ValueMeta.elems must be a non-negative integer");
      return d;
    }
    napi_get_named_property(env, v[i], "dtype", &x);
    char dt[16] = {0};
    size_t n = 0;
    napi_get_value_string_utf8(env, x, dt, sizeof dt, &n);
    d.dtype = !strcmp(dt, "f32") ? MOE_VALUE_F32 : !strcmp(dt, "f16") ? MOE_VALUE_F16
              : !strcmp(dt, "quantW") ? MOE_VALUE_QUANTW : 9;
    bool has = false;
    napi_has_named_property(env, v[i], "dims", &has);
    if (has) {
      napi_get_named_property(env, v[i], "dims", &x);
      bool arr = false;
      napi_is_array(env, x, &arr);
      if (!arr) {
        fail("argument " + std::to_string(i) + ": ValueMeta.dims must be an array");
        return d;
      }
      uint32_t len = 0;
      napi_get_array_length(env, x, &len);
      if (len > 4) {
        fail("argument " + std::to_string(i) + ": ValueMeta.dims has rank " + std::to_string(len) +
             "; at most 4 is supported");
        return d;
      }
      d.rank = (int)len;
      for (uint32_t k = 0; k < len; k++) {
        napi_value el;
        napi_get_element(env, x, k, &el);
        if (!whole(el, &d.dims[k])) {
          fail("argument " + std::to_string(i) + ": ValueMeta.dims[" + std::to_string(k) +
               "] must be a non-negative integer");
          return d;
        }
      }
    }
    return d;
  }
  // A QuantExpertWeight's device buffers: three pointer arguments.
  moe_expert_weight weight(size_t i) {
    moe_expert_weight w{};
    w.w = (const uint32_t *)ptr(i);
    w.scales = (const float *)ptr(i + 1);
    w.bias = (const float *)ptr(i + 2);
    return w;
  }
  napi_value bad() { return throw_error(env, "INVALID_ARGUMENT", what); }
};

napi_value undefined(napi_env env) {
  napi_value u;
  napi_get_undefined(env, &u);
  return u;
}

napi_value bigint(napi_env env, const void *p) {
  napi_value b;
  napi_create_bigint_uint64(env, (uint64_t)(uintptr_t)p, &b);
  return b;
}

#define FINISH(rc) return (rc) ? throw_status(env, (rc)) : undefined(env)

// version(): number
napi_value Version(napi_env env, napi_callback_info) {
  napi_value r;
  napi_create_int32(env, moe_version(), &r);
  return r;
}

// ctxCreate(device, stream = null): bigint. stream: a hipStream_t as
// BigInt, null for the context's own, 1n for the null stream.
napi_value CtxCreate(napi_env env, napi_callback_info info) {
  size_t argc = 2;
  napi_value v[2];
  napi_get_cb_info(env, info, &argc, v, nullptr, nullptr);
  Args a(env, info, argc < 1 ? 1 : argc);
  const int device = a.i32(0);
  void *stream = argc > 1 ? a.ptr(1) : nullptr;
  if (!a.ok) return a.bad();
  moe_ctx *ctx = nullptr;
  const int rc = moe_ctx_create(device, stream, &ctx);
  if (rc) return throw_status(env, rc);
  return bigint(env, ctx);
}

napi_value CtxDestroy(napi_env env, napi_callback_info info) {
  Args a(env, info, 1);
  moe_ctx *ctx = (moe_ctx *)a.ptr(0);
  if (!a.ok) return a.bad();
  FINISH(moe_ctx_destroy(ctx));
}

napi_value CtxSetStream(napi_env env, napi_callback_info info) {
  Args a(env, info, 2);
  moe_ctx *ctx = (moe_ctx *)a.ptr(0);
  void *s = a.ptr(1);
  if (!a.ok) return a.bad();
  FINISH(moe_ctx_set_stream(ctx, s));
}

napi_value Sync(napi_env env, napi_callback_info info) {
  Args a(env, info, 1);
  moe_ctx *ctx = (moe_ctx *)a.ptr(0);
  if (!a.ok) return a.bad();
  FINISH(moe_sync(ctx));
}

// bufferAlloc(ctx, bytes): bigint
napi_value BufferAlloc(napi_env env, napi_callback_info info) {
  Args a(env, info, 2);
  moe_ctx *ctx = (moe_ctx *)a.ptr(0);
  const int64_t n = a.i64(1);
  if (!a.ok) return a.bad();
  if (n < 0) return throw_error(env, "INVALID_ARGUMENT", "bufferAlloc: negative size");
  void *p = nullptr;
  const int rc = moe_buffer_alloc(ctx, (size_t)n, &p);
  if (rc) return throw_status(env, rc);
  return bigint(env, p);
}

napi_value BufferFree(napi_env env, napi_callback_info info) {
  Args a(env, info, 2);
  moe_ctx *ctx = (moe_ctx *)a.ptr(0);
  void *p = a.ptr(1);
  if (!a.ok) return a.bad();
  FINISH(moe_buffer_free(ctx, p));
}

// bufferWrite(ctx, dst, hostBytes) / bufferRead(ctx, src, hostBytes)
napi_value BufferWrite(napi_env env, napi_callback_info info) {
  Args a(env, info, 3);
  moe_ctx *ctx = (moe_ctx *)a.ptr(0);
  void *dst = a.ptr(1);
  size_t n = 0;
  void *host = a.bytes(2, &n);
  if (!a.ok) return a.bad();
  FINISH(moe_buffer_write(ctx, dst, host, n));
}

napi_value BufferRead(napi_env env, napi_callback_info info) {
  Args a(env, info, 3);
  moe_ctx *ctx = (moe_ctx *)a.ptr(0);
  const void *src = a.ptr(1);
  size_t n = 0;
  void *host = a.bytes(2, &n);
  if (!a.ok) return a.bad();
  FINISH(moe_buffer_read(ctx, host, src, n));
}

// checkExpertWeight(op, w, scales, bias, route, kIn, t, slots, bits,
// groupSize): {n, experts}. Arguments 1-4 are ValueMeta objects.
napi_value CheckExpertWeight(napi_env env, napi_callback_info info) {
  Args a(env, info, 10);
  const std::string op = a.str(0);
  const moe_value_desc w = a.meta(1), sc = a.meta(2), b = a.meta(3), r = a.meta(4);
  const int64_t k_in = a.i64(5), t = a.i64(6);
  const int slots = a.i32(7), bits = a.i32(8), g = a.i32(9);
  if (!a.ok) return a.bad();
  int64_t n = 0, e = 0;
  const int rc = moe_check_expert_weight(op.c_str(), &w, &sc, &b, &r, k_in, t, slots, bits, g, &n, &e);
  if (rc) return throw_status(env, rc);
  napi_value o, nv, ev;
  napi_create_object(env, &o);
  napi_create_int64(env, n, &nv);
  napi_create_int64(env, e, &ev);
  napi_set_named_property(env, o, "n", nv);
  napi_set_named_property(env, o, "experts", ev);
  return o;
}

// topk(ctx, logits, dtype, T, E, k, route)
napi_value Topk(napi_env env, napi_callback_info info) {
  Args a(env, info, 7);
  moe_ctx *ctx = (moe_ctx *)a.ptr(0);
  const void *x = a.ptr(1);
  const int dt = a.i32(2), T = a.i32(3), E = a.i32(4), k = a.i32(5);
  float *route = (float *)a.ptr(6);
  if (!a.ok) return a.bad();
  FINISH(moe_topk(ctx, x, (moe_dtype)dt, T, E, k, route));
}

// routerTopk(ctx, x, dtype, w, b, T, d, E, k, route)
napi_value RouterTopk(napi_env env, napi_callback_info info) {
  Args a(env, info, 10);
  moe_ctx *ctx = (moe_ctx *)a.ptr(0);
  const void *x = a.ptr(1);
  const int dt = a.i32(2);
  const float *w = (const float *)a.ptr(3), *b = (const float *)a.ptr(4);
  const int T = a.i32(5), d = a.i32(6), E = a.i32(7), k = a.i32(8);
  float *route = (float *)a.ptr(9);
  if (!a.ok) return a.bad();
  FINISH(moe_router_topk(ctx, x, (moe_dtype)dt, w, b, T, d, E, k, route));
}

// moeUp(ctx, x, dtype, route, gluW, gluScales, gluBias, linW, linScales,
//       linBias, T, K, N, E, k, bits, groupSize, act)
napi_value MoeUp(napi_env env, napi_callback_info info) {
  Args a(env, info, 18);
  moe_ctx *ctx = (moe_ctx *)a.ptr(0);
  const void *x = a.ptr(1);
  const int dt = a.i32(2);
  const float *route = (const float *)a.ptr(3);
  const moe_expert_weight glu = a.weight(4), lin = a.weight(7);
  const int T = a.i32(10), K = a.i32(11), N = a.i32(12), E = a.i32(13), k = a.i32(14);
  const int bits = a.i32(15), g = a.i32(16);
  float *act = (float *)a.ptr(17);
  if (!a.ok) return a.bad();
  FINISH(moe_up(ctx, x, (moe_dtype)dt, route, &glu, &lin, T, K, N, E, k, bits, g, act));
}

// moeDown(ctx, act, route, w, scales, bias, residual, T, K, N, E, k, bits,
//         groupSize, out)
napi_value MoeDown(napi_env env, napi_callback_info info) {
  Args a(env, info, 15);
  moe_ctx *ctx = (moe_ctx *)a.ptr(0);
  const float *act = (const float *)a.ptr(1), *route = (const float *)a.ptr(2);
  const moe_expert_weight w = a.weight(3);
  const float *res = (const float *)a.ptr(6);
  const int T = a.i32(7), K = a.i32(8), N = a.i32(9), E = a.i32(10), k = a.i32(11);
  const int bits = a.i32(12), g = a.i32(13);
  float *out = (float *)a.ptr(14);
  if (!a.ok) return a.bad();
  FINISH(moe_down(ctx, act, route, &w, res, T, K, N, E, k, bits, g, out));
}

// moeLayer(ctx, x, dtype, routerW, routerB, glu×3, lin×3, down×3, residual,
//          T, d, I, E, k, bits, groupUp, groupDown, routeOut, out)
napi_value MoeLayer(napi_env env, napi_callback_info info) {
  Args a(env, info, 25);
  moe_ctx *ctx = (moe_ctx *)a.ptr(0);
  const void *x = a.ptr(1);
  const int dt = a.i32(2);
  const float *rw = (const float *)a.ptr(3), *rb = (const float *)a.ptr(4);
  const moe_expert_weight glu = a.weight(5), lin = a.weight(8), down = a.weight(11);
  const float *res = (const float *)a.ptr(14);
  const int T = a.i32(15), d = a.i32(16), I = a.i32(17), E = a.i32(18), k = a.i32(19);
  const int bits = a.i32(20), gu = a.i32(21), gd = a.i32(22);
  float *route = (float *)a.ptr(23), *out = (float *)a.ptr(24);
  if (!a.ok) return a.bad();
  FINISH(moe_layer(ctx, x, (moe_dtype)dt, rw, rb, &glu, &lin, &down, res, T, d, I, E, k, bits, gu,
                   gd, route, out));
}

// moeBlock(ctx, x, dtype, normW, eps, routerW, routerB, glu×3, lin×3,
//          down×3, T, d, I, E, k, bits, groupUp, groupDown, routeOut, out)
napi_value MoeBlock(napi_env env, napi_callback_info info) {
  Args a(env, info, 26);
  moe_ctx *ctx = (moe_ctx *)a.ptr(0);
  const void *x = a.ptr(1);
  const int dt = a.i32(2);
  const void *nw = a.ptr(3);
  const float eps = a.f32(4);
  const float *rw = (const float *)a.ptr(5), *rb = (const float *)a.ptr(6);
  const moe_expert_weight glu = a.weight(7), lin = a.weight(10), down = a.weight(13);
  const int T = a.i32(16), d = a.i32(17), I = a.i32(18), E = a.i32(19), k = a.i32(20);
  const int bits = a.i32(21), gu = a.i32(22), gd = a.i32(23);
  float *route = (float *)a.ptr(24), *out = (float *)a.ptr(25);
  if (!a.ok) return a.bad();
  FINISH(moe_block(ctx, x, (moe_dtype)dt, nw, eps, rw, rb, &glu, &lin, &down, T, d, I, E, k, bits,
                   gu, gd, route, out));
}

// rmsNorm(ctx, x, dtype, rows, cols, weight, weightLen, eps, group,
//         residual, scale, out)
napi_value RmsNorm(napi_env env, napi_callback_info info) {
  Args a(env, info, 12);
  moe_ctx *ctx = (moe_ctx *)a.ptr(0);
  const void *x = a.ptr(1);
  const int dt = a.i32(2), rows = a.i32(3), cols = a.i32(4);
  const void *w = a.ptr(5);
  const int wl = a.i32(6);
  const float eps = a.f32(7);
  const int group = a.i32(8);
  const void *res = a.ptr(9);
  const float scale = a.f32(10);
  void *out = a.ptr(11);
  if (!a.ok) return a.bad();
  FINISH(moe_rmsnorm(ctx, x, (moe_dtype)dt, rows, cols, w, wl, eps, group, res, scale, out));
}

// linear(ctx, x, w, bias, addend, T, K, N, out)
napi_value Linear(napi_env env, napi_callback_info info) {
  Args a(env, info, 9);
  moe_ctx *ctx = (moe_ctx *)a.ptr(0);
  const float *x = (const float *)a.ptr(1), *w = (const float *)a.ptr(2);
  const float *b = (const float *)a.ptr(3), *add = (const float *)a.ptr(4);
  const int T = a.i32(5), K = a.i32(6), N = a.i32(7);
  float *out = (float *)a.ptr(8);
  if (!a.ok) return a.bad();
  FINISH(moe_linear(ctx, x, w, b, add, T, K, N, out));
}

// packQuantW(ctx, ints, E, k, n, bits, words)
napi_value PackQuantW(napi_env env, napi_callback_info info) {
  Args a(env, info, 7);
  moe_ctx *ctx = (moe_ctx *)a.ptr(0);
  const int8_t *ints = (const int8_t *)a.ptr(1);
  const int E = a.i32(2), k = a.i32(3), n = a.i32(4), bits = a.i32(5);
  uint32_t *words = (uint32_t *)a.ptr(6);
  if (!a.ok) return a.bad();
  FINISH(moe_pack_quantw(ctx, ints, E, k, n, bits, words));
}

// attention(ctx, qkv, dtype, T, qHeads, kvHeads, headDim, windowLeft,
//           windowRight, sinks, cos, sin, out)
napi_value Attention(napi_env env, napi_callback_info info) {
  Args a(env, info, 13);
  moe_ctx *ctx = (moe_ctx *)a.ptr(0);
  const void *qkv = a.ptr(1);
  const int dt = a.i32(2), T = a.i32(3), qh = a.i32(4), kvh = a.i32(5), hd = a.i32(6);
  const int64_t wl = a.i64(7), wr = a.i64(8);
  const float *sinks = (const float *)a.ptr(9), *cs = (const float *)a.ptr(10),
              *sn = (const float *)a.ptr(11);
  void *out = a.ptr(12);
  if (!a.ok) return a.bad();
  FINISH(moe_attention(ctx, qkv, (moe_dtype)dt, T, qh, kvh, hd, wl, wr, sinks, cs, sn, out));
}

// Weights owned by the library (Parameter, src/core/nn/module.ts:20-65):
// weightsUpload(ctx, host, rawInt8, scales, bias, E, K, N, bits, groupSize)
// returns an external handle released with the JS object (or by
// weightsDispose); weightsView(h) gives {w, scales, bias} pointers.
void release_weights(napi_env, void *h, void *) { moe_weights_release((moe_weights *)h); }

napi_value WeightsUpload(napi_env env, napi_callback_info info) {
  Args a(env, info, 10);
  moe_ctx *ctx = (moe_ctx *)a.ptr(0);
  size_t nh = 0, ns = 0, nb = 0;
  const void *host = a.bytes(1, &nh);
  const int raw = a.i32(2);
  const float *sc = (const float *)a.bytes(3, &ns);
  const float *b = nullptr;
  if (a.ok && a.type(4) != napi_null && a.type(4) != napi_undefined) b = (const float *)a.bytes(4, &nb);
  const int E = a.i32(5), K = a.i32(6), N = a.i32(7), bits = a.i32(8), g = a.i32(9);
  if (!a.ok) return a.bad();
  // The host arrays must hold what the shapes say (the C ABI cannot tell).
  const int64_t want_w = raw ? (int64_t)E * K * N : (int64_t)E * K * N * bits / 8;
  if (E < 1 || K < 1 || N < 1 || g < 1 || (int64_t)nh < want_w || (int64_t)ns < (int64_t)E * K / g * N * 4 ||
      (b && (int64_t)nb < (int64_t)E * N * 4))
    return throw_error(env, "INVALID_ARGUMENT", "weightsUpload: host arrays smaller than the shape");
  moe_weights *h = nullptr;
  const int rc = moe_weights_upload(ctx, host, raw, sc, b, E, K, N, bits, g, &h);
  if (rc) return throw_status(env, rc);
  napi_value ext;
  napi_create_external(env, h, release_weights, nullptr, &ext);
  return ext;
}

moe_weights *handle(Args &a, size_t i) {
  void *h = nullptr;
  if (a.ok && napi_get_value_external(a.env, a.v[i], &h) != napi_ok) a.fail("expected a weights handle");
  return (moe_weights *)h;
}

napi_value WeightsView(napi_env env, napi_callback_info info) {
  Args a(env, info, 1);
  moe_weights *h = handle(a, 0);
  if (!a.ok) return a.bad();
  moe_expert_weight v{};
  const int rc = moe_weights_view(h, &v);
  if (rc) return throw_status(env, rc);
  napi_value o;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "w", bigint(env, v.w));
  napi_set_named_property(env, o, "scales", bigint(env, v.scales));
  napi_set_named_property(env, o, "bias", bigint(env, v.bias));
  return o;
}

napi_value WeightsDispose(napi_env env, napi_callback_info info) {
  Args a(env, info, 1);
  moe_weights *h = handle(a, 0);
  if (!a.ok) return a.bad();
  FINISH(moe_weights_dispose(h));
}

napi_value Init(napi_env env, napi_value exports) {
  const struct {
    const char *name;
    napi_callback fn;
  } fns[] = {{"version", Version},
             {"ctxCreate", CtxCreate},
             {"ctxDestroy", CtxDestroy},
             {"ctxSetStream", CtxSetStream},
             {"sync", Sync},
             {"bufferAlloc", BufferAlloc},
             {"bufferFree", BufferFree},
             {"bufferWrite", BufferWrite},
             {"bufferRead", BufferRead},
             {"checkExpertWeight", CheckExpertWeight},
             {"topk", Topk},
             {"routerTopk", RouterTopk},
             {"moeUp", MoeUp},
             {"moeDown", MoeDown},
             {"moeLayer", MoeLayer},
             {"moeBlock", MoeBlock},
             {"rmsNorm", RmsNorm},
             {"linear", Linear},
             {"packQuantW", PackQuantW},
             {"attention", Attention},
             {"weightsUpload", WeightsUpload},
             {"weightsView", WeightsView},
             {"weightsDispose", WeightsDispose}};
  for (const auto &f : fns) {
    napi_value v;
    napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.fn, nullptr, &v);
    napi_set_named_property(env, exports, f.name, v);
  }
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Init)
