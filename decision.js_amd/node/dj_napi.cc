// N-API binding of the decision.js MI355X library (include/dj.h) for the Node host: one JS function per C
// entry point. Device pointers and opaque handles (context, recorder, weight) cross as BigInt; host data as
// typed arrays (their bytes are passed as they are); a nonzero status throws Error(dj_last_error()), whose
// text already reads "decision.js: ..." as the reference's errors do (gpu.ts:260, d1.ts:68).
//
// recFinishAsync runs dj_rec_finish on the libuv thread pool and returns a Promise, so a forward does not
// block the event loop; the D1 queue keeps one forward in flight per engine (d1.ts:112-119), which is what the
// library requires of a context. Built with plain g++ against /usr/include/node (see build.py).
#include <node_api.h>
#include <stdint.h>
#include <string.h>

#include <string>
#include <vector>

#include "dj.h"

namespace {

constexpr size_t kMaxArgs = 24;

struct Call {
  napi_env env;
  size_t argc = kMaxArgs;
  napi_value argv[kMaxArgs];
  bool ok = true;
};

bool fail(napi_env env, const char *msg) {
  bool pending = false;
  napi_is_exception_pending(env, &pending);
  if (!pending) napi_throw_error(env, nullptr, msg);
  return false;
}

bool args(napi_env env, napi_callback_info info, Call &c, size_t need) {
  c.env = env;
  if (napi_get_cb_info(env, info, &c.argc, c.argv, nullptr, nullptr) != napi_ok) return fail(env, "decision.js: bad call");
  if (need > kMaxArgs) return fail(env, "decision.js: binding takes more arguments than the call buffer holds");
  if (c.argc < need) {
    std::string m = "decision.js: expected " + std::to_string(need) + " arguments, got " + std::to_string(c.argc);
    return fail(env, m.c_str());
  }
  return true;
}

// A device pointer or handle: BigInt, or null / undefined / 0 for a null pointer.
void *ptr(Call &c, size_t i) {
  napi_valuetype t;
  napi_typeof(c.env, c.argv[i], &t);
  if (t == napi_null || t == napi_undefined) return nullptr;
  if (t == napi_number) {
    double d;
    napi_get_value_double(c.env, c.argv[i], &d);
    if (d == 0) return nullptr;
  }
  if (t != napi_bigint) {
    c.ok = fail(c.env, "decision.js: a device pointer or handle must be a BigInt");
    return nullptr;
  }
  uint64_t v;
  bool lossless;
  napi_get_value_bigint_uint64(c.env, c.argv[i], &v, &lossless);
  return (void *)(uintptr_t)v;
}

int64_t num(Call &c, size_t i) {
  napi_valuetype t;
  napi_typeof(c.env, c.argv[i], &t);
  if (t == napi_boolean) {
    bool b;
    napi_get_value_bool(c.env, c.argv[i], &b);
    return b ? 1 : 0;
  }
  if (t == napi_bigint) {
    int64_t v;
    bool lossless;
    napi_get_value_bigint_int64(c.env, c.argv[i], &v, &lossless);
    return v;
  }
  double d;
  if (napi_get_value_double(c.env, c.argv[i], &d) != napi_ok) c.ok = fail(c.env, "decision.js: expected a number");
  return (int64_t)d;
}

double real(Call &c, size_t i) {
  double d;
  if (napi_get_value_double(c.env, c.argv[i], &d) != napi_ok) c.ok = fail(c.env, "decision.js: expected a number");
  return d;
}

// The bytes of a typed array (or Buffer).
void *bytes(Call &c, size_t i, size_t *n) {
  bool is;
  napi_is_typedarray(c.env, c.argv[i], &is);
  if (!is) {
    c.ok = fail(c.env, "decision.js: expected a typed array");
    return nullptr;
  }
  napi_typedarray_type type;
  size_t length, offset;
  void *data;
  napi_value ab;
  napi_get_typedarray_info(c.env, c.argv[i], &type, &length, &data, &ab, &offset);
  size_t el = 1;
  switch (type) {
    case napi_int16_array: case napi_uint16_array: el = 2; break;
    case napi_int32_array: case napi_uint32_array: case napi_float32_array: el = 4; break;
    case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: el = 8; break;
    default: el = 1;
  }
  *n = length * el;
  return data;
}

napi_value big(napi_env env, const void *p) {
  napi_value v;
  napi_create_bigint_uint64(env, (uint64_t)(uintptr_t)p, &v);
  return v;
}

napi_value undef(napi_env env) {
  napi_value v;
  napi_get_undefined(env, &v);
  return v;
}

napi_value number(napi_env env, double d) {
  napi_value v;
  napi_create_double(env, d, &v);
  return v;
}

// The status of a C call: throw on failure.
napi_value done(napi_env env, int st, napi_value ok = nullptr) {
  if (st != DJ_OK) {
    fail(env, dj_last_error());
    return nullptr;
  }
  return ok ? ok : undef(env);
}

#define BEGIN(need)          \
  Call c;                    \
  if (!args(env, info, c, need)) return nullptr;
#define END(expr)                        \
  if (!c.ok) return nullptr;             \
  return done(env, (expr));

dj_kv_src kvsrc(Call &c, size_t i) {
  dj_kv_src s{};
  napi_value v = c.argv[i], f;
  auto field = [&](const char *name) -> napi_value {
    napi_get_named_property(c.env, v, name, &f);
    return f;
  };
  Call one;
  one.env = c.env;
  one.argc = 1;
  one.argv[0] = field("base");
  s.base = (const uint16_t *)ptr(one, 0);
  one.argv[0] = field("rows");
  s.rows = (int)num(one, 0);
  one.argv[0] = field("stride");
  s.stride = (int)num(one, 0);
  one.argv[0] = field("kCol");
  s.k_col = (int)num(one, 0);
  one.argv[0] = field("vCol");
  s.v_col = (int)num(one, 0);
  if (!one.ok) c.ok = false;
  return s;
}

// ---------------------------------------------------------------- context, buffers, weights

napi_value LastError(napi_env env, napi_callback_info) {
  napi_value v;
  napi_create_string_utf8(env, dj_last_error(), NAPI_AUTO_LENGTH, &v);
  return v;
}

napi_value AbiVersion(napi_env env, napi_callback_info) { return number(env, dj_abi_version()); }

napi_value Init(napi_env env, napi_callback_info info) {
  BEGIN(1);
  dj_ctx *ctx = nullptr;
  const int st = dj_init((int)num(c, 0), &ctx);
  if (!c.ok) return nullptr;
  return done(env, st, big(env, ctx));
}

napi_value Destroy(napi_env env, napi_callback_info info) {
  BEGIN(1);
  END(dj_destroy((dj_ctx *)ptr(c, 0)));
}

napi_value DeviceInfo(napi_env env, napi_callback_info info) {
  BEGIN(1);
  char name[128] = {0};
  int cus = 0;
  size_t mem = 0;
  const int st = dj_device_info((dj_ctx *)ptr(c, 0), name, sizeof name, &cus, &mem);
  if (!c.ok || st != DJ_OK) return done(env, st);
  napi_value o, v;
  napi_create_object(env, &o);
  napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &v);
  napi_set_named_property(env, o, "arch", v);
  napi_set_named_property(env, o, "computeUnits", number(env, cus));
  napi_set_named_property(env, o, "memory", number(env, (double)mem));
  return o;
}

napi_value BufAlloc(napi_env env, napi_callback_info info) {
  BEGIN(2);
  void *p = nullptr;
  const int st = dj_buf_alloc((dj_ctx *)ptr(c, 0), (size_t)num(c, 1), &p);
  if (!c.ok) return nullptr;
  return done(env, st, big(env, p));
}

napi_value BufFree(napi_env env, napi_callback_info info) {
  BEGIN(2);
  END(dj_buf_free((dj_ctx *)ptr(c, 0), ptr(c, 1)));
}

napi_value BufWrite(napi_env env, napi_callback_info info) {  // (ctx, dev, typedArray)
  BEGIN(3);
  size_t n = 0;
  const void *h = bytes(c, 2, &n);
  END(dj_buf_write((dj_ctx *)ptr(c, 0), ptr(c, 1), h, n));
}

napi_value BufRead(napi_env env, napi_callback_info info) {  // (ctx, typedArray, dev): fills the array
  BEGIN(3);
  size_t n = 0;
  void *h = bytes(c, 1, &n);
  END(dj_buf_read((dj_ctx *)ptr(c, 0), h, ptr(c, 2), n));
}

napi_value Upload(napi_env env, napi_callback_info info) {  // (ctx, dev, typedArray)
  BEGIN(3);
  size_t n = 0;
  const void *h = bytes(c, 2, &n);
  END(dj_upload((dj_ctx *)ptr(c, 0), ptr(c, 1), h, n));
}

napi_value BufCopy(napi_env env, napi_callback_info info) {  // (ctx, dst, src, bytes)
  BEGIN(4);
  END(dj_buf_copy((dj_ctx *)ptr(c, 0), ptr(c, 1), ptr(c, 2), (size_t)num(c, 3)));
}

napi_value WeightQ(napi_env env, napi_callback_info info) {  // (ctx, codes, scales, N, K, bits, layout)
  BEGIN(7);
  size_t nc = 0, ns = 0;
  const void *codes = bytes(c, 1, &nc);
  const void *scales = bytes(c, 2, &ns);
  const int N = (int)num(c, 3), K = (int)num(c, 4), bits = (int)num(c, 5), layout = (int)num(c, 6);
  if (!c.ok) return nullptr;
  if ((bits != 8 && bits != 4) || N <= 0 || K <= 0 || nc != (size_t)N * K * bits / 8 || ns != (size_t)N * (K / 32) * 2) {
    fail(env, "decision.js: weight codes/scales do not match N x K at this bit width");
    return nullptr;
  }
  dj_weight *w = nullptr;
  const int st = dj_weight_q((dj_ctx *)ptr(c, 0), codes, scales, N, K, bits, layout, &w);
  return done(env, st, big(env, w));
}

napi_value WeightFree(napi_env env, napi_callback_info info) {
  BEGIN(2);
  END(dj_weight_free((dj_ctx *)ptr(c, 0), (dj_weight *)ptr(c, 1)));
}

napi_value WeightBytes(napi_env env, napi_callback_info info) {
  BEGIN(1);
  const void *w = ptr(c, 0);
  if (!c.ok) return nullptr;
  return number(env, (double)dj_weight_bytes((const dj_weight *)w));
}

// ---------------------------------------------------------------- recorder

napi_value RecBegin(napi_env env, napi_callback_info info) {  // (ctx, key BigInt) -> [rec, replay]
  BEGIN(2);
  dj_rec *rec = nullptr;
  int replay = 0;
  const int st = dj_rec_begin((dj_ctx *)ptr(c, 0), (uint64_t)num(c, 1), &rec, &replay);
  if (!c.ok || st != DJ_OK) return done(env, st);
  napi_value a, r;
  napi_create_array_with_length(env, 2, &a);
  napi_set_element(env, a, 0, big(env, rec));
  napi_get_boolean(env, replay != 0, &r);
  napi_set_element(env, a, 1, r);
  return a;
}

napi_value RecSnapshot(napi_env env, napi_callback_info info) {  // (rec, dev, typedArray): filled at finish
  BEGIN(3);
  size_t n = 0;
  void *h = bytes(c, 2, &n);
  END(dj_rec_snapshot((dj_rec *)ptr(c, 0), ptr(c, 1), n, h));
}

napi_value RecFinish(napi_env env, napi_callback_info info) {
  BEGIN(1);
  END(dj_rec_finish((dj_rec *)ptr(c, 0)));
}

struct FinishWork {
  napi_async_work work;
  napi_deferred deferred;
  dj_rec *rec;
  int status;
  std::string error;  // dj_last_error is per thread: copied on the worker
};

void finish_execute(napi_env, void *data) {
  FinishWork *w = (FinishWork *)data;
  w->status = dj_rec_finish(w->rec);
  if (w->status != DJ_OK) w->error = dj_last_error();
}

void finish_complete(napi_env env, napi_status, void *data) {
  FinishWork *w = (FinishWork *)data;
  if (w->status == DJ_OK) {
    napi_resolve_deferred(env, w->deferred, undef(env));
  } else {
    napi_value msg, err;
    napi_create_string_utf8(env, w->error.c_str(), NAPI_AUTO_LENGTH, &msg);
    napi_create_error(env, nullptr, msg, &err);
    napi_reject_deferred(env, w->deferred, err);
  }
  napi_delete_async_work(env, w->work);
  delete w;
}

napi_value RecFinishAsync(napi_env env, napi_callback_info info) {
  BEGIN(1);
  FinishWork *w = new FinishWork();
  w->rec = (dj_rec *)ptr(c, 0);
  if (!c.ok) {
    delete w;
    return nullptr;
  }
  napi_value promise, name;
  napi_create_promise(env, &w->deferred, &promise);
  napi_create_string_utf8(env, "dj_rec_finish", NAPI_AUTO_LENGTH, &name);
  napi_create_async_work(env, nullptr, name, finish_execute, finish_complete, w, &w->work);
  napi_queue_async_work(env, w->work);
  return promise;
}

napi_value RecAbort(napi_env env, napi_callback_info info) {  // (rec)
  BEGIN(1);
  END(dj_rec_abort((dj_rec *)ptr(c, 0)));
}

napi_value GraphClear(napi_env env, napi_callback_info info) {
  BEGIN(1);
  END(dj_graph_clear((dj_ctx *)ptr(c, 0)));
}

napi_value GraphDrop(napi_env env, napi_callback_info info) {  // (ctx, key BigInt)
  BEGIN(2);
  END(dj_graph_drop((dj_ctx *)ptr(c, 0), (uint64_t)num(c, 1)));
}

napi_value GraphCount(napi_env env, napi_callback_info info) {  // (ctx) -> number of cached graphs
  BEGIN(1);
  int n = 0;
  const int st = dj_graph_count((dj_ctx *)ptr(c, 0), &n);
  if (!c.ok) return nullptr;
  return done(env, st, number(env, n));
}

napi_value TimerBegin(napi_env env, napi_callback_info info) {
  BEGIN(1);
  END(dj_timer_begin((dj_ctx *)ptr(c, 0)));
}

napi_value TimerEnd(napi_env env, napi_callback_info info) {
  BEGIN(1);
  float ms = 0;
  const int st = dj_timer_end((dj_ctx *)ptr(c, 0), &ms);
  if (!c.ok) return nullptr;
  return done(env, st, number(env, ms));
}

napi_value ProfileEnable(napi_env env, napi_callback_info info) {
  BEGIN(2);
  END(dj_profile_enable((dj_ctx *)ptr(c, 0), (int)num(c, 1)));
}

napi_value ProfileReset(napi_env env, napi_callback_info info) {
  BEGIN(1);
  END(dj_profile_reset((dj_ctx *)ptr(c, 0)));
}

napi_value ProfileGet(napi_env env, napi_callback_info info) {  // -> [{name, ms, launches}]
  BEGIN(1);
  std::vector<dj_profile_entry> e(1024);
  int n = 0;
  const int st = dj_profile_get((dj_ctx *)ptr(c, 0), e.data(), (int)e.size(), &n);
  if (!c.ok || st != DJ_OK) return done(env, st);
  napi_value a;
  napi_create_array_with_length(env, n, &a);
  for (int i = 0; i < n; ++i) {
    napi_value o, s;
    napi_create_object(env, &o);
    napi_create_string_utf8(env, e[i].name, NAPI_AUTO_LENGTH, &s);
    napi_set_named_property(env, o, "name", s);
    napi_set_named_property(env, o, "ms", number(env, e[i].ms));
    napi_set_named_property(env, o, "launches", number(env, (double)e[i].launches));
    napi_set_element(env, a, i, o);
  }
  return a;
}

// ---------------------------------------------------------------- ops (argument order of include/dj.h)

#define R(i) ((dj_rec *)ptr(c, i))
#define P16(i) ((uint16_t *)ptr(c, i))
#define PU32(i) ((uint32_t *)ptr(c, i))
#define PI32(i) ((int32_t *)ptr(c, i))
#define PF32(i) ((float *)ptr(c, i))
#define W(i) ((const dj_weight *)ptr(c, i))
#define I(i) ((int)num(c, i))
#define F(i) ((float)real(c, i))

napi_value GatherQ(napi_env env, napi_callback_info info) {
  BEGIN(5);
  END(dj_gather_q(R(0), PU32(1), I(2), W(3), P16(4)));
}
napi_value AddRmsnorm(napi_env env, napi_callback_info info) {
  BEGIN(9);
  END(dj_add_rmsnorm(R(0), I(1), I(2), I(3), F(4), P16(5), P16(6), P16(7), P16(8)));
}
napi_value Sandwich(napi_env env, napi_callback_info info) {
  BEGIN(10);
  END(dj_sandwich(R(0), I(1), I(2), F(3), F(4), P16(5), P16(6), P16(7), P16(8), P16(9)));
}
napi_value Matmul(napi_env env, napi_callback_info info) {
  BEGIN(5);
  END(dj_matmul(R(0), P16(1), W(2), P16(3), I(4)));
}
napi_value MatmulGlu(napi_env env, napi_callback_info info) {
  BEGIN(6);
  END(dj_matmul_glu(R(0), P16(1), W(2), P16(3), I(4), I(5)));
}
napi_value QkNormRope(napi_env env, napi_callback_info info) {
  BEGIN(16);
  END(dj_qk_norm_rope(R(0), I(1), I(2), I(3), I(4), I(5), P16(6), P16(7), P16(8), I(9), PI32(10), I(11), F(12), F(13),
                      I(14), I(15)));
}
napi_value RopeTable(napi_env env, napi_callback_info info) {
  BEGIN(8);
  END(dj_rope_table(R(0), I(1), PI32(2), I(3), F(4), I(5), I(6), PF32(7)));
}
napi_value MatmulQkvRope(napi_env env, napi_callback_info info) {
  BEGIN(18);
  END(dj_matmul_qkv_rope(R(0), P16(1), W(2), P16(3), I(4), I(5), I(6), I(7), P16(8), P16(9), I(10), PI32(11), I(12),
                         F(13), F(14), I(15), I(16), PF32(17)));
}
napi_value MatmulResidual(napi_env env, napi_callback_info info) {
  BEGIN(8);
  END(dj_matmul_residual(R(0), P16(1), W(2), I(3), P16(4), P16(5), P16(6), PF32(7)));
}
napi_value MatmulNormed(napi_env env, napi_callback_info info) {
  BEGIN(9);
  END(dj_matmul_normed(R(0), P16(1), W(2), P16(3), I(4), I(5), PF32(6), I(7), F(8)));
}
napi_value MatmulQkvRopeNormed(napi_env env, napi_callback_info info) {
  BEGIN(21);
  END(dj_matmul_qkv_rope_normed(R(0), P16(1), W(2), P16(3), I(4), I(5), I(6), I(7), P16(8), P16(9), I(10), PI32(11), I(12),
                                F(13), F(14), I(15), I(16), PF32(17), PF32(18), I(19), F(20)));
}
napi_value Attention(napi_env env, napi_callback_info info) {
  BEGIN(12);
  const dj_kv_src a = kvsrc(c, 7), b = kvsrc(c, 8);
  END(dj_attention(R(0), I(1), I(2), I(3), I(4), P16(5), I(6), a, b, PI32(9), F(10), P16(11)));
}

napi_value AttentionNoalloc(napi_env env, napi_callback_info info) {
  BEGIN(12);
  const dj_kv_src a = kvsrc(c, 7), b = kvsrc(c, 8);
  END(dj_attention_noalloc(R(0), I(1), I(2), I(3), I(4), P16(5), I(6), a, b, PI32(9), F(10), P16(11)));
}
napi_value AttentionQkRope(napi_env env, napi_callback_info info) {
  BEGIN(17);
  const dj_kv_src a = kvsrc(c, 7), b = kvsrc(c, 8);
  END(dj_attention_qk_rope(R(0), I(1), I(2), I(3), I(4), P16(5), I(6), a, b, PI32(9), F(10), P16(11), P16(12), F(13),
                           PF32(14), I(15), P16(16)));
}
napi_value AttentionGated(napi_env env, napi_callback_info info) {
  BEGIN(14);
  const dj_kv_src a = kvsrc(c, 7), b = kvsrc(c, 8);
  END(dj_attention_gated(R(0), I(1), I(2), I(3), I(4), P16(5), I(6), a, b, PI32(9), F(10), P16(11), I(12), P16(13)));
}

napi_value Gdn(napi_env env, napi_callback_info info) {
  BEGIN(13);
  END(dj_gdn(R(0), I(1), I(2), PU32(3), I(4), I(5), P16(6), P16(7), P16(8), P16(9), P16(10), F(11), P16(12)));
}

napi_value PleMix(napi_env env, napi_callback_info info) {
  BEGIN(8);
  END(dj_ple_mix(R(0), I(1), I(2), P16(3), P16(4), P16(5), F(6), P16(7)));
}

napi_value PoolProject(napi_env env, napi_callback_info info) {
  BEGIN(9);
  END(dj_pool_project(R(0), I(1), I(2), I(3), I(4), P16(5), PU32(6), P16(7), PF32(8)));
}

napi_value KvStore(napi_env env, napi_callback_info info) {
  BEGIN(9);
  END(dj_kv_store(R(0), I(1), I(2), I(3), P16(4), I(5), I(6), P16(7), I(8)));
}
napi_value LeafLogits(napi_env env, napi_callback_info info) {
  BEGIN(12);
  END(dj_leaf_logits(R(0), I(1), I(2), I(3), I(4), F(5), P16(6), PU32(7), P16(8), PU32(9), W(10), PF32(11)));
}
napi_value AddRows(napi_env env, napi_callback_info info) {
  BEGIN(8);
  END(dj_add_rows(R(0), I(1), I(2), P16(3), PU32(4), P16(5), I(6), P16(7)));
}

napi_value BiasAct(napi_env env, napi_callback_info info) {
  BEGIN(6);
  END(dj_bias_act(R(0), I(1), I(2), P16(3), P16(4), I(5)));
}

napi_value AddLayernorm(napi_env env, napi_callback_info info) {
  BEGIN(10);
  END(dj_add_layernorm(R(0), I(1), I(2), I(3), F(4), P16(5), P16(6), P16(7), P16(8), P16(9)));
}

napi_value GatherRows(napi_env env, napi_callback_info info) {
  BEGIN(7);
  END(dj_gather_rows(R(0), I(1), I(2), I(3), P16(4), PU32(5), P16(6)));
}

napi_value Score(napi_env env, napi_callback_info info) {
  BEGIN(7);
  END(dj_score(R(0), I(1), I(2), P16(3), P16(4), P16(5), PF32(6)));
}

napi_value ShortConv(napi_env env, napi_callback_info info) {
  BEGIN(7);
  END(dj_short_conv(R(0), I(1), I(2), P16(3), P16(4), PI32(5), P16(6)));
}

napi_value Readout(napi_env env, napi_callback_info info) {
  BEGIN(9);
  END(dj_readout(R(0), I(1), I(2), I(3), P16(4), PF32(5), I(6), PU32(7), PF32(8)));
}
napi_value MeanPool(napi_env env, napi_callback_info info) {
  BEGIN(7);
  END(dj_mean_pool(R(0), I(1), I(2), I(3), P16(4), PU32(5), PF32(6)));
}
napi_value DenseF32(napi_env env, napi_callback_info info) {
  BEGIN(5);
  END(dj_dense_f32(R(0), I(1), PF32(2), W(3), PF32(4)));
}

napi_value Module(napi_env env, napi_value exports) {
  const struct {
    const char *name;
    napi_callback fn;
  } fns[] = {
      {"lastError", LastError}, {"abiVersion", AbiVersion}, {"init", Init}, {"destroy", Destroy},
      {"deviceInfo", DeviceInfo}, {"bufAlloc", BufAlloc}, {"bufFree", BufFree}, {"bufWrite", BufWrite},
      {"bufRead", BufRead}, {"upload", Upload}, {"bufCopy", BufCopy}, {"weightQ", WeightQ},
      {"weightFree", WeightFree}, {"weightBytes", WeightBytes}, {"recBegin", RecBegin},
      {"recSnapshot", RecSnapshot}, {"recFinish", RecFinish}, {"recFinishAsync", RecFinishAsync},
      {"recAbort", RecAbort}, {"graphClear", GraphClear}, {"graphDrop", GraphDrop}, {"graphCount", GraphCount},
      {"timerBegin", TimerBegin}, {"timerEnd", TimerEnd},
      {"profileEnable", ProfileEnable}, {"profileGet", ProfileGet}, {"profileReset", ProfileReset},
      {"gatherQ", GatherQ}, {"addRmsnorm", AddRmsnorm}, {"sandwich", Sandwich}, {"matmul", Matmul},
      {"matmulGlu", MatmulGlu}, {"qkNormRope", QkNormRope}, {"ropeTable", RopeTable}, {"matmulQkvRope", MatmulQkvRope}, {"matmulResidual", MatmulResidual}, {"matmulNormed", MatmulNormed}, {"matmulQkvRopeNormed", MatmulQkvRopeNormed}, {"attention", Attention}, {"attentionNoalloc", AttentionNoalloc}, {"attentionQkRope", AttentionQkRope}, {"kvStore", KvStore},
      {"leafLogits", LeafLogits}, {"readout", Readout}, {"shortConv", ShortConv}, {"attentionGated", AttentionGated}, {"gdn", Gdn}, {"pleMix", PleMix},
      {"poolProject", PoolProject}, {"addRows", AddRows}, {"biasAct", BiasAct},
      {"addLayernorm", AddLayernorm}, {"gatherRows", GatherRows}, {"score", Score}, {"meanPool", MeanPool}, {"denseF32", DenseF32},
  };
  for (const auto &f : fns) {
    napi_value v;
    napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.fn, nullptr, &v);
    napi_set_named_property(env, exports, f.name, v);
  }
  const struct {
    const char *name;
    int value;
  } consts[] = {{"W_PLAIN", DJ_W_PLAIN}, {"W_MFMA", DJ_W_MFMA}, {"W_MFMA_GLU", DJ_W_MFMA_GLU},
                {"W_DIRECT", DJ_W_DIRECT}, {"ACT_SILU", DJ_ACT_SILU}, {"ACT_GELU_TANH", DJ_ACT_GELU_TANH}, {"ACT_GELU_ERF", DJ_ACT_GELU_ERF},
                {"ROPE_POW_NEG", DJ_ROPE_POW_NEG}, {"ROPE_INV_POW", DJ_ROPE_INV_POW},
                {"BIAS_NONE", DJ_BIAS_NONE}, {"BIAS_RELU", DJ_BIAS_RELU}, {"BIAS_GELU_ERF", DJ_BIAS_GELU_ERF}, {"ABI_VERSION", DJ_ABI_VERSION}};
  for (const auto &k : consts) napi_set_named_property(env, exports, k.name, number(env, k.value));
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Module)
