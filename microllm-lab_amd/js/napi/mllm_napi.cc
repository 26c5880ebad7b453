// mllm_napi.cc -- Node-API binding of libmllm (include/mllm.h).
//
// The thin shim between the JavaScript engine (js/engine.mjs, the PetitGPT API
// of engine/infer.js) and the C ABI.  Every call is synchronous and throws a
// JS Error carrying mllm_last_error() on a non-zero status.  Typed arrays are
// passed by pointer without copies; the model handle is a napi_external whose
// finaliser frees the device memory if JS never calls destroy().
#include <node_api.h>
#include <stdint.h>
#include <string.h>

#include <string>
#include <vector>

#include "mllm.h"

namespace {

struct Handle {
  mllm_model *model = nullptr;
  std::vector<std::string> names;  // keep tensor-name storage alive
};

#define NAPI_OK(call)                                  \
  do {                                                 \
    if ((call) != napi_ok) {                           \
      napi_throw_error(env, nullptr, "N-API failure: " #call); \
      return nullptr;                                  \
    }                                                  \
  } while (0)

napi_value throw_mllm(napi_env env, const char *fn, int rc) {
  std::string msg = std::string(fn) + " failed (" + std::to_string(rc) + "): " + mllm_last_error();
  napi_throw_error(env, nullptr, msg.c_str());
  return nullptr;
}

#define MLLM_OK_OR_THROW(fn, call)           \
  do {                                       \
    int rc_ = (call);                        \
    if (rc_ != 0) return throw_mllm(env, fn, rc_); \
  } while (0)

bool get_args(napi_env env, napi_callback_info info, size_t want, napi_value *argv) {
  size_t argc = want;
  if (napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr) != napi_ok) return false;
  for (size_t i = argc; i < want; ++i) napi_get_undefined(env, &argv[i]);
  return true;
}

Handle *get_handle(napi_env env, napi_value v) {
  void *p = nullptr;
  if (napi_get_value_external(env, v, &p) != napi_ok || !p) {
    napi_throw_type_error(env, nullptr, "expected a model handle");
    return nullptr;
  }
  Handle *h = static_cast<Handle *>(p);
  if (!h->model) {
    napi_throw_error(env, nullptr, "model was destroyed");
    return nullptr;
  }
  return h;
}

bool is_nullish(napi_env env, napi_value v) {
  napi_valuetype t;
  napi_typeof(env, v, &t);
  return t == napi_undefined || t == napi_null;
}

// Typed-array view: data pointer and element count, with a type check.
template <typename T>
bool typed(napi_env env, napi_value v, napi_typedarray_type want, T **data, size_t *len) {
  bool is = false;
  napi_is_typedarray(env, v, &is);
  if (!is) {
    napi_throw_type_error(env, nullptr, "expected a typed array");
    return false;
  }
  napi_typedarray_type type;
  size_t length = 0, offset = 0;
  void *ptr = nullptr;
  napi_value ab;
  napi_get_typedarray_info(env, v, &type, &length, &ptr, &ab, &offset);
  if (type != want) {
    napi_throw_type_error(env, nullptr, want == napi_float32_array ? "expected a Float32Array" : "expected an Int32Array");
    return false;
  }
  *data = static_cast<T *>(ptr);
  *len = length;
  return true;
}

int32_t get_i32(napi_env env, napi_value v, int32_t dflt = 0) {
  int32_t out = dflt;
  napi_get_value_int32(env, v, &out);
  return out;
}

double get_prop_num(napi_env env, napi_value obj, const char *key, double dflt) {
  bool has = false;
  napi_has_named_property(env, obj, key, &has);
  if (!has) return dflt;
  napi_value v;
  napi_get_named_property(env, obj, key, &v);
  double d = dflt;
  if (napi_get_value_double(env, v, &d) != napi_ok) return dflt;
  return d;
}

std::string get_prop_str(napi_env env, napi_value obj, const char *key) {
  napi_value v;
  if (napi_get_named_property(env, obj, key, &v) != napi_ok) return "";
  size_t n = 0;
  if (napi_get_value_string_utf8(env, v, nullptr, 0, &n) != napi_ok) return "";
  std::string s(n, '\0');
  napi_get_value_string_utf8(env, v, &s[0], n + 1, &n);
  return s;
}

void finalize_handle(napi_env, void *data, void *) {
  Handle *h = static_cast<Handle *>(data);
  if (h->model) mllm_model_destroy(h->model);
  delete h;
}

napi_value make_int(napi_env env, int64_t v) {
  napi_value out;
  napi_create_int64(env, v, &out);
  return out;
}

// createModel(cfg, payload: Uint8Array, tensors: [{name, storage, rows, cols, group,
//             offset, nbytes, scaleOffset, scaleNbytes}]) -> handle
napi_value CreateModel(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!get_args(env, info, 3, argv)) return nullptr;
  mllm_config cfg;
  memset(&cfg, 0, sizeof cfg);
  cfg.arch = (int32_t)get_prop_num(env, argv[0], "arch", 0);
  cfg.vocab_size = (int32_t)get_prop_num(env, argv[0], "vocabSize", 0);
  cfg.n_layers = (int32_t)get_prop_num(env, argv[0], "nLayers", 0);
  cfg.d_model = (int32_t)get_prop_num(env, argv[0], "dModel", 0);
  cfg.n_heads = (int32_t)get_prop_num(env, argv[0], "nHeads", 0);
  cfg.n_kv_heads = (int32_t)get_prop_num(env, argv[0], "nKvHeads", 0);
  cfg.d_ff = (int32_t)get_prop_num(env, argv[0], "dFf", 0);
  cfg.max_seq_len = (int32_t)get_prop_num(env, argv[0], "maxSeqLen", 0);
  cfg.rope_theta = get_prop_num(env, argv[0], "ropeTheta", 10000.0);
  cfg.rope_pct = get_prop_num(env, argv[0], "ropePct", 1.0);
  cfg.norm_eps = (float)get_prop_num(env, argv[0], "normEps", 1e-6);
  cfg.kv_fp16 = (int32_t)get_prop_num(env, argv[0], "kvFp16", 0);

  bool is = false;
  napi_is_typedarray(env, argv[1], &is);
  if (!is) {
    napi_throw_type_error(env, nullptr, "payload must be a Uint8Array");
    return nullptr;
  }
  napi_typedarray_type type;
  size_t plen = 0, poff = 0;
  void *pdata = nullptr;
  napi_value ab;
  NAPI_OK(napi_get_typedarray_info(env, argv[1], &type, &plen, &pdata, &ab, &poff));

  uint32_t n = 0;
  NAPI_OK(napi_get_array_length(env, argv[2], &n));
  Handle *h = new Handle();
  h->names.resize(n);
  std::vector<mllm_tensor> ts(n);
  for (uint32_t i = 0; i < n; ++i) {
    napi_value e;
    NAPI_OK(napi_get_element(env, argv[2], i, &e));
    h->names[i] = get_prop_str(env, e, "name");
    mllm_tensor &t = ts[i];
    t.name = h->names[i].c_str();
    t.storage = (int32_t)get_prop_num(env, e, "storage", 0);
    t.rows = (int32_t)get_prop_num(env, e, "rows", 0);
    t.cols = (int32_t)get_prop_num(env, e, "cols", 0);
    t.group = (int32_t)get_prop_num(env, e, "group", 32);
    t.offset = (uint64_t)get_prop_num(env, e, "offset", 0);
    t.nbytes = (uint64_t)get_prop_num(env, e, "nbytes", 0);
    t.scale_offset = (uint64_t)get_prop_num(env, e, "scaleOffset", 0);
    t.scale_nbytes = (uint64_t)get_prop_num(env, e, "scaleNbytes", 0);
  }
  int rc = mllm_model_create(&cfg, pdata, plen, ts.data(), (int)n, &h->model);
  if (rc != 0) {
    delete h;
    return throw_mllm(env, "mllm_model_create", rc);
  }
  napi_value out;
  NAPI_OK(napi_create_external(env, h, finalize_handle, nullptr, &out));
  return out;
}

napi_value Destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return nullptr;
  void *p = nullptr;
  if (napi_get_value_external(env, argv[0], &p) == napi_ok && p) {
    Handle *h = static_cast<Handle *>(p);
    if (h->model) mllm_model_destroy(h->model);
    h->model = nullptr;
  }
  return nullptr;
}

napi_value ResetCache(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return nullptr;
  Handle *h = get_handle(env, argv[0]);
  if (!h) return nullptr;
  MLLM_OK_OR_THROW("mllm_reset_cache", mllm_reset_cache(h->model));
  return nullptr;
}

napi_value CacheLen(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return nullptr;
  Handle *h = get_handle(env, argv[0]);
  if (!h) return nullptr;
  return make_int(env, mllm_cache_len(h->model));
}

napi_value SetCacheLen(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return nullptr;
  Handle *h = get_handle(env, argv[0]);
  if (!h) return nullptr;
  MLLM_OK_OR_THROW("mllm_set_cache_len", mllm_set_cache_len(h->model, get_i32(env, argv[1])));
  return nullptr;
}

// forwardPrompt(h, ids: Int32Array, logits: Float32Array) -> argmax
napi_value ForwardPrompt(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!get_args(env, info, 3, argv)) return nullptr;
  Handle *h = get_handle(env, argv[0]);
  if (!h) return nullptr;
  int32_t *ids;
  float *logits = nullptr;
  size_t n, nl;
  if (!typed(env, argv[1], napi_int32_array, &ids, &n)) return nullptr;
  if (!is_nullish(env, argv[2]) && !typed(env, argv[2], napi_float32_array, &logits, &nl)) return nullptr;
  int32_t am = 0;
  MLLM_OK_OR_THROW("mllm_forward_prompt", mllm_forward_prompt(h->model, ids, (int)n, logits, &am));
  return make_int(env, am);
}

// forwardDecode(h, id, logits: Float32Array | null) -> argmax
napi_value ForwardDecode(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!get_args(env, info, 3, argv)) return nullptr;
  Handle *h = get_handle(env, argv[0]);
  if (!h) return nullptr;
  float *logits = nullptr;
  size_t nl;
  if (!is_nullish(env, argv[2]) && !typed(env, argv[2], napi_float32_array, &logits, &nl)) return nullptr;
  int32_t am = 0;
  MLLM_OK_OR_THROW("mllm_forward_decode", mllm_forward_decode(h->model, get_i32(env, argv[1]), logits, &am));
  return make_int(env, am);
}

// forwardVerify(h, ids: Int32Array, argmax: Int32Array, logits: Float32Array | null)
napi_value ForwardVerify(napi_env env, napi_callback_info info) {
  napi_value argv[4];
  if (!get_args(env, info, 4, argv)) return nullptr;
  Handle *h = get_handle(env, argv[0]);
  if (!h) return nullptr;
  int32_t *ids, *am;
  float *logits = nullptr;
  size_t n, na, nl;
  if (!typed(env, argv[1], napi_int32_array, &ids, &n)) return nullptr;
  if (!typed(env, argv[2], napi_int32_array, &am, &na)) return nullptr;
  if (!is_nullish(env, argv[3]) && !typed(env, argv[3], napi_float32_array, &logits, &nl)) return nullptr;
  if (na < n) {
    napi_throw_range_error(env, nullptr, "argmax array shorter than ids");
    return nullptr;
  }
  MLLM_OK_OR_THROW("mllm_forward_verify", mllm_forward_verify(h->model, ids, (int)n, am, logits));
  return nullptr;
}

// decodeChain(h, first, nSteps, eosId, hist: Int32Array | null, out: Int32Array) -> count
napi_value DecodeChain(napi_env env, napi_callback_info info) {
  napi_value argv[6];
  if (!get_args(env, info, 6, argv)) return nullptr;
  Handle *h = get_handle(env, argv[0]);
  if (!h) return nullptr;
  int32_t *hist = nullptr, *out;
  size_t nh = 0, no;
  if (!is_nullish(env, argv[4]) && !typed(env, argv[4], napi_int32_array, &hist, &nh)) return nullptr;
  if (!typed(env, argv[5], napi_int32_array, &out, &no)) return nullptr;
  const int steps = get_i32(env, argv[2]);
  if ((size_t)steps > no) {
    napi_throw_range_error(env, nullptr, "output array shorter than nSteps");
    return nullptr;
  }
  int n_out = 0;
  MLLM_OK_OR_THROW("mllm_decode_chain", mllm_decode_chain(h->model, get_i32(env, argv[1]), steps,
                                                         get_i32(env, argv[3], -1), hist, (int)nh, out, &n_out));
  return make_int(env, n_out);
}

// gemv(h, name, x: Float32Array, y: Float32Array)
napi_value Gemv(napi_env env, napi_callback_info info) {
  napi_value argv[4];
  if (!get_args(env, info, 4, argv)) return nullptr;
  Handle *h = get_handle(env, argv[0]);
  if (!h) return nullptr;
  size_t len = 0;
  napi_get_value_string_utf8(env, argv[1], nullptr, 0, &len);
  std::string name(len, '\0');
  napi_get_value_string_utf8(env, argv[1], &name[0], len + 1, &len);
  float *x, *y;
  size_t nx, ny;
  if (!typed(env, argv[2], napi_float32_array, &x, &nx)) return nullptr;
  if (!typed(env, argv[3], napi_float32_array, &y, &ny)) return nullptr;
  MLLM_OK_OR_THROW("mllm_model_gemv", mllm_model_gemv(h->model, name.c_str(), x, y));
  return nullptr;
}

napi_value SetExecMode(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return nullptr;
  Handle *h = get_handle(env, argv[0]);
  if (!h) return nullptr;
  MLLM_OK_OR_THROW("mllm_set_exec_mode", mllm_set_exec_mode(h->model, get_i32(env, argv[1])));
  return nullptr;
}

napi_value SetPrefill(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!get_args(env, info, 3, argv)) return nullptr;
  Handle *h = get_handle(env, argv[0]);
  if (!h) return nullptr;
  MLLM_OK_OR_THROW("mllm_set_prefill", mllm_set_prefill(h->model, get_i32(env, argv[1]), get_i32(env, argv[2])));
  return nullptr;
}

napi_value SetDebug(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  if (!get_args(env, info, 5, argv)) return nullptr;
  Handle *h = get_handle(env, argv[0]);
  if (!h) return nullptr;
  MLLM_OK_OR_THROW("mllm_set_debug", mllm_set_debug(h->model, get_i32(env, argv[1]), get_i32(env, argv[2]),
                                                    get_i32(env, argv[3]), get_i32(env, argv[4])));
  return nullptr;
}

napi_value LastTiming(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return nullptr;
  Handle *h = get_handle(env, argv[0]);
  if (!h) return nullptr;
  float ms = 0;
  int n = 0;
  MLLM_OK_OR_THROW("mllm_last_timing", mllm_last_timing(h->model, &ms, &n));
  napi_value out, vms, vn;
  napi_create_object(env, &out);
  napi_create_double(env, ms, &vms);
  napi_create_int32(env, n, &vn);
  napi_set_named_property(env, out, "gpuMs", vms);
  napi_set_named_property(env, out, "n", vn);
  return out;
}

napi_value DeviceBytes(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return nullptr;
  Handle *h = get_handle(env, argv[0]);
  if (!h) return nullptr;
  napi_value out;
  napi_create_double(env, (double)mllm_model_device_bytes(h->model), &out);
  return out;
}

napi_value MaxPass(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return nullptr;
  Handle *h = get_handle(env, argv[0]);
  if (!h) return nullptr;
  return make_int(env, mllm_max_pass_tokens(h->model));
}

napi_value Version(napi_env env, napi_callback_info) { return make_int(env, mllm_kernel_version()); }

napi_value Init(napi_env env, napi_value exports) {
  const struct {
    const char *name;
    napi_callback fn;
  } fns[] = {
      {"createModel", CreateModel}, {"destroy", Destroy},           {"resetCache", ResetCache},
      {"cacheLen", CacheLen},       {"setCacheLen", SetCacheLen},   {"forwardPrompt", ForwardPrompt},
      {"forwardDecode", ForwardDecode}, {"forwardVerify", ForwardVerify}, {"decodeChain", DecodeChain},
      {"gemv", Gemv},               {"setExecMode", SetExecMode},   {"setPrefill", SetPrefill},   {"lastTiming", LastTiming},
      {"deviceBytes", DeviceBytes}, {"maxPassTokens", MaxPass},     {"version", Version},
      {"setDebug", SetDebug},
  };
  for (const auto &f : fns) {
    napi_value v;
    napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.fn, nullptr, &v);
    napi_set_named_property(env, exports, f.name, v);
  }
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Init)
