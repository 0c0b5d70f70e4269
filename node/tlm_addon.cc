// Node.js N-API binding of include/tlm.h: the layer a TypeScript
// DecoderHIPRunner (beside createTSLRunner, src/runtime/factory.ts:29-43 of
// the reference) calls.  The addon loads libtlm.so at run time (dlopen:
// $TLM_LIB, else three-llm_amd/libtlm.so of the repository: ../ from the addon
// built in node/, ../../../ from node-gyp's node/build/Release),
// so it builds without ROCm.  Every failing tlm_* call throws an Error whose
// message is tlm_last_error() ("Component: message", like the reference's
// "TSLCompute: ..." errors) and whose `code` is the TLM_ERR_* value.
//
// Exports (camelCase of the C names; handles are opaque externals):
//   abiVersion() lastError() open(device) close(ctx) sync(ctx) deviceInfo(ctx)
//   modelCreate(ctx, desc) modelUpload(model, tensor, layer, typedArray)
//   modelFinalize(model) modelDestroy(model) computeToken(model, token, pos, flags)
//   prefill(model, Int32Array, start, end) readLogits(model, Float32Array)
//   readToken(model) decodeGreedy(model, token, pos, n) resetCache(model)
//   readCandidates(model, k, softcap) quantizeQ4(Float32Array, nOut, kIn)
//   f32ToF16(Float32Array) synthNormal(seed, stream, n, stddev)
//   synthTokens(seed, stream, n, vocab) modelCounts(model)
//   modelSetPrefill(model, minRows, chunk)
// and the reads as Promises, each run on the libuv thread pool so the JS
// thread is not blocked while the device finishes (the counterpart of the
// reference's renderer.getArrayBufferAsync, src/tsl/TSLLogits.ts:71-83,
// 359-377): readLogitsAsync(model, Float32Array) -> the array,
// readTokenAsync(model) -> token, readCandidatesAsync(model, k, softcap) ->
// {tokens, scores}, decodeGreedyAsync(model, token, pos, n) -> Int32Array,
// prefillAsync(model, Int32Array, start, end) -> undefined.
// A failing read rejects with the same Error(tlm_last_error(), code).  While
// a read of a model is pending, every other call on that model throws
// (TLM_ERR_STATE): a model is used by one call at a time.
#include <dlfcn.h>
#include <node_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <utility>

#include "tlm.h"

namespace {

// ------------------------------------------------------------ the library --
struct Api {
  int (*abi_version)(void);
  const char* (*last_error)(void);
  int (*open)(int, tlm_ctx**);
  void (*close)(tlm_ctx*);
  int (*sync)(tlm_ctx*);
  int (*device_info)(tlm_ctx*, char*, size_t, int*);
  int (*model_create)(tlm_ctx*, const tlm_model_desc*, tlm_model**);
  void (*model_destroy)(tlm_model*);
  int (*model_upload)(tlm_model*, int, int, const void*, size_t);
  int (*model_finalize)(tlm_model*);
  int (*model_set_prefill)(tlm_model*, int32_t, int32_t);
  int (*compute_token)(tlm_model*, int32_t, int32_t, int);
  int (*prefill)(tlm_model*, const int32_t*, int32_t, int32_t);
  int (*read_logits)(tlm_model*, float*, size_t);
  int (*read_token)(tlm_model*, int32_t*);
  int (*decode_greedy)(tlm_model*, int32_t, int32_t, int, int32_t*);
  int (*reset_cache)(tlm_model*);
  int (*read_candidates)(tlm_model*, int, double, int32_t*, float*);
  int (*quantize_q4)(const float*, int, int, uint8_t*, uint16_t*);
  int (*f32_to_f16)(const float*, size_t, uint16_t*);
  int (*synth_normal)(uint64_t, uint64_t, size_t, float, float*);
  int (*synth_tokens)(uint64_t, uint64_t, size_t, int32_t, int32_t*);
  int (*model_counts_read)(tlm_model*, tlm_model_counts*);
};
Api g_api;
std::string g_load_error;

template <typename T>
bool bind(void* lib, const char* name, T& fn) {
  fn = reinterpret_cast<T>(dlsym(lib, name));
  if (!fn) g_load_error = std::string("TLMAddon: libtlm.so lacks ") + name;
  return fn != nullptr;
}

std::string addon_dir() {
  Dl_info info;
  if (dladdr(reinterpret_cast<void*>(&addon_dir), &info) && info.dli_fname) {
    std::string p = info.dli_fname;
    const size_t s = p.rfind('/');
    if (s != std::string::npos) return p.substr(0, s);
  }
  return ".";
}

// The structs this file passes (tlm_model_desc, tlm_model_counts) are the
// header's: a library of another ABI version is refused at load.
bool abi_matches() {
  const int v = g_api.abi_version();
  if (v == TLM_ABI_VERSION) return true;
  g_load_error = "TLMAddon: libtlm.so has ABI version " + std::to_string(v) + ", this addon was built for " +
                 std::to_string(TLM_ABI_VERSION);
  return false;
}

bool load_library() {
  const char* env = getenv("TLM_LIB");
  std::string path = env && *env ? env : addon_dir() + "/../three-llm_amd/libtlm.so";
  void* lib = dlopen(path.c_str(), RTLD_NOW | RTLD_LOCAL);
  if (!lib) {  // node-gyp puts the addon in build/Release: one level deeper
    const std::string alt = addon_dir() + "/../../../three-llm_amd/libtlm.so";
    if (!(env && *env)) lib = dlopen(alt.c_str(), RTLD_NOW | RTLD_LOCAL);
    if (!lib) {
      const char* e = dlerror();
      g_load_error = std::string("TLMAddon: cannot load ") + path + ": " + (e ? e : "unknown error");
      return false;
    }
  }
  Api& a = g_api;
  return bind(lib, "tlm_abi_version", a.abi_version) && bind(lib, "tlm_last_error", a.last_error) &&
         bind(lib, "tlm_open", a.open) && bind(lib, "tlm_close", a.close) && bind(lib, "tlm_sync", a.sync) &&
         bind(lib, "tlm_device_info", a.device_info) && bind(lib, "tlm_model_create", a.model_create) &&
         bind(lib, "tlm_model_destroy", a.model_destroy) && bind(lib, "tlm_model_upload", a.model_upload) &&
         bind(lib, "tlm_model_finalize", a.model_finalize) && bind(lib, "tlm_compute_token", a.compute_token) &&
         bind(lib, "tlm_prefill", a.prefill) && bind(lib, "tlm_read_logits", a.read_logits) &&
         bind(lib, "tlm_read_token", a.read_token) && bind(lib, "tlm_decode_greedy", a.decode_greedy) &&
         bind(lib, "tlm_reset_cache", a.reset_cache) && bind(lib, "tlm_read_candidates", a.read_candidates) &&
         bind(lib, "tlm_quantize_q4", a.quantize_q4) && bind(lib, "tlm_f32_to_f16", a.f32_to_f16) &&
         bind(lib, "tlm_synth_normal", a.synth_normal) && bind(lib, "tlm_synth_tokens", a.synth_tokens) &&
         bind(lib, "tlm_model_counts_read", a.model_counts_read) &&
         bind(lib, "tlm_model_set_prefill", a.model_set_prefill) && abi_matches();
}

// ---------------------------------------------------------------- helpers --
// Throws Error(message, code) and returns nullptr (the N-API convention).
napi_value throw_error(napi_env env, int code, const std::string& message) {
  napi_value msg, err, c;
  napi_create_string_utf8(env, message.c_str(), NAPI_AUTO_LENGTH, &msg);
  napi_create_error(env, nullptr, msg, &err);
  napi_create_int32(env, code, &c);
  napi_set_named_property(env, err, "code", c);
  napi_throw(env, err);
  return nullptr;
}

// A tlm_* return code: 0 passes, anything else throws tlm_last_error().
bool check(napi_env env, int rc) {
  if (rc == TLM_OK) return true;
  const char* m = g_api.last_error ? g_api.last_error() : "";
  throw_error(env, rc, m && *m ? m : "TLMAddon: call failed with code " + std::to_string(rc));
  return false;
}

struct Args {
  napi_value v[8];
  size_t n = 8;
  Args(napi_env env, napi_callback_info info) { napi_get_cb_info(env, info, &n, v, nullptr, nullptr); }
};

bool get_i32(napi_env env, napi_value v, int32_t* out, const char* what) {
  if (napi_get_value_int32(env, v, out) != napi_ok) {
    throw_error(env, TLM_ERR_INVALID, std::string("TLMAddon: ") + what + " must be a number");
    return false;
  }
  return true;
}

bool get_f64(napi_env env, napi_value v, double* out, const char* what) {
  if (napi_get_value_double(env, v, out) != napi_ok) {
    throw_error(env, TLM_ERR_INVALID, std::string("TLMAddon: ") + what + " must be a number");
    return false;
  }
  return true;
}

bool get_u64(napi_env env, napi_value v, uint64_t* out, const char* what) {
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t == napi_bigint) {
    bool lossless = true;
    if (napi_get_value_bigint_uint64(env, v, out, &lossless) == napi_ok && lossless) return true;
  } else if (t == napi_number) {
    double d = 0;
    napi_get_value_double(env, v, &d);
    if (d >= 0 && d <= 9007199254740991.0 && d == (double)(uint64_t)d) {
      *out = (uint64_t)d;
      return true;
    }
  }
  throw_error(env, TLM_ERR_INVALID, std::string("TLMAddon: ") + what + " must be a non-negative integer or BigInt");
  return false;
}

// Data pointer and byte length of a typed array of the given type.
bool get_typed(napi_env env, napi_value v, napi_typedarray_type want, void** data, size_t* count, const char* what) {
  bool is = false;
  napi_is_typedarray(env, v, &is);
  napi_typedarray_type t;
  size_t len = 0;
  napi_value ab;
  size_t off = 0;
  if (!is || napi_get_typedarray_info(env, v, &t, &len, data, &ab, &off) != napi_ok || t != want) {
    throw_error(env, TLM_ERR_INVALID, std::string("TLMAddon: ") + what + " has the wrong array type");
    return false;
  }
  *count = len;
  return true;
}

// Any typed array: data and byte length (weights of any format).
bool get_bytes(napi_env env, napi_value v, void** data, size_t* bytes) {
  bool is = false;
  napi_is_typedarray(env, v, &is);
  napi_typedarray_type t;
  size_t len = 0, off = 0;
  napi_value ab;
  if (!is || napi_get_typedarray_info(env, v, &t, &len, data, &ab, &off) != napi_ok) {
    throw_error(env, TLM_ERR_INVALID, "TLMAddon: tensor data must be a typed array");
    return false;
  }
  size_t esz = 1;
  switch (t) {
    case napi_int16_array: case napi_uint16_array: esz = 2; break;
    case napi_int32_array: case napi_uint32_array: case napi_float32_array: esz = 4; break;
    case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: esz = 8; break;
    default: esz = 1;
  }
  *bytes = len * esz;
  return true;
}

napi_value new_typed(napi_env env, napi_typedarray_type t, size_t count, size_t esz, void** data) {
  napi_value ab, arr;
  napi_create_arraybuffer(env, count * esz, data, &ab);
  napi_create_typedarray(env, t, count, ab, 0, &arr);
  return arr;
}

// Opaque handles: an external wrapping a slot, cleared when closed (a second
// close is a no-op, a use after close throws).
struct Handle {
  void* p;
  int kind;      // 1 context, 2 model
  int pending;   // model: reads running on the thread pool
};

napi_value wrap(napi_env env, void* p, int kind) {
  Handle* h = new Handle{p, kind, 0};
  napi_value v;
  napi_create_external(env, h, [](napi_env, void* d, void*) { delete static_cast<Handle*>(d); }, nullptr, &v);
  return v;
}

Handle* unwrap(napi_env env, napi_value v, int kind) {
  void* d = nullptr;
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t != napi_external || napi_get_value_external(env, v, &d) != napi_ok || !d ||
      static_cast<Handle*>(d)->kind != kind) {
    throw_error(env, TLM_ERR_INVALID, kind == 1 ? "TLMAddon: expected a context" : "TLMAddon: expected a model");
    return nullptr;
  }
  Handle* h = static_cast<Handle*>(d);
  if (!h->p) {
    throw_error(env, TLM_ERR_STATE, kind == 1 ? "TLMContext: closed" : "TLMModel: destroyed");
    return nullptr;
  }
  return h;
}

napi_value undefined(napi_env env) {
  napi_value u;
  napi_get_undefined(env, &u);
  return u;
}

napi_value num(napi_env env, double d) {
  napi_value v;
  napi_create_double(env, d, &v);
  return v;
}

// -------------------------------------------------------------- functions --
napi_value AbiVersion(napi_env env, napi_callback_info) { return num(env, g_api.abi_version()); }

napi_value LastError(napi_env env, napi_callback_info) {
  napi_value s;
  napi_create_string_utf8(env, g_api.last_error(), NAPI_AUTO_LENGTH, &s);
  return s;
}

napi_value Open(napi_env env, napi_callback_info info) {
  Args a(env, info);
  int32_t dev = 0;
  if (a.n >= 1 && !get_i32(env, a.v[0], &dev, "device")) return nullptr;
  tlm_ctx* ctx = nullptr;
  if (!check(env, g_api.open(dev, &ctx))) return nullptr;
  return wrap(env, ctx, 1);
}

napi_value Close(napi_env env, napi_callback_info info) {
  Args a(env, info);
  void* d = nullptr;
  if (a.n >= 1 && napi_get_value_external(env, a.v[0], &d) == napi_ok && d) {
    Handle* h = static_cast<Handle*>(d);
    if (h->kind == 1 && h->p) g_api.close(static_cast<tlm_ctx*>(h->p));
    if (h->kind == 1) h->p = nullptr;
  }
  return undefined(env);
}

napi_value Sync(napi_env env, napi_callback_info info) {
  Args a(env, info);
  Handle* h = unwrap(env, a.v[0], 1);
  if (!h || !check(env, g_api.sync(static_cast<tlm_ctx*>(h->p)))) return nullptr;
  return undefined(env);
}

napi_value DeviceInfo(napi_env env, napi_callback_info info) {
  Args a(env, info);
  Handle* h = unwrap(env, a.v[0], 1);
  if (!h) return nullptr;
  char name[256] = {0};
  int cus = 0;
  if (!check(env, g_api.device_info(static_cast<tlm_ctx*>(h->p), name, sizeof name, &cus))) return nullptr;
  napi_value o, s;
  napi_create_object(env, &o);
  napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &s);
  napi_set_named_property(env, o, "name", s);
  napi_set_named_property(env, o, "cus", num(env, cus));
  return o;
}

bool field_i32(napi_env env, napi_value o, const char* name, int32_t* out, bool required, int32_t dflt) {
  bool has = false;
  napi_has_named_property(env, o, name, &has);
  if (!has) {
    if (required) throw_error(env, TLM_ERR_INVALID, std::string("TLMModel: desc.") + name + " is required");
    *out = dflt;
    return !required;
  }
  napi_value v;
  napi_get_named_property(env, o, name, &v);
  return get_i32(env, v, out, name);
}

bool field_f64(napi_env env, napi_value o, const char* name, double* out, double dflt) {
  bool has = false;
  napi_has_named_property(env, o, name, &has);
  if (!has) {
    *out = dflt;
    return true;
  }
  napi_value v;
  napi_get_named_property(env, o, name, &v);
  return get_f64(env, v, out, name);
}

// desc: {hiddenSize, intermediateSize, numLayers, numHeads, numKvHeads,
// headDim, vocabSize, maxTokens, rotaryDim, slidingWindow, linearFmt,
// headFmt, embedFmt, kvFmt, qkvBias, tied, rmsEps, attentionFactor,
// invFreq: Float32Array(rotaryDim / 2), attnScale, layerWindows:
// Int32Array(numLayers)} -- the fields of tlm_model_desc.
napi_value ModelCreate(napi_env env, napi_callback_info info) {
  Args a(env, info);
  Handle* h = unwrap(env, a.v[0], 1);
  if (!h) return nullptr;
  if (a.n < 2) return throw_error(env, TLM_ERR_INVALID, "TLMModel: a desc object is required");
  napi_value o = a.v[1];
  tlm_model_desc d;
  memset(&d, 0, sizeof d);
  bool has_windows = false;
  const bool ok = field_i32(env, o, "hiddenSize", &d.hidden_size, true, 0) &&
                  field_i32(env, o, "intermediateSize", &d.intermediate_size, true, 0) &&
                  field_i32(env, o, "numLayers", &d.num_layers, true, 0) &&
                  field_i32(env, o, "numHeads", &d.num_heads, true, 0) &&
                  field_i32(env, o, "numKvHeads", &d.num_kv_heads, true, 0) &&
                  field_i32(env, o, "headDim", &d.head_dim, true, 0) &&
                  field_i32(env, o, "vocabSize", &d.vocab_size, true, 0) &&
                  field_i32(env, o, "maxTokens", &d.max_tokens, true, 0) &&
                  field_i32(env, o, "rotaryDim", &d.rotary_dim, false, d.head_dim) &&
                  field_i32(env, o, "slidingWindow", &d.sliding_window, false, 0) &&
                  field_i32(env, o, "linearFmt", &d.linear_fmt, false, TLM_FMT_Q4) &&
                  field_i32(env, o, "headFmt", &d.head_fmt, false, TLM_FMT_F16) &&
                  field_i32(env, o, "embedFmt", &d.embed_fmt, false, TLM_FMT_F16) &&
                  field_i32(env, o, "kvFmt", &d.kv_fmt, false, TLM_FMT_F16) &&
                  field_i32(env, o, "qkvBias", &d.qkv_bias, false, 0) && field_i32(env, o, "tied", &d.tied, false, 0) &&
                  field_f64(env, o, "rmsEps", &d.rms_eps, 1e-6) &&
                  field_f64(env, o, "attentionFactor", &d.attention_factor, 1.0) &&
                  field_f64(env, o, "attnScale", &d.attn_scale, 0.0);
  if (!ok) return nullptr;
  napi_has_named_property(env, o, "layerWindows", &has_windows);
  if (has_windows) {
    napi_value v;
    void* w = nullptr;
    size_t n_w = 0;
    napi_get_named_property(env, o, "layerWindows", &v);
    if (!get_typed(env, v, napi_int32_array, &w, &n_w, "desc.layerWindows")) return nullptr;
    if ((int)n_w != d.num_layers)
      return throw_error(env, TLM_ERR_INVALID, "TLMModel: desc.layerWindows needs numLayers entries");
    d.layer_windows = static_cast<const int32_t*>(w);
  }
  void* inv = nullptr;
  size_t n_inv = 0;
  bool has = false;
  napi_has_named_property(env, o, "invFreq", &has);
  if (has) {
    napi_value v;
    napi_get_named_property(env, o, "invFreq", &v);
    if (!get_typed(env, v, napi_float32_array, &inv, &n_inv, "desc.invFreq")) return nullptr;
    if ((int)n_inv * 2 < d.rotary_dim)
      return throw_error(env, TLM_ERR_INVALID, "TLMModel: desc.invFreq needs rotaryDim / 2 entries");
  } else if (d.rotary_dim > 0) {
    return throw_error(env, TLM_ERR_INVALID, "TLMModel: desc.invFreq is required when rotaryDim > 0");
  }
  d.inv_freq = static_cast<const float*>(inv);
  tlm_model* m = nullptr;
  if (!check(env, g_api.model_create(static_cast<tlm_ctx*>(h->p), &d, &m))) return nullptr;
  return wrap(env, m, 2);
}

napi_value ModelDestroy(napi_env env, napi_callback_info info) {
  Args a(env, info);
  void* d = nullptr;
  if (a.n >= 1 && napi_get_value_external(env, a.v[0], &d) == napi_ok && d) {
    Handle* h = static_cast<Handle*>(d);
    if (h->kind == 2 && h->pending)
      return throw_error(env, TLM_ERR_STATE, "TLMModel: a read of this model is still pending");
    if (h->kind == 2 && h->p) g_api.model_destroy(static_cast<tlm_model*>(h->p));
    if (h->kind == 2) h->p = nullptr;
  }
  return undefined(env);
}

tlm_model* model_arg(napi_env env, napi_value v) {
  Handle* h = unwrap(env, v, 2);
  if (h && h->pending) {
    throw_error(env, TLM_ERR_STATE, "TLMModel: a read of this model is still pending");
    return nullptr;
  }
  return h ? static_cast<tlm_model*>(h->p) : nullptr;
}

napi_value ModelUpload(napi_env env, napi_callback_info info) {
  Args a(env, info);
  tlm_model* m = model_arg(env, a.v[0]);
  int32_t tensor = 0, layer = 0;
  void* data = nullptr;
  size_t bytes = 0;
  if (!m || !get_i32(env, a.v[1], &tensor, "tensor") || !get_i32(env, a.v[2], &layer, "layer") ||
      !get_bytes(env, a.v[3], &data, &bytes))
    return nullptr;
  if (!check(env, g_api.model_upload(m, tensor, layer, data, bytes))) return nullptr;
  return undefined(env);
}

napi_value ModelFinalize(napi_env env, napi_callback_info info) {
  Args a(env, info);
  tlm_model* m = model_arg(env, a.v[0]);
  if (!m || !check(env, g_api.model_finalize(m))) return nullptr;
  return undefined(env);
}

// modelSetPrefill(model, minRows, chunk): the batched-prefill threshold and
// chunk (tlm_model_set_prefill; minRows <= 0 replays the decode graph).
napi_value ModelSetPrefill(napi_env env, napi_callback_info info) {
  Args a(env, info);
  tlm_model* m = model_arg(env, a.v[0]);
  int32_t min_rows = 0, chunk = 0;
  if (!m || !get_i32(env, a.v[1], &min_rows, "minRows") || !get_i32(env, a.v[2], &chunk, "chunk")) return nullptr;
  if (!check(env, g_api.model_set_prefill(m, min_rows, chunk))) return nullptr;
  return undefined(env);
}

napi_value ComputeToken(napi_env env, napi_callback_info info) {
  Args a(env, info);
  tlm_model* m = model_arg(env, a.v[0]);
  int32_t token = 0, pos = 0, flags = TLM_LOGITS;
  if (!m || !get_i32(env, a.v[1], &token, "token") || !get_i32(env, a.v[2], &pos, "position")) return nullptr;
  if (a.n >= 4 && !get_i32(env, a.v[3], &flags, "flags")) return nullptr;
  if (!check(env, g_api.compute_token(m, token, pos, flags))) return nullptr;
  return undefined(env);
}

napi_value Prefill(napi_env env, napi_callback_info info) {
  Args a(env, info);
  tlm_model* m = model_arg(env, a.v[0]);
  void* toks = nullptr;
  size_t n = 0;
  int32_t start = 0, end = 0;
  if (!m || !get_typed(env, a.v[1], napi_int32_array, &toks, &n, "tokens") ||
      !get_i32(env, a.v[2], &start, "start") || !get_i32(env, a.v[3], &end, "end"))
    return nullptr;
  if (start < 0 || end < start || (size_t)end > n)
    return throw_error(env, TLM_ERR_RANGE, "TLMModel: prefill range outside the token array");
  if (!check(env, g_api.prefill(m, static_cast<const int32_t*>(toks), start, end))) return nullptr;
  return undefined(env);
}

napi_value ReadLogits(napi_env env, napi_callback_info info) {
  Args a(env, info);
  tlm_model* m = model_arg(env, a.v[0]);
  void* out = nullptr;
  size_t n = 0;
  if (!m || !get_typed(env, a.v[1], napi_float32_array, &out, &n, "logits")) return nullptr;
  if (!check(env, g_api.read_logits(m, static_cast<float*>(out), n))) return nullptr;
  return a.v[1];
}

napi_value ReadToken(napi_env env, napi_callback_info info) {
  Args a(env, info);
  tlm_model* m = model_arg(env, a.v[0]);
  int32_t t = 0;
  if (!m || !check(env, g_api.read_token(m, &t))) return nullptr;
  return num(env, t);
}

// {graphLaunches, kernelLaunches, prefillChunks, replayedPositions,
// recomputedPositions, persistentTokens}: the submission counts of the model
// (tlm_model_counts_read).
napi_value ModelCounts(napi_env env, napi_callback_info info) {
  Args a(env, info);
  tlm_model* m = model_arg(env, a.v[0]);
  tlm_model_counts c;
  if (!m || !check(env, g_api.model_counts_read(m, &c))) return nullptr;
  napi_value o;
  napi_create_object(env, &o);
  const std::pair<const char*, uint64_t> fields[] = {{"graphLaunches", c.graph_launches},
                                                     {"kernelLaunches", c.kernel_launches},
                                                     {"prefillChunks", c.prefill_chunks},
                                                     {"replayedPositions", c.replayed_positions},
                                                     {"recomputedPositions", c.recomputed_positions},
                                                     {"persistentTokens", c.persistent_tokens}};
  for (const auto& f : fields) {
    napi_value v;
    napi_create_double(env, (double)f.second, &v);
    napi_set_named_property(env, o, f.first, v);
  }
  return o;
}

napi_value DecodeGreedy(napi_env env, napi_callback_info info) {
  Args a(env, info);
  tlm_model* m = model_arg(env, a.v[0]);
  int32_t token = 0, pos = 0, n = 0;
  if (!m || !get_i32(env, a.v[1], &token, "token") || !get_i32(env, a.v[2], &pos, "position") ||
      !get_i32(env, a.v[3], &n, "n"))
    return nullptr;
  if (n < 0) return throw_error(env, TLM_ERR_INVALID, "TLMModel: n must be non-negative");
  void* data = nullptr;
  napi_value arr = new_typed(env, napi_int32_array, (size_t)n, 4, &data);
  if (n > 0 && !check(env, g_api.decode_greedy(m, token, pos, n, static_cast<int32_t*>(data)))) return nullptr;
  return arr;
}

napi_value ResetCache(napi_env env, napi_callback_info info) {
  Args a(env, info);
  tlm_model* m = model_arg(env, a.v[0]);
  if (!m || !check(env, g_api.reset_cache(m))) return nullptr;
  return undefined(env);
}

napi_value ReadCandidates(napi_env env, napi_callback_info info) {
  Args a(env, info);
  tlm_model* m = model_arg(env, a.v[0]);
  int32_t k = 0;
  double cap = 0;
  if (!m || !get_i32(env, a.v[1], &k, "k")) return nullptr;
  if (a.n >= 3 && !get_f64(env, a.v[2], &cap, "softcap")) return nullptr;
  if (k < 1 || k > 16) return throw_error(env, TLM_ERR_INVALID, "TLMLogitSampler: k must be in [1, 16]");
  void *t = nullptr, *s = nullptr;
  napi_value ta = new_typed(env, napi_int32_array, (size_t)k, 4, &t);
  napi_value sa = new_typed(env, napi_float32_array, (size_t)k, 4, &s);
  if (!check(env, g_api.read_candidates(m, k, cap, static_cast<int32_t*>(t), static_cast<float*>(s)))) return nullptr;
  napi_value o;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "tokens", ta);
  napi_set_named_property(env, o, "scores", sa);
  return o;
}

// ------------------------------------------------------------ async reads --
// One read on the thread pool: execute() calls the library (which waits for
// the model's stream) off the JS thread, complete() settles the Promise on it.
// The arrays the read fills are kept alive by references until then, and
// the model handle counts the read as pending.
struct AsyncRead {
  enum Kind { LOGITS, TOKEN, CANDIDATES, GREEDY, PREFILL } kind;
  Handle* model;
  napi_ref model_ref = nullptr;  // the handle's external
  napi_ref out_ref = nullptr;    // the value the Promise resolves with (arrays: filled in place)
  napi_deferred deferred = nullptr;
  napi_async_work work = nullptr;
  void* a = nullptr;  // logits / candidate ids / greedy tokens
  void* b = nullptr;  // candidate scores
  size_t n = 0;
  int32_t token = 0, pos = 0, k = 0;
  double cap = 0;
  int rc = 0;
  std::string err;  // tlm_last_error() of the worker thread (thread-local)
  AsyncRead(Kind k, Handle* h) : kind(k), model(h) {}
};

void read_execute(napi_env, void* data) {
  AsyncRead* r = static_cast<AsyncRead*>(data);
  tlm_model* m = static_cast<tlm_model*>(r->model->p);
  switch (r->kind) {
    case AsyncRead::LOGITS: r->rc = g_api.read_logits(m, static_cast<float*>(r->a), r->n); break;
    case AsyncRead::TOKEN: r->rc = g_api.read_token(m, &r->token); break;
    case AsyncRead::CANDIDATES:
      r->rc = g_api.read_candidates(m, r->k, r->cap, static_cast<int32_t*>(r->a), static_cast<float*>(r->b));
      break;
    case AsyncRead::GREEDY:
      r->rc = r->n ? g_api.decode_greedy(m, r->token, r->pos, (int)r->n, static_cast<int32_t*>(r->a)) : TLM_OK;
      break;
    case AsyncRead::PREFILL:  // [pos, k) of the token array
      r->rc = g_api.prefill(m, static_cast<const int32_t*>(r->a), r->pos, r->k);
      break;
  }
  if (r->rc != TLM_OK) {
    const char* e = g_api.last_error();
    r->err = e && *e ? e : "TLMAddon: call failed with code " + std::to_string(r->rc);
  }
}

void read_complete(napi_env env, napi_status status, void* data) {
  AsyncRead* r = static_cast<AsyncRead*>(data);
  r->model->pending--;
  if (status != napi_ok && r->rc == TLM_OK) {
    r->rc = TLM_ERR_STATE;
    r->err = "TLMAddon: the read was cancelled";
  }
  if (r->rc != TLM_OK) {
    napi_value msg, err, c;
    napi_create_string_utf8(env, r->err.c_str(), NAPI_AUTO_LENGTH, &msg);
    napi_create_error(env, nullptr, msg, &err);
    napi_create_int32(env, r->rc, &c);
    napi_set_named_property(env, err, "code", c);
    napi_reject_deferred(env, r->deferred, err);
  } else {
    napi_value v;
    if (r->kind == AsyncRead::TOKEN) napi_create_double(env, r->token, &v);
    else if (r->kind == AsyncRead::PREFILL) napi_get_undefined(env, &v);
    else napi_get_reference_value(env, r->out_ref, &v);
    napi_resolve_deferred(env, r->deferred, v);
  }
  if (r->out_ref) napi_delete_reference(env, r->out_ref);
  napi_delete_reference(env, r->model_ref);
  napi_delete_async_work(env, r->work);
  delete r;
}

// Queues r (its model handle is args[0]); returns the Promise, or throws.
napi_value read_start(napi_env env, napi_value model, napi_value out, AsyncRead* r, const char* name) {
  napi_value promise, res;
  napi_create_promise(env, &r->deferred, &promise);
  napi_create_reference(env, model, 1, &r->model_ref);
  if (out) napi_create_reference(env, out, 1, &r->out_ref);
  napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &res);
  if (napi_create_async_work(env, nullptr, res, read_execute, read_complete, r, &r->work) != napi_ok ||
      napi_queue_async_work(env, r->work) != napi_ok) {
    if (r->out_ref) napi_delete_reference(env, r->out_ref);
    napi_delete_reference(env, r->model_ref);
    delete r;
    return throw_error(env, TLM_ERR_STATE, "TLMAddon: cannot queue the read");
  }
  r->model->pending++;
  return promise;
}

Handle* model_handle(napi_env env, napi_value v) {
  return model_arg(env, v) ? unwrap(env, v, 2) : nullptr;
}

napi_value ReadLogitsAsync(napi_env env, napi_callback_info info) {
  Args a(env, info);
  Handle* h = model_handle(env, a.v[0]);
  void* out = nullptr;
  size_t n = 0;
  if (!h || !get_typed(env, a.v[1], napi_float32_array, &out, &n, "logits")) return nullptr;
  AsyncRead* r = new AsyncRead(AsyncRead::LOGITS, h);
  r->a = out;
  r->n = n;
  return read_start(env, a.v[0], a.v[1], r, "tlmReadLogits");
}

napi_value ReadTokenAsync(napi_env env, napi_callback_info info) {
  Args a(env, info);
  Handle* h = model_handle(env, a.v[0]);
  if (!h) return nullptr;
  AsyncRead* r = new AsyncRead(AsyncRead::TOKEN, h);
  return read_start(env, a.v[0], nullptr, r, "tlmReadToken");
}

napi_value ReadCandidatesAsync(napi_env env, napi_callback_info info) {
  Args a(env, info);
  Handle* h = model_handle(env, a.v[0]);
  int32_t k = 0;
  double cap = 0;
  if (!h || !get_i32(env, a.v[1], &k, "k")) return nullptr;
  if (a.n >= 3 && !get_f64(env, a.v[2], &cap, "softcap")) return nullptr;
  if (k < 1 || k > 16) return throw_error(env, TLM_ERR_INVALID, "TLMLogitSampler: k must be in [1, 16]");
  AsyncRead* r = new AsyncRead(AsyncRead::CANDIDATES, h);
  r->k = k;
  r->cap = cap;
  napi_value ta = new_typed(env, napi_int32_array, (size_t)k, 4, &r->a);
  napi_value sa = new_typed(env, napi_float32_array, (size_t)k, 4, &r->b);
  napi_value o;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "tokens", ta);
  napi_set_named_property(env, o, "scores", sa);
  return read_start(env, a.v[0], o, r, "tlmReadCandidates");
}

napi_value DecodeGreedyAsync(napi_env env, napi_callback_info info) {
  Args a(env, info);
  Handle* h = model_handle(env, a.v[0]);
  int32_t token = 0, pos = 0, n = 0;
  if (!h || !get_i32(env, a.v[1], &token, "token") || !get_i32(env, a.v[2], &pos, "position") ||
      !get_i32(env, a.v[3], &n, "n"))
    return nullptr;
  if (n < 0) return throw_error(env, TLM_ERR_INVALID, "TLMModel: n must be non-negative");
  AsyncRead* r = new AsyncRead(AsyncRead::GREEDY, h);
  r->token = token;
  r->pos = pos;
  r->n = (size_t)n;
  napi_value arr = new_typed(env, napi_int32_array, (size_t)n, 4, &r->a);
  return read_start(env, a.v[0], arr, r, "tlmDecodeGreedy");
}

// prefillAsync(model, Int32Array, start, end): tlm_prefill on the thread pool
// (it waits for each batched chunk's overflow flag).
napi_value PrefillAsync(napi_env env, napi_callback_info info) {
  Args a(env, info);
  Handle* h = model_handle(env, a.v[0]);
  void* toks = nullptr;
  size_t n = 0;
  int32_t start = 0, end = 0;
  if (!h || !get_typed(env, a.v[1], napi_int32_array, &toks, &n, "tokens") ||
      !get_i32(env, a.v[2], &start, "start") || !get_i32(env, a.v[3], &end, "end"))
    return nullptr;
  if (start < 0 || end < start || (size_t)end > n)
    return throw_error(env, TLM_ERR_RANGE, "TLMModel: prefill range outside the token array");
  AsyncRead* r = new AsyncRead(AsyncRead::PREFILL, h);
  r->a = toks;
  r->pos = start;
  r->k = end;
  return read_start(env, a.v[0], a.v[1], r, "tlmPrefill");
}

napi_value QuantizeQ4(napi_env env, napi_callback_info info) {
  Args a(env, info);
  void* w = nullptr;
  size_t n = 0;
  int32_t n_out = 0, k_in = 0;
  if (!get_typed(env, a.v[0], napi_float32_array, &w, &n, "weights") || !get_i32(env, a.v[1], &n_out, "nOut") ||
      !get_i32(env, a.v[2], &k_in, "kIn"))
    return nullptr;
  if (n_out <= 0 || k_in <= 0 || (size_t)n_out * (size_t)k_in != n)
    return throw_error(env, TLM_ERR_INVALID, "TLMQuantize: weights must hold nOut * kIn floats");
  void *p = nullptr, *s = nullptr;
  const size_t groups = (size_t)n_out * (size_t)(k_in / 32 > 0 ? k_in / 32 : 1);
  napi_value pa = new_typed(env, napi_uint8_array, (size_t)n_out * (size_t)k_in / 2, 1, &p);
  napi_value sa = new_typed(env, napi_uint16_array, groups, 2, &s);
  if (!check(env, g_api.quantize_q4(static_cast<const float*>(w), n_out, k_in, static_cast<uint8_t*>(p),
                                    static_cast<uint16_t*>(s))))
    return nullptr;
  napi_value o;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "packed", pa);
  napi_set_named_property(env, o, "scales", sa);
  return o;
}

napi_value F32ToF16(napi_env env, napi_callback_info info) {
  Args a(env, info);
  void* in = nullptr;
  size_t n = 0;
  if (!get_typed(env, a.v[0], napi_float32_array, &in, &n, "values")) return nullptr;
  void* out = nullptr;
  napi_value arr = new_typed(env, napi_uint16_array, n, 2, &out);
  if (!check(env, g_api.f32_to_f16(static_cast<const float*>(in), n, static_cast<uint16_t*>(out)))) return nullptr;
  return arr;
}

napi_value SynthNormal(napi_env env, napi_callback_info info) {
  Args a(env, info);
  uint64_t seed = 0, stream = 0;
  int32_t n = 0;
  double sd = 1.0;
  if (!get_u64(env, a.v[0], &seed, "seed") || !get_u64(env, a.v[1], &stream, "stream") ||
      !get_i32(env, a.v[2], &n, "n") || !get_f64(env, a.v[3], &sd, "stddev"))
    return nullptr;
  if (n < 0) return throw_error(env, TLM_ERR_INVALID, "TLMSynth: n must be non-negative");
  void* out = nullptr;
  napi_value arr = new_typed(env, napi_float32_array, (size_t)n, 4, &out);
  if (!check(env, g_api.synth_normal(seed, stream, (size_t)n, (float)sd, static_cast<float*>(out)))) return nullptr;
  return arr;
}

napi_value SynthTokens(napi_env env, napi_callback_info info) {
  Args a(env, info);
  uint64_t seed = 0, stream = 0;
  int32_t n = 0, vocab = 0;
  if (!get_u64(env, a.v[0], &seed, "seed") || !get_u64(env, a.v[1], &stream, "stream") ||
      !get_i32(env, a.v[2], &n, "n") || !get_i32(env, a.v[3], &vocab, "vocab"))
    return nullptr;
  if (n < 0) return throw_error(env, TLM_ERR_INVALID, "TLMSynth: n must be non-negative");
  void* out = nullptr;
  napi_value arr = new_typed(env, napi_int32_array, (size_t)n, 4, &out);
  if (!check(env, g_api.synth_tokens(seed, stream, (size_t)n, vocab, static_cast<int32_t*>(out)))) return nullptr;
  return arr;
}

napi_value Init(napi_env env, napi_value exports) {
  if (!load_library()) return throw_error(env, TLM_ERR_STATE, g_load_error);
  const napi_property_descriptor props[] = {
      {"abiVersion", nullptr, AbiVersion, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"lastError", nullptr, LastError, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"open", nullptr, Open, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"close", nullptr, Close, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"sync", nullptr, Sync, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"deviceInfo", nullptr, DeviceInfo, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"modelCreate", nullptr, ModelCreate, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"modelUpload", nullptr, ModelUpload, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"modelFinalize", nullptr, ModelFinalize, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"modelDestroy", nullptr, ModelDestroy, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"computeToken", nullptr, ComputeToken, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"prefill", nullptr, Prefill, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"readLogits", nullptr, ReadLogits, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"readToken", nullptr, ReadToken, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"decodeGreedy", nullptr, DecodeGreedy, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"resetCache", nullptr, ResetCache, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"readCandidates", nullptr, ReadCandidates, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"quantizeQ4", nullptr, QuantizeQ4, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"f32ToF16", nullptr, F32ToF16, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"synthNormal", nullptr, SynthNormal, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"synthTokens", nullptr, SynthTokens, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"modelCounts", nullptr, ModelCounts, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"modelSetPrefill", nullptr, ModelSetPrefill, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"readLogitsAsync", nullptr, ReadLogitsAsync, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"readTokenAsync", nullptr, ReadTokenAsync, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"readCandidatesAsync", nullptr, ReadCandidatesAsync, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"decodeGreedyAsync", nullptr, DecodeGreedyAsync, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"prefillAsync", nullptr, PrefillAsync, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
  };
  napi_define_properties(env, exports, sizeof props / sizeof props[0], props);
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Init)
