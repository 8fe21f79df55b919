// napi.cc - the Node.js N-API addon over the C ABI (include/p0pc0rn.h).
//
// The JS host (p0pc0rn_amd/js/*.mjs) keeps the reference's op call surface (gemv / gemvM / gemm and the Gpu object's
// buffer / upload / read / free / done); this addon only marshals flat argument objects into the C structs and turns a
// nonzero status into a thrown JS Error carrying the library's message (the reference's own text for argument errors).
// Device addresses cross as JS numbers (exact below 2^53).
#include <node_api.h>

#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "p0pc0rn.h"

namespace {

bool fail(napi_env env, int rc) {
  if (rc == P0_OK) return false;
  napi_throw_error(env, nullptr, p0_last_error());
  return true;
}

std::vector<napi_value> args(napi_env env, napi_callback_info info, size_t n) {
  std::vector<napi_value> v(n);
  size_t got = n;
  napi_get_cb_info(env, info, &got, v.data(), nullptr, nullptr);
  for (size_t i = got; i < n; ++i) napi_get_undefined(env, &v[i]);
  return v;
}

double num(napi_env env, napi_value v, double dflt = 0.0) {
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t != napi_number) return dflt;
  double d = 0;
  napi_get_value_double(env, v, &d);
  return d;
}

double field(napi_env env, napi_value obj, const char* name, double dflt = 0.0) {
  bool has = false;
  napi_has_named_property(env, obj, name, &has);
  if (!has) return dflt;
  napi_value v;
  napi_get_named_property(env, obj, name, &v);
  return num(env, v, dflt);
}

template <class T> T* ptr(napi_env env, napi_value obj, const char* name) {
  return reinterpret_cast<T*>(static_cast<uintptr_t>(field(env, obj, name)));
}
int64_t i64(napi_env env, napi_value obj, const char* name) { return static_cast<int64_t>(field(env, obj, name)); }
int32_t i32(napi_env env, napi_value obj, const char* name) { return static_cast<int32_t>(field(env, obj, name)); }

napi_value make_num(napi_env env, double d) {
  napi_value v;
  napi_create_double(env, d, &v);
  return v;
}
napi_value undef(napi_env env) {
  napi_value v;
  napi_get_undefined(env, &v);
  return v;
}

// (data pointer, byte length) of a TypedArray / ArrayBuffer / DataView argument
bool bytes_of(napi_env env, napi_value v, void** data, size_t* len) {
  bool is = false;
  napi_is_typedarray(env, v, &is);
  if (is) {
    napi_typedarray_type t;
    size_t n, off;
    napi_value ab;
    void* base;
    napi_get_typedarray_info(env, v, &t, &n, &base, &ab, &off);
    size_t el = 1;
    switch (t) {
      case napi_int16_array: case napi_uint16_array: el = 2; break;
      case napi_int32_array: case napi_uint32_array: case napi_float32_array: el = 4; break;
      case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: el = 8; break;
      default: el = 1;
    }
    *data = base;
    *len = n * el;
    return true;
  }
  napi_is_arraybuffer(env, v, &is);
  if (is) return napi_get_arraybuffer_info(env, v, data, len) == napi_ok;
  napi_is_dataview(env, v, &is);
  if (is) {
    napi_value ab;
    size_t off;
    return napi_get_dataview_info(env, v, len, data, &ab, &off) == napi_ok;
  }
  return false;
}

napi_value Open(napi_env env, napi_callback_info info) {
  auto a = args(env, info, 1);
  if (fail(env, p0_open((int)num(env, a[0], 0)))) return nullptr;
  return undef(env);
}

napi_value Close(napi_env env, napi_callback_info) {
  p0_close();
  return undef(env);
}

napi_value Info(napi_env env, napi_callback_info) {
  p0_device_info_t d;
  if (fail(env, p0_device_info(&d))) return nullptr;
  napi_value o, s;
  napi_create_object(env, &o);
  napi_create_string_utf8(env, d.name, NAPI_AUTO_LENGTH, &s);
  napi_set_named_property(env, o, "name", s);
  napi_set_named_property(env, o, "device", make_num(env, d.device));
  napi_set_named_property(env, o, "cuCount", make_num(env, d.cu_count));
  napi_set_named_property(env, o, "xcdCount", make_num(env, d.xcd_count));
  napi_set_named_property(env, o, "hbmBytes", make_num(env, (double)d.hbm_bytes));
  napi_set_named_property(env, o, "ldsBytesPerCU", make_num(env, (double)d.lds_bytes_per_cu));
  napi_set_named_property(env, o, "clockKHz", make_num(env, d.clock_khz));
  napi_set_named_property(env, o, "workspaceBytes", make_num(env, (double)d.workspace_bytes));
  return o;
}

napi_value Buffer(napi_env env, napi_callback_info info) {
  auto a = args(env, info, 1);
  void* p = nullptr;
  if (fail(env, p0_buffer((size_t)num(env, a[0]), &p))) return nullptr;
  return make_num(env, (double)(uintptr_t)p);
}

napi_value Free(napi_env env, napi_callback_info info) {
  auto a = args(env, info, 1);
  if (fail(env, p0_free((void*)(uintptr_t)num(env, a[0])))) return nullptr;
  return undef(env);
}

napi_value Upload(napi_env env, napi_callback_info info) {   // upload(dst, dstOff, typedArray)
  auto a = args(env, info, 3);
  void* data;
  size_t len;
  if (!bytes_of(env, a[2], &data, &len)) {
    napi_throw_type_error(env, nullptr, "upload: expected a TypedArray, ArrayBuffer or DataView");
    return nullptr;
  }
  if (fail(env, p0_upload((void*)(uintptr_t)num(env, a[0]), (size_t)num(env, a[1]), data, len))) return nullptr;
  return undef(env);
}

napi_value Read(napi_env env, napi_callback_info info) {   // read(src, off, bytes) -> ArrayBuffer
  auto a = args(env, info, 3);
  size_t n = (size_t)num(env, a[2]);
  void* data = nullptr;
  napi_value ab;
  napi_create_arraybuffer(env, n, &data, &ab);
  if (fail(env, p0_read(data, (const void*)(uintptr_t)num(env, a[0]), (size_t)num(env, a[1]), n))) return nullptr;
  return ab;
}

napi_value Fill(napi_env env, napi_callback_info info) {   // fill(dst, off, u32 value, words)
  auto a = args(env, info, 4);
  if (fail(env, p0_fill((void*)(uintptr_t)num(env, a[0]), (size_t)num(env, a[1]), (uint32_t)num(env, a[2]), (size_t)num(env, a[3]))))
    return nullptr;
  return undef(env);
}

napi_value Copy(napi_env env, napi_callback_info info) {   // copy(src, srcOff, dst, dstOff, size)
  auto a = args(env, info, 5);
  if (fail(env, p0_copy((const void*)(uintptr_t)num(env, a[0]), (size_t)num(env, a[1]), (void*)(uintptr_t)num(env, a[2]),
                        (size_t)num(env, a[3]), (size_t)num(env, a[4]))))
    return nullptr;
  return undef(env);
}

napi_value Done(napi_env env, napi_callback_info) {
  if (fail(env, p0_done())) return nullptr;
  return undef(env);
}

napi_value TimerStart(napi_env env, napi_callback_info) {
  if (fail(env, p0_timer_start())) return nullptr;
  return undef(env);
}

napi_value TimerStop(napi_env env, napi_callback_info) {
  float ms = 0;
  if (fail(env, p0_timer_stop(&ms))) return nullptr;
  return make_num(env, ms);
}

napi_value Gemv(napi_env env, napi_callback_info info) {
  auto a = args(env, info, 1);
  napi_value o = a[0];
  p0_gemv_args_t g{};
  g.w = ptr<const void>(env, o, "w"); g.w_off = i64(env, o, "w_off"); g.w_enc = i32(env, o, "w_enc");
  g.w_rows = i64(env, o, "w_rows"); g.w_cols = i64(env, o, "w_cols");
  g.x = ptr<const float>(env, o, "x"); g.x_rowB = i64(env, o, "x_rowB");
  g.N = i64(env, o, "N"); g.K = i64(env, o, "K"); g.kPer = i64(env, o, "kPer");
  g.pro = i32(env, o, "pro"); g.epi = i32(env, o, "epi");
  g.y = ptr<float>(env, o, "y"); g.ldy = i64(env, o, "ldy");
  g.stat = ptr<const float>(env, o, "stat"); g.stat_off = i64(env, o, "stat_off");
  g.norm = ptr<const float>(env, o, "norm"); g.norm_off = i64(env, o, "norm_off");
  g.src_n = i64(env, o, "src_n"); g.src_ld = i64(env, o, "src_ld");
  g.ev = ptr<const float>(env, o, "ev"); g.ev_off = i64(env, o, "ev_off");
  g.mx = ptr<float>(env, o, "mx"); g.cap = (float)field(env, o, "cap");
  int32_t nsplit = 0;
  if (fail(env, p0_q4_gemv(&g, &nsplit))) return nullptr;
  return make_num(env, nsplit);
}

napi_value GemvM(napi_env env, napi_callback_info info) {
  auto a = args(env, info, 1);
  napi_value o = a[0];
  p0_gemvm_args_t g{};
  g.w = ptr<const void>(env, o, "w"); g.w_off = i64(env, o, "w_off"); g.w_enc = i32(env, o, "w_enc");
  g.w_rows = i64(env, o, "w_rows"); g.w_cols = i64(env, o, "w_cols");
  g.x = ptr<const float>(env, o, "x"); g.x_ldx = i64(env, o, "x_ldx"); g.x_rowB = i64(env, o, "x_rowB");
  g.M = i64(env, o, "M"); g.N = i64(env, o, "N"); g.K = i64(env, o, "K"); g.kPer = i64(env, o, "kPer");
  g.pro = i32(env, o, "pro"); g.epi = i32(env, o, "epi");
  g.y = ptr<float>(env, o, "y"); g.y_ldy = i64(env, o, "y_ldy"); g.y_ldm = i64(env, o, "y_ldm");
  g.stat = ptr<const float>(env, o, "stat"); g.stat_off = i64(env, o, "stat_off"); g.stat_ld = i64(env, o, "stat_ld");
  g.norm = ptr<const float>(env, o, "norm"); g.norm_off = i64(env, o, "norm_off");
  g.src_n = i64(env, o, "src_n"); g.src_ld = i64(env, o, "src_ld");
  g.ev = ptr<const float>(env, o, "ev"); g.ev_off = i64(env, o, "ev_off"); g.ev_ld = i64(env, o, "ev_ld");
  g.mx = ptr<float>(env, o, "mx"); g.cap = (float)field(env, o, "cap");
  int32_t nsplit = 0;
  if (fail(env, p0_q4_gemvM(&g, &nsplit))) return nullptr;
  return make_num(env, nsplit);
}

napi_value Gemm(napi_env env, napi_callback_info info) {
  auto a = args(env, info, 1);
  napi_value o = a[0];
  p0_gemm_args_t g{};
  g.w = ptr<const void>(env, o, "w"); g.w_off = i64(env, o, "w_off"); g.w_enc = i32(env, o, "w_enc");
  g.w_rows = i64(env, o, "w_rows"); g.w_cols = i64(env, o, "w_cols");
  g.x = ptr<const void>(env, o, "x"); g.x_off = i64(env, o, "x_off"); g.x_ld = i64(env, o, "x_ld");
  g.x_k0 = i64(env, o, "x_k0"); g.x_mode = i32(env, o, "x_mode");
  g.M = i64(env, o, "M"); g.N = i64(env, o, "N"); g.K = i64(env, o, "K");
  g.wr0 = i64(env, o, "wr0"); g.wr1 = i64(env, o, "wr1"); g.wk0 = i64(env, o, "wk0");
  g.epi = i32(env, o, "epi");
  g.y = ptr<void>(env, o, "y"); g.y_off = i64(env, o, "y_off"); g.y_ld = i64(env, o, "y_ld"); g.y_n0 = i64(env, o, "y_n0");
  g.ev = ptr<const float>(env, o, "ev"); g.ev_off = i64(env, o, "ev_off");
  g.stats = ptr<const float>(env, o, "stats"); g.stats_off = i64(env, o, "stats_off");
  g.pv = ptr<const float>(env, o, "pv"); g.pv_off = i64(env, o, "pv_off"); g.pv_stride = i64(env, o, "pv_stride");
  g.bv = ptr<const float>(env, o, "bv"); g.bv_off = i64(env, o, "bv_off"); g.bv_up = i64(env, o, "bv_up");
  g.act = i32(env, o, "act"); g.store = i32(env, o, "store"); g.res = i32(env, o, "res");
  g.heads_ltot = i64(env, o, "heads_ltot"); g.heads_row_off = i64(env, o, "heads_row_off");
  g.heads_hq = i32(env, o, "heads_hq"); g.heads_hkv = i32(env, o, "heads_hkv");
  g.heads_eps = (float)field(env, o, "heads_eps"); g.heads_rope = i32(env, o, "heads_rope");
  g.rope = ptr<const float>(env, o, "rope");
  double flops = 0;
  if (fail(env, p0_q4_gemm(&g, &flops))) return nullptr;
  return make_num(env, flops);
}

napi_value Rowstats(napi_env env, napi_callback_info info) {
  auto a = args(env, info, 1);
  napi_value o = a[0];
  p0_rowstats_args_t r{};
  r.x = ptr<const void>(env, o, "x"); r.x_off = i64(env, o, "x_off"); r.x_ld = i64(env, o, "x_ld");
  r.x_c0 = i64(env, o, "x_c0"); r.rows = i64(env, o, "rows"); r.cols = i64(env, o, "cols");
  r.mode = i32(env, o, "mode"); r.eps = (float)field(env, o, "eps");
  r.st = ptr<float>(env, o, "st"); r.st_off = i64(env, o, "st_off");
  if (fail(env, p0_rowstats(&r))) return nullptr;
  return undef(env);
}

napi_value Normadd(napi_env env, napi_callback_info info) {
  auto a = args(env, info, 1);
  napi_value o = a[0];
  p0_normadd_args_t r{};
  r.t = ptr<const float>(env, o, "t"); r.t_n = i64(env, o, "t_n"); r.t_ld = i64(env, o, "t_ld");
  r.w = ptr<const float>(env, o, "w"); r.w_off = i64(env, o, "w_off");
  r.x = ptr<float>(env, o, "x"); r.st = ptr<float>(env, o, "st"); r.st_off = i64(env, o, "st_off");
  r.D = i64(env, o, "D"); r.M = i64(env, o, "M"); r.eps = (float)field(env, o, "eps");
  r.scale = (float)field(env, o, "scale", 1.0); r.mode = i32(env, o, "mode");
  if (fail(env, p0_normadd(&r))) return nullptr;
  return undef(env);
}

napi_value ArgmaxM(napi_env env, napi_callback_info info) {   // argmaxM(mx, n, M, out)
  auto a = args(env, info, 4);
  if (fail(env, p0_argmaxM((const float*)(uintptr_t)num(env, a[0]), (int64_t)num(env, a[1]), (int64_t)num(env, a[2]),
                           (uint32_t*)(uintptr_t)num(env, a[3]))))
    return nullptr;
  return undef(env);
}

napi_value UploadFile(napi_env env, napi_callback_info info) {   // uploadFile(path, offset, bytes, dst, dstOff)
  auto a = args(env, info, 5);
  size_t len = 0;
  napi_get_value_string_utf8(env, a[0], nullptr, 0, &len);
  std::string path(len, '\0');
  napi_get_value_string_utf8(env, a[0], &path[0], len + 1, &len);
  if (fail(env, p0_upload_file(path.c_str(), (int64_t)num(env, a[1]), (int64_t)num(env, a[2]),
                               (void*)(uintptr_t)num(env, a[3]), (int64_t)num(env, a[4]))))
    return nullptr;
  return undef(env);
}

napi_value Dequant(napi_env env, napi_callback_info info) {   // dequant(w, wOff, N, K, out32, out16)
  auto a = args(env, info, 6);
  if (fail(env, p0_q4_dequant((const void*)(uintptr_t)num(env, a[0]), (int64_t)num(env, a[1]), (int64_t)num(env, a[2]),
                              (int64_t)num(env, a[3]), (float*)(uintptr_t)num(env, a[4]), (uint16_t*)(uintptr_t)num(env, a[5]))))
    return nullptr;
  return undef(env);
}

napi_value FillQ4Sym(napi_env env, napi_callback_info info) {   // fillQ4Sym(w, wOff, N, K, seed, sigma)
  auto a = args(env, info, 6);
  if (fail(env, p0_fill_q4_sym((void*)(uintptr_t)num(env, a[0]), (int64_t)num(env, a[1]), (int64_t)num(env, a[2]),
                               (int64_t)num(env, a[3]), (uint32_t)num(env, a[4]), (float)num(env, a[5], 0.02))))
    return nullptr;
  return undef(env);
}

napi_value FillRandn(napi_env env, napi_callback_info info) {   // fillRandn(dst, offBytes, n, seed, sigma, asF16)
  auto a = args(env, info, 6);
  if (fail(env, p0_fill_randn((void*)(uintptr_t)num(env, a[0]), (int64_t)num(env, a[1]), (int64_t)num(env, a[2]),
                              (uint32_t)num(env, a[3]), (float)num(env, a[4], 1.0), (int32_t)num(env, a[5]))))
    return nullptr;
  return undef(env);
}

// ---- recorded op sequences and chains: opaque handles cross as numbers (host addresses, exact below 2^53)
void* handle(napi_env env, napi_value v) { return reinterpret_cast<void*>(static_cast<uintptr_t>(num(env, v))); }

napi_value RecordBegin(napi_env env, napi_callback_info) {
  if (fail(env, p0_record_begin())) return nullptr;
  return undef(env);
}
napi_value RecordEnd(napi_env env, napi_callback_info) {
  void* h = nullptr;
  if (fail(env, p0_record_end(&h))) return nullptr;
  return make_num(env, (double)reinterpret_cast<uintptr_t>(h));
}
napi_value Replay(napi_env env, napi_callback_info info) {
  auto a = args(env, info, 1);
  if (fail(env, p0_replay(handle(env, a[0])))) return nullptr;
  return undef(env);
}
napi_value RecordInfo(napi_env env, napi_callback_info info) {
  auto a = args(env, info, 1);
  int32_t n = 0;
  if (fail(env, p0_record_info(handle(env, a[0]), &n))) return nullptr;
  return make_num(env, n);
}
napi_value ChainInfo(napi_env env, napi_callback_info info) {
  auto a = args(env, info, 1);
  p0_chain_info_t ci{};
  if (fail(env, p0_chain_info(handle(env, a[0]), &ci))) return nullptr;
  return make_num(env, ci.n_ops);
}
napi_value RecordFree(napi_env env, napi_callback_info info) {
  auto a = args(env, info, 1);
  if (fail(env, p0_record_free(handle(env, a[0])))) return nullptr;
  return undef(env);
}
napi_value ChainBegin(napi_env env, napi_callback_info) {
  if (fail(env, p0_chain_begin())) return nullptr;
  return undef(env);
}
napi_value ChainEnd(napi_env env, napi_callback_info) {
  void* h = nullptr;
  if (fail(env, p0_chain_end(&h))) return nullptr;
  return make_num(env, (double)reinterpret_cast<uintptr_t>(h));
}
napi_value ChainRun(napi_env env, napi_callback_info info) {
  auto a = args(env, info, 1);
  if (fail(env, p0_chain_run(handle(env, a[0])))) return nullptr;
  return undef(env);
}
napi_value ChainStatus(napi_env env, napi_callback_info info) {   // -> true if a wait of an earlier run gave up
  auto a = args(env, info, 1);
  int32_t t = 0;
  if (fail(env, p0_chain_status(handle(env, a[0]), &t))) return nullptr;
  napi_value v;
  napi_get_boolean(env, t != 0, &v);
  return v;
}
napi_value ChainFree(napi_env env, napi_callback_info info) {
  auto a = args(env, info, 1);
  if (fail(env, p0_chain_free(handle(env, a[0])))) return nullptr;
  return undef(env);
}

napi_value Version(napi_env env, napi_callback_info) { return make_num(env, p0_version()); }

napi_value Init(napi_env env, napi_value exports) {
  struct { const char* name; napi_callback fn; } fns[] = {
      {"open", Open}, {"close", Close}, {"info", Info}, {"buffer", Buffer}, {"free", Free}, {"upload", Upload},
      {"read", Read}, {"fill", Fill}, {"copy", Copy}, {"done", Done}, {"timerStart", TimerStart}, {"timerStop", TimerStop},
      {"gemv", Gemv}, {"gemvM", GemvM}, {"gemm", Gemm}, {"dequant", Dequant}, {"fillQ4Sym", FillQ4Sym},
      {"fillRandn", FillRandn}, {"version", Version}, {"recordBegin", RecordBegin}, {"recordEnd", RecordEnd},
      {"replay", Replay}, {"recordInfo", RecordInfo}, {"recordFree", RecordFree}, {"chainInfo", ChainInfo}, {"chainBegin", ChainBegin}, {"chainEnd", ChainEnd},
      {"chainRun", ChainRun}, {"chainStatus", ChainStatus}, {"chainFree", ChainFree},
      {"rowstats", Rowstats}, {"normadd", Normadd}, {"argmaxM", ArgmaxM}, {"uploadFile", UploadFile},
  };
  for (auto& f : fns) {
    napi_value v;
    napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.fn, nullptr, &v);
    napi_set_named_property(env, exports, f.name, v);
  }
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Init)
