// t0mi_tuner.hip — GemmTuner: measure-and-pick with an in-memory and a disk cache.
//
//   GemmTuner::new / with_cache_dir / tune / invalidate / clear / report
//       src/t0/auto_gemm.rs:46-527
//   smoke_test_256 (pre-flight correctness gate)   src/t0/auto_gemm.rs:223-272
//   benchmark_one (median of n_iters)              src/t0/auto_gemm.rs:279-348
//   global_tuner / auto_gemm                       src/t0/auto_gemm.rs:535-590
//
// Same pipeline: memory cache -> disk JSON -> cost-model candidates -> 256^3
// integer-pattern smoke test against a CPU sum -> timing (median) -> persist.
// gfx950 differences: candidates come from the gfx950 cost model over the
// prebuilt kernels (t0mi_config.cpp), timing uses hipEvents around each launch
// rather than host wall clock, and results live in their own directory
// ($HOME/.t0mi_autotune_gfx950) keyed by shape, layout and output dtype.
#include <errno.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <dirent.h>
#include <unistd.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include "t0mi_ctx.h"

using namespace t0mi;

namespace {

struct TuneResult {
  t0mi_gemm_config best;
  double best_tflops = 0;
  std::vector<std::pair<std::string, double>> all;
  bool from_cache = false;
};

typedef std::tuple<uint32_t, uint32_t, uint32_t, uint32_t, uint32_t> Key;  // m, n, k, transpose, out_dtype

bool parse_u32(const std::string& js, const char* key, uint32_t* out) {
  // auto_gemm.rs:603-611: find "key": then digits.
  std::string needle = std::string("\"") + key + "\":";
  size_t p = js.find(needle);
  if (p == std::string::npos) return false;
  p += needle.size();
  size_t e = p;
  while (e < js.size() && js[e] >= '0' && js[e] <= '9') ++e;
  if (e == p) return false;
  *out = (uint32_t)strtoul(js.substr(p, e - p).c_str(), nullptr, 10);
  return true;
}

bool parse_f64(const std::string& js, const char* key, double* out) {
  std::string needle = std::string("\"") + key + "\":";
  size_t p = js.find(needle);
  if (p == std::string::npos) return false;
  p += needle.size();
  size_t e = p;
  while (e < js.size() && ((js[e] >= '0' && js[e] <= '9') || js[e] == '.' || js[e] == '-')) ++e;
  if (e == p) return false;
  char* end = nullptr;
  std::string s = js.substr(p, e - p);
  *out = strtod(s.c_str(), &end);
  return end && *end == 0;
}

bool parse_bool(const std::string& js, const char* key, uint32_t* out) {
  std::string t = std::string("\"") + key + "\":true", f = std::string("\"") + key + "\":false";
  if (js.find(t) != std::string::npos) {
    *out = 1;
    return true;
  }
  if (js.find(f) != std::string::npos) {
    *out = 0;
    return true;
  }
  return false;
}

}  // namespace

struct t0mi_tuner {
  std::string cache_dir;
  uint32_t max_candidates = 8;  // auto_gemm.rs:61
  uint32_t n_iters = 5;         // auto_gemm.rs:62
  std::map<Key, TuneResult> cache;
  std::mutex mu;

  std::string path(const Key& key) const {
    // gemm_{M}x{N}x{K}.json (auto_gemm.rs:435-437), plus layout / dtype tags.
    char buf[128];
    snprintf(buf, sizeof buf, "gemm_%ux%ux%u%s%s.json", std::get<0>(key), std::get<1>(key), std::get<2>(key),
             std::get<3>(key) == T0MI_NN ? "_nn" : "", std::get<4>(key) == T0MI_OUT_BF16 ? "_bf16o" : "");
    return cache_dir + "/" + buf;
  }

  bool load(const Key& key, TuneResult* r) const {
    FILE* f = fopen(path(key).c_str(), "rb");
    if (!f) return false;
    std::string js;
    char buf[4096];
    size_t n;
    while ((n = fread(buf, 1, sizeof buf, f)) > 0) js.append(buf, n);
    fclose(f);
    t0mi_gemm_config c;
    memset(&c, 0, sizeof c);
    uint32_t sk = 1;
    if (!parse_u32(js, "tile_m", &c.tile_m) || !parse_u32(js, "tile_n", &c.tile_n) ||
        !parse_u32(js, "tile_k", &c.tile_k) || !parse_u32(js, "wg_size", &c.wg_size) ||
        !parse_f64(js, "tflops", &r->best_tflops))
      return false;
    parse_u32(js, "split_k", &sk);
    c.split_k = sk > 1 ? sk : 0;
    parse_u32(js, "lds_pad", &c.lds_pad);
    c.n_col_passes = 1;
    parse_u32(js, "n_col_passes", &c.n_col_passes);
    parse_bool(js, "wgp", &c.wgp_mode);
    parse_bool(js, "swap", &c.swap_grid);
    parse_u32(js, "wave_m", &c.wave_m);
    parse_u32(js, "wave_n", &c.wave_n);
    parse_u32(js, "stages", &c.stages);
    if (c.stages == 2) c.stages = 0;
    c.use_lds = 1;
    c.double_buffer = 1;
    c.transpose = std::get<3>(key);
    c.out_dtype = std::get<4>(key);
    // A cache entry must name a feasible, prebuilt kernel, else it is stale.
    if (!config_feasible(c, nullptr) || !has_variant(c)) return false;
    r->best = c;
    r->all.clear();
    r->from_cache = true;
    return true;
  }

  void save(const Key& key, const TuneResult& r) const {
    mkdir(cache_dir.c_str(), 0755);
    std::string all;
    for (const auto& a : r.all) {
      char b[256];
      snprintf(b, sizeof b, "%s[\"%s\",%.2f]", all.empty() ? "" : ",", a.first.c_str(), a.second);
      all += b;
    }
    const t0mi_gemm_config& c = r.best;
    char head[512];
    snprintf(head, sizeof head,
             "{\"tile_m\":%u,\"tile_n\":%u,\"tile_k\":%u,\"wg_size\":%u,\"split_k\":%u,\"lds_pad\":%u,"
             "\"n_col_passes\":%u,\"wgp\":%s,\"swap\":%s,\"wave_m\":%u,\"wave_n\":%u,\"stages\":%u,\"tflops\":%.2f,"
             "\"all\":[",
             c.tile_m, c.tile_n, c.tile_k, c.wg_size, split_k_of(c), c.lds_pad, c.n_col_passes,
             c.wgp_mode ? "true" : "false", c.swap_grid ? "true" : "false", c.wave_m, c.wave_n, stages_of(c),
             r.best_tflops);
    std::string js = std::string(head) + all + "]}";
    FILE* f = fopen(path(key).c_str(), "wb");
    if (!f) {
      fprintf(stderr, "[t0mi autotune] cache write failed: %s\n", strerror(errno));
      return;
    }
    fwrite(js.data(), 1, js.size(), f);
    fclose(f);
  }
};

namespace {

uint16_t bf16_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return (uint16_t)(u >> 16);  // exact for the small integers used here
}

// smoke_test_256 (auto_gemm.rs:223-272): 256^3 with a=(i%7)-3, b=(j%5)-2 (sums
// are exact integers), one dispatch, CPU check of diagonal + scattered points.
int smoke_test_256(t0mi_ctx* ctx, const t0mi_gemm_config& cfg, bool* ok) {
  const uint32_t S = 256;
  std::vector<uint16_t> a(S * S), b(S * S);
  for (uint32_t i = 0; i < S * S; ++i) a[i] = bf16_bits((float)(int)(i % 7) - 3.0f);
  for (uint32_t j = 0; j < S * S; ++j) b[j] = bf16_bits((float)(int)(j % 5) - 2.0f);
  uint64_t da = 0, db = 0, dc = 0;
  int rc = t0mi_alloc(ctx, S * S * 2, &da);
  if (!rc) rc = t0mi_alloc(ctx, S * S * 2, &db);
  if (!rc) rc = t0mi_alloc(ctx, S * S * 4, &dc);
  if (!rc) rc = t0mi_h2d(ctx, da, a.data(), S * S * 2);
  if (!rc) rc = t0mi_h2d(ctx, db, b.data(), S * S * 2);
  t0mi_gemm_config c = cfg;
  c.out_dtype = T0MI_OUT_F32;
  c.epilogue = T0MI_EPI_STORE_F32;
  if (!rc) rc = t0mi_gemm(ctx, &c, da, db, dc, 0, S, S, S);
  if (!rc) rc = t0mi_wait_idle(ctx);
  std::vector<float> out(S * S);
  if (!rc) rc = t0mi_d2h(ctx, out.data(), dc, S * S * 4);
  if (!rc) {
    *ok = true;
    std::vector<uint32_t> idx;
    for (uint32_t i = 0; i < 16; ++i) idx.push_back(i * S + i);
    for (uint32_t i = 0; i < 56; ++i) idx.push_back(i * 331 + 97);
    for (uint32_t id : idx) {
      const uint32_t r = id / S, col = id % S;
      long s = 0;
      for (uint32_t kk = 0; kk < S; ++kk) {
        const long av = (long)((r * S + kk) % 7) - 3;
        const long bv = c.transpose == T0MI_NN ? (long)((kk * S + col) % 5) - 2 : (long)((col * S + kk) % 5) - 2;
        s += av * bv;
      }
      if (fabs((double)out[id] - (double)s) > 0.05) *ok = false;
    }
  }
  if (da) t0mi_free(ctx, da);
  if (db) t0mi_free(ctx, db);
  if (dc) t0mi_free(ctx, dc);
  return rc;
}

// bf16 values of mean 0 and variance 1 (the sum of four uniforms from a
// counter hash, centred and scaled): random mantissas and signs, so timed
// candidates draw the power of a real GEMM.  On MI355X power sets the clock; a
// constant pattern toggles few multiplier bits and lets a kernel clock higher
// than it will on real data, which can reorder the candidates.
__global__ __launch_bounds__(256) void t0mi_fill_normal_bf16(uint16_t* __restrict__ dst, size_t n, uint64_t seed) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    uint64_t z = seed + (uint64_t)i * 0x9E3779B97F4A7C15ull;  // splitmix64 of the index
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    const float u = (float)(z & 0xFFFF) + (float)((z >> 16) & 0xFFFF) + (float)((z >> 32) & 0xFFFF) +
                    (float)(z >> 48);
    const float x = (u * (1.0f / 65536.0f) - 2.0f) * 1.7320508f;  // Var(sum of 4 U(0,1)) = 1/3
    dst[i] = (uint16_t)(__builtin_bit_cast(uint32_t, x) >> 16);
  }
}

int fill_normal(t0mi_ctx* ctx, uint64_t dst, size_t n, uint64_t seed) {
  const size_t blocks = std::max<size_t>(1, std::min<size_t>((n + 255) / 256, (size_t)ctx->cu_count * 8));
  hipLaunchKernelGGL(t0mi_fill_normal_bf16, dim3((uint32_t)blocks), dim3(256), 0, ctx->stream, (uint16_t*)dst, n,
                     seed);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? T0MI_OK : set_error(T0MI_ERR_HIP, "fill launch: %s", hipGetErrorString(e));
}

// benchmark_one (auto_gemm.rs:279-348): warm-up, then n_iters timed launches;
// median -> TFLOPS.  Inputs are N(0, 1) bf16 data (fill_normal), not the
// reference's zero fill (made for a GPU whose clock power does not limit).
int benchmark_one(t0mi_ctx* ctx, const t0mi_gemm_config& cfg, uint32_t m, uint32_t n, uint32_t k, uint32_t n_iters,
                  double* tflops) {
  const size_t ab = (size_t)m * k * 2, bb = (size_t)k * n * 2, cb = (size_t)m * n * 4;
  uint64_t da = 0, db = 0, dc = 0;
  int rc = t0mi_alloc(ctx, ab, &da);
  if (!rc) rc = t0mi_alloc(ctx, bb, &db);
  if (!rc) rc = t0mi_alloc(ctx, cb, &dc);
  if (!rc) rc = fill_normal(ctx, da, (size_t)m * k, 1);
  if (!rc) rc = fill_normal(ctx, db, (size_t)k * n, 2);
  std::vector<float> ms;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (!rc && (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess))
    rc = set_error(T0MI_ERR_HIP, "hipEventCreate failed");
  if (!rc) rc = t0mi_gemm(ctx, &cfg, da, db, dc, 0, m, n, k);  // warm-up
  if (!rc) rc = t0mi_wait_idle(ctx);
  for (uint32_t i = 0; !rc && i < n_iters; ++i) {
    (void)hipEventRecord(e0, ctx->stream);
    rc = t0mi_gemm(ctx, &cfg, da, db, dc, 0, m, n, k);
    (void)hipEventRecord(e1, ctx->stream);
    if (!rc) rc = t0mi_wait_idle(ctx);
    float t = 0;
    if (!rc && hipEventElapsedTime(&t, e0, e1) == hipSuccess) ms.push_back(t);
  }
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (da) t0mi_free(ctx, da);
  if (db) t0mi_free(ctx, db);
  if (dc) t0mi_free(ctx, dc);
  if (rc) return rc;
  if (ms.empty()) return set_error(T0MI_ERR_HIP, "no timing samples");
  std::sort(ms.begin(), ms.end());
  const double med = ms[ms.size() / 2];
  *tflops = 2.0 * m * (double)n * k / (med * 1e-3) / 1e12;
  return T0MI_OK;
}

std::string default_cache_dir() {
  const char* home = getenv("HOME");
  return std::string(home ? home : "/tmp") + "/.t0mi_autotune_gfx950";
}

}  // namespace

extern "C" int t0mi_tuner_create(const char* dir, t0mi_tuner** out) {
  if (!out) return set_error(T0MI_ERR_INVALID, "null out");
  t0mi_tuner* t = new t0mi_tuner();
  t->cache_dir = dir && *dir ? std::string(dir) : default_cache_dir();
  *out = t;
  return T0MI_OK;
}

extern "C" void t0mi_tuner_destroy(t0mi_tuner* t) { delete t; }

extern "C" void t0mi_tuner_set_params(t0mi_tuner* t, uint32_t max_candidates, uint32_t n_iters) {
  if (!t) return;
  t->max_candidates = max_candidates ? max_candidates : 1;
  t->n_iters = n_iters ? n_iters : 1;
}

extern "C" int t0mi_tuner_tune(t0mi_tuner* t, t0mi_ctx* ctx, uint32_t m, uint32_t n, uint32_t k, uint32_t transpose,
                               uint32_t out_dtype, t0mi_gemm_config* best, double* tflops, int* from_cache) {
  if (!t || !best) return set_error(T0MI_ERR_INVALID, "null argument");
  if (!m || !n || !k) return set_error(T0MI_ERR_INVALID, "zero dimension");
  if (transpose > T0MI_NN || out_dtype > T0MI_OUT_BF16) return set_error(T0MI_ERR_INVALID, "bad layout/dtype");
  std::lock_guard<std::mutex> lk(t->mu);
  const Key key(m, n, k, transpose, out_dtype);
  // 1. memory cache
  auto it = t->cache.find(key);
  if (it != t->cache.end()) {
    fprintf(stderr, "[t0mi autotune] cache hit: %ux%ux%u -> %s (%.1f TF)\n", m, n, k,
            config_name(it->second.best).c_str(), it->second.best_tflops);
    *best = it->second.best;
    if (tflops) *tflops = it->second.best_tflops;
    if (from_cache) *from_cache = 1;
    return T0MI_OK;
  }
  // 2. disk cache (a corrupt or stale file is ignored and re-tuned)
  TuneResult r;
  if (t->load(key, &r)) {
    fprintf(stderr, "[t0mi autotune] cache hit: %ux%ux%u -> %s (%.1f TF)\n", m, n, k, config_name(r.best).c_str(),
            r.best_tflops);
    t->cache[key] = r;
    *best = r.best;
    if (tflops) *tflops = r.best_tflops;
    if (from_cache) *from_cache = 1;
    return T0MI_OK;
  }
  int rc = check_ctx(ctx);
  if (rc) return rc;
  if (ctx->null_backend) return set_error(T0MI_ERR_NO_DEVICE, "tuning needs a device runtime");
  // Other threads' work on this runtime waits until the timings are done.
  T0MI_SUBMIT_GUARD(ctx);
  // 3. candidates from the gfx950 cost model
  std::vector<t0mi_gemm_config> cand = rank_candidates(m, n, k, transpose, out_dtype, nullptr);
  if (cand.size() > t->max_candidates) cand.resize(t->max_candidates);
  // 3b. 256^3 smoke test; failing candidates are dropped (auto_gemm.rs:151-163)
  std::vector<t0mi_gemm_config> ok_c;
  for (const auto& c : cand) {
    bool ok = false;
    rc = smoke_test_256(ctx, c, &ok);
    if (rc == T0MI_OK && ok) {
      ok_c.push_back(c);
    } else {
      fprintf(stderr, "[t0mi autotune]   %s -> SKIP (%s)\n", config_name(c).c_str(),
              rc ? t0mi_last_error() : "256^3 correctness FAIL");
      if (ctx->poisoned.load()) return check_ctx(ctx);
    }
  }
  if (ok_c.empty()) {
    fprintf(stderr, "[t0mi autotune] all candidates failed the smoke test, falling back to legacy\n");
    rc = t0mi_auto_select_legacy(m, k, n, best);
    best->transpose = transpose;
    best->out_dtype = out_dtype;
    if (tflops) *tflops = 0;
    if (from_cache) *from_cache = 0;
    return rc;
  }
  // 4. benchmark
  fprintf(stderr, "[t0mi autotune] benchmarking %zu candidates for %ux%ux%u\n", ok_c.size(), m, n, k);
  std::vector<std::pair<t0mi_gemm_config, double>> res;
  for (const auto& c : ok_c) {
    double tf = 0;
    rc = benchmark_one(ctx, c, m, n, k, t->n_iters, &tf);
    if (rc == T0MI_OK) {
      fprintf(stderr, "[t0mi autotune]   %s -> %.1f TFLOPS\n", config_name(c).c_str(), tf);
      res.push_back({c, tf});
    } else {
      fprintf(stderr, "[t0mi autotune]   %s -> FAILED: %s\n", config_name(c).c_str(), t0mi_last_error());
      if (ctx->poisoned.load()) return check_ctx(ctx);
    }
  }
  if (res.empty()) return set_error(T0MI_ERR_HIP, "autotune: all candidates failed");
  // 5. sort by TFLOPS descending
  std::stable_sort(res.begin(), res.end(), [](const std::pair<t0mi_gemm_config, double>& a,
                                              const std::pair<t0mi_gemm_config, double>& b) { return a.second > b.second; });
  r = TuneResult();
  r.best = res[0].first;
  r.best_tflops = res[0].second;
  fprintf(stderr, "[t0mi autotune] best: %s (%.1f TFLOPS)\n", config_name(r.best).c_str(), r.best_tflops);
  for (const auto& x : res) r.all.push_back({config_name(x.first), x.second});
  // 6. persist
  t->save(key, r);
  t->cache[key] = r;
  *best = r.best;
  if (tflops) *tflops = r.best_tflops;
  if (from_cache) *from_cache = 0;
  return T0MI_OK;
}

extern "C" void t0mi_tuner_invalidate(t0mi_tuner* t, uint32_t m, uint32_t n, uint32_t k, uint32_t transpose,
                                      uint32_t out_dtype) {
  if (!t) return;
  std::lock_guard<std::mutex> lk(t->mu);
  const Key key(m, n, k, transpose, out_dtype);
  t->cache.erase(key);
  unlink(t->path(key).c_str());
}

extern "C" void t0mi_tuner_clear(t0mi_tuner* t) {
  // GemmTuner::clear removes the whole cache directory (auto_gemm.rs:510-514);
  // here only this tuner's gemm_*.json files are removed.
  if (!t) return;
  std::lock_guard<std::mutex> lk(t->mu);
  t->cache.clear();
  DIR* d = opendir(t->cache_dir.c_str());
  if (!d) return;
  while (struct dirent* e = readdir(d)) {
    std::string nm = e->d_name;
    if (nm.rfind("gemm_", 0) == 0 && nm.size() > 5 && nm.substr(nm.size() - 5) == ".json")
      unlink((t->cache_dir + "/" + nm).c_str());
  }
  closedir(d);
  rmdir(t->cache_dir.c_str());
}

extern "C" int t0mi_tuner_cache_path(t0mi_tuner* t, uint32_t m, uint32_t n, uint32_t k, uint32_t transpose,
                                     uint32_t out_dtype, char* buf, size_t len) {
  if (!t) return set_error(T0MI_ERR_INVALID, "null tuner");
  std::string p = t->path(Key(m, n, k, transpose, out_dtype));
  if (buf && len) {
    strncpy(buf, p.c_str(), len - 1);
    buf[len - 1] = 0;
  }
  return (int)p.size();
}

extern "C" int t0mi_tuner_report(t0mi_tuner* t, char* buf, size_t len) {
  if (!t) return set_error(T0MI_ERR_INVALID, "null tuner");
  std::lock_guard<std::mutex> lk(t->mu);
  std::string s = "GEMM autotune cache (" + std::to_string(t->cache.size()) + " entries)\n";
  for (const auto& kv : t->cache) {
    char line[512];
    snprintf(line, sizeof line, "  %ux%ux%u%s%s -> %s (%.1f TF) %s\n", std::get<0>(kv.first), std::get<1>(kv.first),
             std::get<2>(kv.first), std::get<3>(kv.first) == T0MI_NN ? " nn" : "",
             std::get<4>(kv.first) == T0MI_OUT_BF16 ? " bf16o" : "", config_name(kv.second.best).c_str(),
             kv.second.best_tflops, kv.second.from_cache ? "[cached]" : "[measured]");
    s += line;
  }
  if (buf && len) {
    strncpy(buf, s.c_str(), len - 1);
    buf[len - 1] = 0;
  }
  return (int)s.size();
}

namespace {
std::mutex g_tuner_mu;
t0mi_tuner* g_tuner = nullptr;
}  // namespace

extern "C" int t0mi_auto_gemm(t0mi_ctx* ctx, uint64_t a, uint64_t b, uint64_t c, uint32_t m, uint32_t n, uint32_t k,
                              double* tflops) {
  // auto_gemm (auto_gemm.rs:555-590): global tuner -> tune -> dispatch (NT, f32 out).
  t0mi_gemm_config cfg;
  double tf = 0;
  {
    std::lock_guard<std::mutex> lk(g_tuner_mu);
    if (!g_tuner) t0mi_tuner_create(nullptr, &g_tuner);
    int rc = t0mi_tuner_tune(g_tuner, ctx, m, n, k, T0MI_NT, T0MI_OUT_F32, &cfg, &tf, nullptr);
    if (rc) return rc;
  }
  int rc = t0mi_gemm(ctx, &cfg, a, b, c, 0, m, n, k);
  if (rc) return rc;
  rc = t0mi_wait_idle(ctx);
  if (tflops) *tflops = tf;
  return rc;
}
