// Host-side helpers shared by the C-ABI sources: the error channel and the
// HIP status check, bf16/f16 conversions, host copies of the weight
// tensors callers pass in, and a growable device buffer.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/relpos_mhsa.h"
#include "host_error.hpp"

namespace {

inline int32_t fail(int32_t code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return mhsa::set_error(code, buf);
}

#define HIPCHK(expr)                                                                               \
  do {                                                                                             \
    hipError_t e_ = (expr);                                                                        \
    if (e_ != hipSuccess) return fail(MHSA_EHIP, "%s: %s (%s:%d)", #expr, hipGetErrorString(e_), \
                                      __FILE__, __LINE__);                                         \
  } while (0)

inline float bits_to_f32(uint32_t u) {
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
inline uint32_t f32_to_bits(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}
// bf16 round-to-nearest-even (no NaNs on this path).
inline uint16_t f32_to_bf16(float f) {
  uint32_t u = f32_to_bits(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
inline float bf16_to_f32(uint16_t b) { return bits_to_f32((uint32_t)b << 16); }
inline float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }
inline float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
  if (exp == 0) {
    if (man == 0) return bits_to_f32(sign);
    // subnormal: value = man * 2^-24
    float v = std::ldexp((float)man, -24);
    return sign ? -v : v;
  }
  if (exp == 31) return bits_to_f32(sign | 0x7F800000u | (man << 13));
  return bits_to_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

inline float load_host(int32_t dtype, const void* data, size_t i) {
  switch (dtype) {
    case MHSA_F32: return static_cast<const float*>(data)[i];
    case MHSA_BF16: return bf16_to_f32(static_cast<const uint16_t*>(data)[i]);
    case MHSA_F16: return f16_to_f32(static_cast<const uint16_t*>(data)[i]);
    default: return 0.f;
  }
}
inline bool float_dtype(int32_t d) { return d == MHSA_F32 || d == MHSA_BF16 || d == MHSA_F16; }

struct HostLinear {
  bool quantized = false;
  std::vector<float> w;          // standard [out, in]
  std::vector<float> bias;       // [out], empty = none
  std::vector<uint32_t> codes;   // quantized [out, in/4]
  std::vector<float> qs, qb;     // quantized scales / biases [out, in/64]
};

struct DevLinear {
  bool quantized = false;
  const void* w = nullptr;   // dense [N, K] (compute dtype) or u32 codes
  const float* sb = nullptr; // [N, K/64, 2]
  const float* bias = nullptr;
};

struct DevBuf {
  void* p = nullptr;
  size_t n = 0;
  ~DevBuf() { release(); }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    n = 0;
  }
  hipError_t ensure(size_t bytes) {
    if (bytes <= n) return hipSuccess;
    release();
    hipError_t e = hipMalloc(&p, bytes);
    if (e == hipSuccess) n = bytes;
    else p = nullptr;
    return e;
  }
};

// Tensors a weight map holds, looked up by name.
struct TensorMap {
  const mhsa_tensor* t;
  int n;
  const mhsa_tensor* find(const std::string& key) const {
    for (int i = 0; i < n; ++i)
      if (t[i].name && key == t[i].name) return &t[i];
    return nullptr;
  }
};

inline int64_t numel(const mhsa_tensor* t) {
  int64_t e = 1;
  for (int i = 0; i < t->ndim; ++i) e *= t->shape[i];
  return e;
}

// load_linear_layer (quantization.rs:289-349) for an [O, I] projection at
// `prefix`: MLX affine 8-bit when .weight, .scales and .biases are all there
// (u32 codes, f16 scales/biases), else a float .weight as [O, I] or a
// pointwise-conv [O, 1, I]; the loaded layer's bias is the checkpoint's
// .bias or none. *found is false (and h untouched) when .weight is absent.
inline int32_t load_linear(const TensorMap& m, const std::string& prefix, int O, int I, int bits, int group,
                           HostLinear& h, bool* found) {
  const mhsa_tensor* w = m.find(prefix + ".weight");
  const mhsa_tensor* sc = m.find(prefix + ".scales");
  const mhsa_tensor* qb = m.find(prefix + ".biases");
  const mhsa_tensor* b = m.find(prefix + ".bias");
  *found = w != nullptr;
  if (!w) return MHSA_OK;
  if (b && (!float_dtype(b->dtype) || numel(b) != O))
    return fail(MHSA_EINVAL, "`%s.bias`: expected float [%d]", prefix.c_str(), O);
  HostLinear next;
  if (sc && qb) {  // quantization.rs:299-304
    if (bits != 8 || group != 64)
      return fail(MHSA_ENOTSUP, "`%s`: quantization bits=%d group_size=%d not supported (8, 64)", prefix.c_str(),
                  bits, group);
    if (w->dtype != MHSA_U32 || sc->dtype != MHSA_F16 || qb->dtype != MHSA_F16 || numel(w) != (int64_t)O * I / 4 ||
        numel(sc) != (int64_t)O * I / 64 || numel(qb) != numel(sc))
      return fail(MHSA_EINVAL, "`%s`: expected u32 [%d, %d] and f16 [%d, %d] scales/biases", prefix.c_str(), O,
                  I / 4, O, I / 64);
    next.quantized = true;
    const uint32_t* wp = static_cast<const uint32_t*>(w->data);
    next.codes.assign(wp, wp + (size_t)O * I / 4);
    next.qs.resize((size_t)O * I / 64);
    next.qb.resize(next.qs.size());
    for (size_t e = 0; e < next.qs.size(); ++e) {
      next.qs[e] = f16_to_f32(static_cast<const uint16_t*>(sc->data)[e]);
      next.qb[e] = f16_to_f32(static_cast<const uint16_t*>(qb->data)[e]);
    }
  } else {
    const bool shape_ok = (w->ndim == 2 && w->shape[0] == O && w->shape[1] == I) ||
                          (w->ndim == 3 && w->shape[0] == O && w->shape[1] == 1 && w->shape[2] == I);
    if (!shape_ok || !float_dtype(w->dtype))
      return fail(MHSA_EINVAL, "`%s.weight`: expected float [%d, %d]", prefix.c_str(), O, I);
    next.w.resize((size_t)O * I);
    for (size_t e = 0; e < next.w.size(); ++e) next.w[e] = load_host(w->dtype, w->data, e);
  }
  if (b) {
    next.bias.resize(O);
    for (int e = 0; e < O; ++e) next.bias[e] = load_host(b->dtype, b->data, e);
  }
  h = std::move(next);
  return MHSA_OK;
}

inline int64_t align_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Per-kernel HIP-event timing on the launch stream (off unless enabled).
struct Profiler {
  bool on = false;
  // while on: launches tagged repeat_tag are issued repeat_n times inside
  // one event pair, which spreads the event overhead over repeat_n launches
  std::string repeat_tag;
  int repeat_n = 1;
  struct Pair {
    hipEvent_t a = nullptr, b = nullptr;
    std::string tag;
    int n = 1;
  };
  std::vector<Pair> pool;
  size_t used = 0;
  std::vector<std::string> names;
  std::vector<double> ms;
  std::vector<int> count;

  ~Profiler() {
    for (Pair& p : pool) {
      if (p.a) (void)hipEventDestroy(p.a);
      if (p.b) (void)hipEventDestroy(p.b);
    }
  }
  // `repeatable` false: the launches are issued once whatever the repeat tag
  // (in-place forms, whose second pass would read their own output).
  int begin(const char* tag, hipStream_t s, bool repeatable = true) {
    if (!on) return -1;
    if (used == pool.size()) {
      Pair p;
      if (hipEventCreate(&p.a) != hipSuccess || hipEventCreate(&p.b) != hipSuccess) return -1;
      pool.push_back(p);
    }
    Pair& p = pool[used];
    p.tag = tag;
    p.n = repeatable ? reps(tag) : 1;
    if (hipEventRecord(p.a, s) != hipSuccess) return -1;
    return (int)used++;
  }
  // How many times the launches tagged `tag` are issued.
  int reps(const char* tag) const { return on && repeat_n > 1 && repeat_tag == tag ? repeat_n : 1; }
  void end(int idx, hipStream_t s) {
    if (idx >= 0) (void)hipEventRecord(pool[idx].b, s);
  }
  // Wait for the recorded pairs and fold them into the totals.
  void flush() {
    for (size_t i = 0; i < used; ++i) {
      float t = 0.f;
      if (hipEventSynchronize(pool[i].b) != hipSuccess || hipEventElapsedTime(&t, pool[i].a, pool[i].b) != hipSuccess)
        continue;
      size_t k = 0;
      while (k < names.size() && names[k] != pool[i].tag) ++k;
      if (k == names.size()) {
        names.push_back(pool[i].tag);
        ms.push_back(0.0);
        count.push_back(0);
      }
      ms[k] += t;
      count[k] += pool[i].n;
    }
    used = 0;
  }
  // The C-ABI profile calls shared by every handle type.
  int32_t enable(int32_t e) {
    flush();
    on = e != 0;
    return MHSA_OK;
  }
  int32_t set_repeat(const char* tag, int32_t n) {
    if (n < 1 || (n > 1 && !tag)) return fail(MHSA_EINVAL, "repeat count must be >= 1 (with a tag)");
    repeat_tag = tag ? tag : "";
    repeat_n = n;
    return MHSA_OK;
  }
  int32_t reset() {
    flush();
    names.clear();
    ms.clear();
    count.clear();
    return MHSA_OK;
  }
  int32_t entries() {
    flush();
    return (int32_t)names.size();
  }
  int32_t entry(int32_t idx, const char** name, double* total_ms, int32_t* launches) {
    flush();
    if (idx < 0 || idx >= (int32_t)names.size()) return fail(MHSA_EINVAL, "profile entry %d out of range", idx);
    if (name) *name = names[idx].c_str();
    if (total_ms) *total_ms = ms[idx];
    if (launches) *launches = count[idx];
    return MHSA_OK;
  }
};

// Brackets the kernels launched in its scope with a profiling event pair.
struct ProfScope {
  Profiler& p;
  hipStream_t s;
  int idx;
  ProfScope(Profiler& prof, const char* tag, hipStream_t s_, bool enabled = true, bool repeatable = true)
      : p(prof), s(s_), idx(enabled ? prof.begin(tag, s_, repeatable) : -1) {}
  ~ProfScope() { p.end(idx, s); }
  // How many times the scope's launches are to be issued: the count its span
  // is credited with, so the per-launch average stays right.
  int reps() const { return idx >= 0 ? p.pool[idx].n : 1; }
  // Close the current span and open the next one.
  void next(const char* tag, bool repeatable = true) {
    p.end(idx, s);
    idx = idx >= 0 || p.on ? p.begin(tag, s, repeatable) : -1;
  }
};

}  // namespace
