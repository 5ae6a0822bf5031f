// Shared device helpers for the tsfast scan kernels (gfx950 / CDNA4, wave64).
//
// Everything here is plain HIP: float / float2 arithmetic, bf16 <-> f32 conversion with
// round-to-nearest-even (the rounding torch uses for .to(torch.bfloat16)), and the
// transcendental building blocks the Mamba kernels need. No host code lives here.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define TSF_DEV __device__ __forceinline__
#define TSF_HOST_DEV __host__ __device__ __forceinline__

namespace tsf {

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;

// ------------------------------------------------------------------ bf16 storage
// bf16 values travel as raw uint16_t; the kernels compute in fp32.
struct bf16 {
  uint16_t bits;
};

TSF_DEV float to_f32(float x) { return x; }
TSF_DEV float to_f32(bf16 x) { return __uint_as_float(static_cast<uint32_t>(x.bits) << 16); }

template <typename T>
TSF_DEV T from_f32(float x);
template <>
TSF_DEV float from_f32<float>(float x) { return x; }
// Round to nearest even with NaN kept quiet: the fptrunc lowers to gfx950's v_cvt_pk_bf16_f32.
template <>
TSF_DEV bf16 from_f32<bf16>(float x) {
  bf16 r;
  r.bits = __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
  return r;
}

// Row access by a 32-bit element index: the byte offset is formed in 32 bits, so the access
// is an SGPR base plus a VGPR byte offset (the global load/store "saddr" form) with no 64-bit
// address arithmetic. The caller guarantees that idx * sizeof(T) fits in 32 bits.
template <typename T>
TSF_DEV T ld32(const T* __restrict__ base, uint32_t idx) {
  return *reinterpret_cast<const T*>(reinterpret_cast<const char*>(base) + idx * (uint32_t)sizeof(T));
}
template <typename T>
TSF_DEV void st32(T* __restrict__ base, uint32_t idx, T v) {
  *reinterpret_cast<T*>(reinterpret_cast<char*>(base) + idx * (uint32_t)sizeof(T)) = v;
}

// ------------------------------------------------------------------ buffer accesses
// A raw buffer resource over [base, base + bytes): the hardware checks every access against
// `bytes`, so a load at or beyond it returns 0 and such a store is dropped. Offsets are a per-lane
// VGPR byte offset plus a wave-uniform SGPR byte offset (stepped by scalar adds), so streaming
// through a row costs no vector address arithmetic. The kernels keep voff + soff below 2^32.
using Rsrc = __amdgpu_buffer_rsrc_t;
// gfx9 raw-buffer descriptor word 3 (32-bit data format, no swizzle)
constexpr int kBufWord3 = 0x00020000;
TSF_DEV Rsrc make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufWord3);
}
TSF_DEV float buf_ld(Rsrc r, uint32_t voff, uint32_t soff, float*) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
TSF_DEV bf16 buf_ld(Rsrc r, uint32_t voff, uint32_t soff, bf16*) {
  bf16 v;
  v.bits = __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
  return v;
}
template <typename T>
TSF_DEV T buf_load(Rsrc r, uint32_t voff, uint32_t soff) {
  return buf_ld(r, voff, soff, static_cast<T*>(nullptr));
}
TSF_DEV void buf_store(float v, Rsrc r, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, voff, soff, 0);
}
TSF_DEV void buf_store(bf16 v, Rsrc r, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b16(v.bits, r, voff, soff, 0);
}

// ------------------------------------------------------------------ complex (interleaved re/im)
TSF_DEV float2 cmul(float2 a, float2 b) { return make_float2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x); }
// a * conj(b)
TSF_DEV float2 cmul_conj(float2 a, float2 b) { return make_float2(a.x * b.x + a.y * b.y, a.y * b.x - a.x * b.y); }
TSF_DEV float2 cconj(float2 a) { return make_float2(a.x, -a.y); }
TSF_DEV float2 cadd(float2 a, float2 b) { return make_float2(a.x + b.x, a.y + b.y); }
// a * x + b
TSF_DEV float2 cfma(float2 a, float2 x, float2 b) {
  return make_float2(fmaf(a.x, x.x, fmaf(-a.y, x.y, b.x)), fmaf(a.x, x.y, fmaf(a.y, x.x, b.y)));
}

// Scalar traits so one kernel body serves float (real) and float2 (complex) lanes.
template <typename T>
struct Num;
template <>
struct Num<float> {
  TSF_DEV static float zero() { return 0.0f; }
  TSF_DEV static float one() { return 1.0f; }
  TSF_DEV static float mul(float a, float b) { return a * b; }
  TSF_DEV static float fma(float a, float x, float b) { return fmaf(a, x, b); }
  TSF_DEV static float add(float a, float b) { return a + b; }
  TSF_DEV static float conj(float a) { return a; }
  TSF_DEV static float mul_conj(float a, float b) { return a * b; }
};
template <>
struct Num<float2> {
  TSF_DEV static float2 zero() { return make_float2(0.0f, 0.0f); }
  TSF_DEV static float2 one() { return make_float2(1.0f, 0.0f); }
  TSF_DEV static float2 mul(float2 a, float2 b) { return cmul(a, b); }
  TSF_DEV static float2 fma(float2 a, float2 x, float2 b) { return cfma(a, x, b); }
  TSF_DEV static float2 add(float2 a, float2 b) { return cadd(a, b); }
  TSF_DEV static float2 conj(float2 a) { return cconj(a); }
  TSF_DEV static float2 mul_conj(float2 a, float2 b) { return cmul_conj(a, b); }
};

template <>
struct Num<double> {
  TSF_DEV static double zero() { return 0.0; }
  TSF_DEV static double one() { return 1.0; }
  TSF_DEV static double mul(double a, double b) { return a * b; }
  TSF_DEV static double fma(double a, double x, double b) { return ::fma(a, x, b); }
  TSF_DEV static double add(double a, double b) { return a + b; }
  TSF_DEV static double conj(double a) { return a; }
  TSF_DEV static double mul_conj(double a, double b) { return a * b; }
};
template <>
struct Num<double2> {
  TSF_DEV static double2 zero() { return make_double2(0.0, 0.0); }
  TSF_DEV static double2 one() { return make_double2(1.0, 0.0); }
  TSF_DEV static double2 mul(double2 a, double2 b) {
    return make_double2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
  }
  TSF_DEV static double2 fma(double2 a, double2 x, double2 b) {
    return make_double2(::fma(a.x, x.x, ::fma(-a.y, x.y, b.x)), ::fma(a.x, x.y, ::fma(a.y, x.x, b.y)));
  }
  TSF_DEV static double2 add(double2 a, double2 b) { return make_double2(a.x + b.x, a.y + b.y); }
  TSF_DEV static double2 conj(double2 a) { return make_double2(a.x, -a.y); }
  TSF_DEV static double2 mul_conj(double2 a, double2 b) {
    return make_double2(a.x * b.x + a.y * b.y, a.y * b.x - a.x * b.y);
  }
};

// fp32 storage type -> fp64 compute type (the scans are HBM-bound, so carrying the state in
// double costs no time and keeps long / slowly-decaying recurrences at fp32 output accuracy).
template <typename T>
struct Wide;
template <>
struct Wide<float> {
  using type = double;
  TSF_DEV static double up(float x) { return (double)x; }
  TSF_DEV static float down(double x) { return (float)x; }
};
template <>
struct Wide<float2> {
  using type = double2;
  TSF_DEV static double2 up(float2 x) { return make_double2((double)x.x, (double)x.y); }
  TSF_DEV static float2 down(double2 x) { return make_float2((float)x.x, (float)x.y); }
};

// x^k for an integer k >= 0 by binary powering (log2(k) squarings; exact for k = 0).
template <typename T>
TSF_DEV T ipow(T x, int64_t k) {
  T r = Num<T>::one();
  while (k > 0) {
    if (k & 1) r = Num<T>::mul(r, x);
    x = Num<T>::mul(x, x);
    k >>= 1;
  }
  return r;
}

// ------------------------------------------------------------------ Mamba scalar maps
// 2^x on the hardware transcendental unit (v_exp_f32); the kernels pre-scale A by log2(e).
TSF_DEV float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr float kLn2 = 0.6931471805599453f;

// softplus with torch.nn.functional.softplus's threshold: x for x > 20, else log(1 + e^x).
TSF_DEV float softplus(float x) { return x > 20.0f ? x : log1pf(__expf(x)); }

TSF_DEV float sigmoid(float x) { return 1.0f / (1.0f + __expf(-x)); }

// log(1 + e^x) on the transcendental unit: e = e^x, u = 1 + e rounded, and
// log1p(e) = e * log(u) / (u - 1), exact to a few ulp because the rounding error of u cancels
// between numerator and denominator (Goldberg, "What every computer scientist should know
// about floating-point arithmetic", 1991, theorem 4). Returns e and u for the caller (the
// derivative of softplus is e / u).
struct SoftplusParts {
  float value, e, u;
};
TSF_DEV SoftplusParts softplus_parts(float x) {
  const float e = __builtin_amdgcn_exp2f(fminf(x, 20.0f) * kLog2e);
  const float u = 1.0f + e;
  const float dm = u - 1.0f;
  const float lg = __builtin_amdgcn_logf(u) * kLn2;
  const float lp = dm == 0.0f ? e : lg * (e * __builtin_amdgcn_rcpf(dm));
  SoftplusParts r;
  r.value = x > 20.0f ? x : lp;
  r.e = e;
  r.u = u;
  return r;
}
TSF_DEV float softplus_fast(float x) { return softplus_parts(x).value; }
// softplus as the reference's kernels write it (mamba_triton.py:75-78): log(1 + e^x) with x
// above 20 passed through, on the transcendental unit (v_exp, v_log)
TSF_DEV float softplus_ref(float x) {
  const float e = __builtin_amdgcn_exp2f(fminf(x, 20.0f) * kLog2e);
  return x > 20.0f ? x : __builtin_amdgcn_logf(1.0f + e) * kLn2;
}
TSF_DEV float sigmoid_fast(float x) { return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * kLog2e)); }

// ------------------------------------------------------------------ wave reductions
// Reduce-scatter of K values (K a power of two, K <= 64) held by every lane of a wave64:
// on return v[0] of lane l holds the sum over all 64 lanes of value index (l >> (6 - log2 K)).
// Each halving level exchanges half of the remaining values with the partner lane, so the
// whole reduction costs K - 1 exchanges instead of 6 * K for independent butterflies.
template <int K>
TSF_DEV void wave_reduce_scatter(float* v, int lane) {
  static_assert(K >= 1 && K <= 64 && (K & (K - 1)) == 0, "K must be a power of two <= 64");
  int k = K;
#pragma unroll
  for (int mask = 32; mask >= 1; mask >>= 1) {
    if (k > 1) {
      const bool upper = (lane & mask) != 0;
      const int half = k >> 1;
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        if (i < half) {
          const float send = upper ? v[i] : v[i + half];
          const float keep = upper ? v[i + half] : v[i];
          v[i] = keep + __shfl_xor(send, mask, kWave);
        }
      }
      k = half;
    } else {
      v[0] += __shfl_xor(v[0], mask, kWave);
    }
  }
}

// Compute units of the current device (queried once per device).
inline unsigned device_cus() {
  static unsigned cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = (unsigned)n;
  }
  return cache[dev];
}

}  // namespace tsf

// Host side: status of the launches just enqueued (records the HIP error for the status string).
int tsf_record_hip_error(hipError_t e);
inline int tsf_launch_status() { return tsf_record_hip_error(hipGetLastError()); }
// Process-wide deterministic mode of the look-back scans (tsfast_hip_set_deterministic).
int tsf_deterministic();
// Look-back failure reporting (csrc/status.hip): the device address of the host-mapped alarm
// word that a give-up sets (nullptr when it could not be allocated) and the current wait bound.
unsigned* tsf_lookback_alarm();
uint32_t tsf_lookback_spin_limit();
uint32_t tsf_next_epoch();  // call number of the next look-back scan (never 0)
