// Device numerics of the W8A8 decoder datapath (gfx950).
//
// Two fp32 regimes, as in the reference:
//  - the vector steps (norm, quant, dequant, RoPE, residual, softmax glue) are plain
//    IEEE binary32 with round-to-nearest-even and gradual underflow, one rounding per
//    step and never a fused multiply-add: DeviceModel runs them in NumPy float32
//    (llm/ref_model.py:191-255). The library is built with -ffp-contract=off and the
//    default f32 denormal mode (preserve), so `a * b` and `a + b` are exactly that.
//  - the SFU (exp / recip / rsqrt) is a fixed sequence of fp32 operations with
//    flush-to-zero (llm/fp32.py:7-13, llm/sfu.py:7-25): a subnormal input is a signed
//    zero, a result below 2^-126 after rounding to 24 bits with an unbounded exponent
//    is a signed zero. fadd_ftz / fmul_ftz / ldexp_ftz give that rule on top of the
//    IEEE instructions (see each for why the fix-up is exact).
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#define T2R_DEV __device__ __forceinline__

namespace t2r {

// Kernel timing: while a profiling scope of the model is open, launches go through
// hipExtLaunchKernelGGL with events recorded at the kernel's own start (the scope's first launch)
// and end (every launch; the last one stands), so the measured time excludes dispatch latency.
struct LaunchEvents {
  hipEvent_t start = nullptr, stop = nullptr;
};
inline thread_local LaunchEvents g_launch_events;

template <typename K, typename... A>
void launch(K kernel, dim3 grid, dim3 block, size_t shmem, hipStream_t st, A... args) {
  LaunchEvents& e = g_launch_events;
  if (e.stop != nullptr) {
    hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)shmem, st, e.start, e.stop, 0, args...);
    e.start = nullptr;
  } else {
    hipLaunchKernelGGL(kernel, grid, block, shmem, st, args...);
  }
}

constexpr uint32_t kQNaN = 0x7FC00000u;
constexpr uint32_t kPInf = 0x7F800000u;
constexpr float kInv127 = (float)(1.0 / 127.0);      // F(1/127): double quotient rounded once

// SFU tables in constant memory: [exp T | exp S | recip T | recip S | rsqrt T(128) | rsqrt S(128)].
constexpr int kSfuExpT = 0, kSfuExpS = 64, kSfuRecT = 128, kSfuRecS = 192, kSfuRsqT = 256, kSfuRsqS = 384;
constexpr int kSfuWords = 512;
extern __constant__ float c_sfu[kSfuWords];

T2R_DEV uint32_t fb(float x) { return __float_as_uint(x); }
T2R_DEV float fv(uint32_t b) { return __uint_as_float(b); }

// subnormal -> zero of the same sign
T2R_DEV float ftz(float x) {
  uint32_t b = fb(x);
  return (b & 0x7F800000u) ? x : fv(b & 0x80000000u);
}

// a + b with the FTZ rule, for a, b already flushed. The exact sum of two normal binary32
// values that lies below 2^-126 is a multiple of 2^-149 with fewer than 24 significant bits,
// so the IEEE instruction returns it exactly and the rule flushes it; every sum at or above
// 2^-126 rounds identically in both.
T2R_DEV float fadd_ftz(float a, float b) { return ftz(a + b); }

// a * b with the FTZ rule, for a, b already flushed. IEEE and the rule agree whenever the
// exact product is >= 2^-126; below it the rule gives +-0 unless the product rounds up to
// 2^-126 at 24-bit precision (exact >= 2^-126 - 2^-151), while IEEE rounds at the subnormal
// spacing. Only a result of exactly 2^-126 is ambiguous: recompute it scaled by 2^128
// (both factors are then below 2 in magnitude, so nothing overflows) and compare.
T2R_DEV float fmul_ftz(float a, float b) {
  float r = a * b;
  uint32_t m = fb(r) & 0x7FFFFFFFu;
  if (m < 0x00800000u) return fv(fb(r) & 0x80000000u);
  if (m == 0x00800000u) {
    float r2 = (a * 0x1p64f) * (b * 0x1p64f);
    if (fabsf(r2) < 4.0f) return fv(fb(r) & 0x80000000u);
  }
  return r;
}

// a * 2^n as an exponent-field add (llm/fp32.py:147-151): below the normal range a signed
// zero, above it a signed inf; zero and inf pass through, NaN gives the canonical NaN.
T2R_DEV float ldexp_ftz(float a, int n) {
  uint32_t b = fb(a), e = (b >> 23) & 0xFFu;
  if (e == 0) return fv(b & 0x80000000u);
  if (e == 255) return (b & 0x7FFFFFu) ? fv(kQNaN) : a;
  int e2 = (int)e + n;
  if (e2 < 1) return fv(b & 0x80000000u);
  if (e2 > 254) return fv((b & 0x80000000u) | kPInf);
  return fv((b & 0x807FFFFFu) | ((uint32_t)e2 << 23));
}

// floor, saturated to int32, NaN -> 0 (llm/fp32.py:169-189, mode "floor")
T2R_DEV int floor_sat(float t) {
  if (t != t) return 0;
  float f = floorf(t);
  if (f >= 2147483648.0f) return 2147483647;
  if (f < -2147483648.0f) return (int)0x80000000;
  return (int)f;
}

// EXP (llm/sfu.py:7-11, 69-82)
T2R_DEV float sfu_exp(float xin) {
  const float x = ftz(xin);
  if (x != x) return fv(kQNaN);
  if (x >= 89.0f) return fv(kPInf);
  if (x <= -104.0f) return 0.0f;
  const float t = fmul_ftz(x, (float)1.4426950408889634);
  const int n = floor_sat(t);
  const float f = fadd_ftz(t, -(float)n);
  const float u = fmul_ftz(f, 64.0f);
  int i = floor_sat(u);
  i = i < 0 ? 0 : (i > 63 ? 63 : i);
  const float r = fadd_ftz(u, -(float)i);
  const float y = fadd_ftz(c_sfu[kSfuExpT + i], fmul_ftz(r, c_sfu[kSfuExpS + i]));
  return ldexp_ftz(y, n < -300 ? -300 : (n > 300 ? 300 : n));
}

// (frac & 0x1FFFF) / 2^17, exact
T2R_DEV float frac17(uint32_t frac) { return ldexp_ftz((float)(int)(frac & 0x1FFFFu), -17); }

// RECIP (llm/sfu.py:12-15, 85-96)
T2R_DEV float sfu_recip(float xin) {
  const uint32_t b = fb(ftz(xin));
  const uint32_t s = b & 0x80000000u, e = (b >> 23) & 0xFFu, frac = b & 0x7FFFFFu;
  if (e == 0) return fv(s | kPInf);
  if (e == 255) return frac ? fv(kQNaN) : fv(s);
  const int i = (int)(frac >> 17);
  const float m = fv(frac | 0x3F800000u);
  const float y0 = fadd_ftz(c_sfu[kSfuRecT + i], fmul_ftz(frac17(frac), c_sfu[kSfuRecS + i]));
  const float y1 = fmul_ftz(y0, fadd_ftz(2.0f, -fmul_ftz(m, y0)));
  return fv(fb(ldexp_ftz(y1, 127 - (int)e)) | s);
}

// RSQRT (llm/sfu.py:16-20, 99-114)
T2R_DEV float sfu_rsqrt(float xin) {
  const uint32_t b = fb(ftz(xin));
  const uint32_t s = b >> 31, e = (b >> 23) & 0xFFu, frac = b & 0x7FFFFFu;
  if (e == 255 && frac) return fv(kQNaN);
  if (e == 0) return fv(kPInf);
  if (s) return fv(kQNaN);
  if (e == 255) return 0.0f;
  const int E = (int)e - 127, odd = E & 1;
  const int j = odd * 64 + (int)(frac >> 17);
  const float m2 = fv(frac | ((uint32_t)(127 + odd) << 23));
  const float y0 = fadd_ftz(c_sfu[kSfuRsqT + j], fmul_ftz(frac17(frac), c_sfu[kSfuRsqS + j]));
  const float d = fadd_ftz(1.5f, -fmul_ftz(fmul_ftz(m2, fmul_ftz(y0, y0)), 0.5f));
  return ldexp_ftz(fmul_ftz(y0, d), -((E - odd) / 2));
}

// fp32 -> int8: round half to even, saturate to +-127, NaN -> 0 (llm/ref_model.py:136-139)
T2R_DEV int to_i8(float y) {
  if (y != y) return 0;
  float r = rintf(y);
  r = fminf(fmaxf(r, -127.0f), 127.0f);
  return (int)r;
}

// max that propagates NaN (NumPy's np.max)
T2R_DEV float nanmax(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  return a > b ? a : b;
}

// int32 accumulator -> fp32 (RNE), times the row scale, times the activation scale:
// y = F(F(f32(acc) * s_w) * s_x) (llm/ref_model.py:198-202)
T2R_DEV float dequant(int acc, float s_w, float s_x) {
  float y = (float)acc * s_w;
  return y * s_x;
}

// SiLU gate: F(F(h1 * recip(F(1 + exp(F(h1 * -1))))) * h3) (llm/ref_model.py:249-250)
T2R_DEV float silu_mul(float h1, float h3) {
  float sig = sfu_recip(1.0f + sfu_exp(h1 * -1.0f));
  float a = h1 * sig;
  return a * h3;
}

// 16 int8 products of a 128-bit weight chunk with a 128-bit activation chunk, accumulated
T2R_DEV int dot16(int4 w, int4 x, int acc) {
  acc = __builtin_amdgcn_sdot4(w.x, x.x, acc, false);
  acc = __builtin_amdgcn_sdot4(w.y, x.y, acc, false);
  acc = __builtin_amdgcn_sdot4(w.z, x.z, acc, false);
  acc = __builtin_amdgcn_sdot4(w.w, x.w, acc, false);
  return acc;
}

typedef int v4i_t __attribute__((ext_vector_type(4)));

#ifndef T2R_NT_LOADS
#define T2R_NT_LOADS 1
#endif
// 16-byte streaming load (non-temporal hint: weights are read once per token)
T2R_DEV int4 load_nt16(const int8_t* p) {
#if T2R_NT_LOADS
  const v4i_t v = __builtin_nontemporal_load((const v4i_t*)p);
  return make_int4(v.x, v.y, v.z, v.w);
#else
  return *(const int4*)p;
#endif
}

T2R_DEV int pack_i8x4(int a, int b, int c, int d) {
  return (a & 0xFF) | ((b & 0xFF) << 8) | ((c & 0xFF) << 16) | ((int)((unsigned)d << 24));
}

// ------------------------------------------------------------------ block-level helpers
// Wave-wide reductions over 64 lanes. Integer sums and maxima are order-free, so any tree works.
T2R_DEV int wave_sum_i32(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
T2R_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = nanmax(v, __shfl_xor(v, o));
  return v;
}

// max over the block (NaN-propagating); every thread gets the result. `red` holds >= 16 floats.
T2R_DEV float block_max(float v, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
  v = wave_max(v);
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float m = red[0];
  for (int i = 1; i < nw; ++i) m = nanmax(m, red[i]);
  return m;
}

// The device's ordered sum of vals[0..n) (llm/ref_model.py:179-186): +0 padding to a multiple
// of D, lane l adds vals[l], vals[D + l], vals[2D + l], ... in order, then lanes pair up
// (0+1, 2+3, ...) until one value is left. Run by the D lanes [lane0, lane0 + D) of one wave,
// vals readable by them (LDS); returns the sum on every one of those lanes. `sq`: sum the
// squares F(v * v) instead (RMSNorm).
template <bool SQ>
T2R_DEV float ordered_sum(const float* vals, int n, int D, int l) {
  float acc = 0.0f;
  const int groups = n > 0 ? (n + D - 1) / D : 1;
  int g = 0;
  // 8 groups at a time: the loads are independent, the adds stay one chain in group order
  for (; g + 8 <= groups; g += 8) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = (g + j) * D + l;
      v[j] = i < n ? vals[i] : 0.0f;
      if (SQ) v[j] = v[j] * v[j];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) acc = (g + j == 0) ? v[j] : acc + v[j];
  }
  for (; g < groups; ++g) {
    const int i = g * D + l;
    float v = i < n ? vals[i] : 0.0f;
    if (SQ) v = v * v;
    acc = g == 0 ? v : acc + v;
  }
  // pairwise tree over the D lanes: lane l (a multiple of 2s) takes lane l + s
  for (int s = 1; s < D; s <<= 1) {
    float o = __shfl_down(acc, s, D);
    if ((l & (2 * s - 1)) == 0) acc = acc + o;
  }
  return __shfl(acc, 0, D);
}

// The same ordered sum over a buffer in the "lane-major" layout: value i (lane i % D, group i / D)
// is at osum_index(i) = (i % D) * P + i / D, with P = osum_stride(n, D) >= the group count, a
// multiple of 4 (16-byte aligned runs). Lane l's chain is then contiguous: its values are read
// 16 at a time with 128-bit loads, so the loads stay off the chain of adds. The writer stores +0
// at the padding positions i in [n, groups * D).
__host__ __device__ inline int osum_stride(int n, int D) {
  const int G = n > 0 ? (n + D - 1) / D : 1;
  return ((G + 3) & ~3) + 4;
}
__host__ __device__ inline int osum_index(int i, int D, int P) { return (i & (D - 1)) * P + i / D; }

template <bool SQ>
T2R_DEV float ordered_sum_t(const float* buf, int n, int D, int P, int l) {
  const int G = n > 0 ? (n + D - 1) / D : 1;
  const float* row = buf + l * P;
  float acc = 0.0f;
  int g = 0;
  for (; g + 16 <= G; g += 16) {
    const float4 a = *(const float4*)(row + g), b = *(const float4*)(row + g + 4);
    const float4 c = *(const float4*)(row + g + 8), d = *(const float4*)(row + g + 12);
    float v[16] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, c.x, c.y, c.z, c.w, d.x, d.y, d.z, d.w};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      if (SQ) v[j] = v[j] * v[j];
      acc = (g + j == 0) ? v[j] : acc + v[j];
    }
  }
  for (; g < G; ++g) {
    float v = row[g];
    if (SQ) v = v * v;
    acc = g == 0 ? v : acc + v;
  }
  for (int s = 1; s < D; s <<= 1) {
    float o = __shfl_down(acc, s, D);
    if ((l & (2 * s - 1)) == 0) acc = acc + o;
  }
  return __shfl(acc, 0, D);
}

}  // namespace t2r
