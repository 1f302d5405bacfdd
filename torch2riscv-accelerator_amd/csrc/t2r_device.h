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

// Native vector types for values that are loaded and stored whole (HIP's int4 / float4 are
// structs; arrays of them copied as aggregates can end up in scratch memory).
typedef int v2i_t __attribute__((ext_vector_type(2)));
typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef float v4f_t __attribute__((ext_vector_type(4)));
typedef int v16i_t __attribute__((ext_vector_type(16)));   // int8 MFMA 32 x 32 accumulators

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

// s_waitcnt with vmcnt(v) only (expcnt / lgkmcnt at their maxima): gfx9 encoding
constexpr int waitcnt_vm(int v) { return (v & 15) | ((v >> 4) << 14) | 0x0F70; }

constexpr uint32_t kQNaN = 0x7FC00000u;
constexpr uint32_t kPInf = 0x7F800000u;
constexpr float kInv127 = (float)(1.0 / 127.0);      // F(1/127): double quotient rounded once

// SFU tables in constant memory: [exp T | exp S | recip T | recip S | rsqrt T(128) | rsqrt S(128)].
// Kernels whose SFU calls sit on a latency chain copy them into LDS at start (sfu_stage) and pass
// the LDS copy: a lookup is then an LDS read instead of a dependent global load.
constexpr int kSfuExpT = 0, kSfuExpS = 64, kSfuRecT = 128, kSfuRecS = 192, kSfuRsqT = 256, kSfuRsqS = 384;
constexpr int kSfuWords = 512;
extern __constant__ float c_sfu[kSfuWords];

// The first kSfuWords / 4 threads of a block store 4 table words each (fetched into a register with
// the block's first loads), before a barrier that precedes the first lookup.
T2R_DEV void sfu_store(float* lds, v4f_t v) {
  const int t = threadIdx.x;
  if (t < kSfuWords / 4) ((v4f_t*)lds)[t] = v;
}

T2R_DEV uint32_t fb(float x) { return __float_as_uint(x); }
T2R_DEV float fv(uint32_t b) { return __uint_as_float(b); }

// A copy of x in a vector register that the compiler cannot prove wave-uniform: the SFU sequences
// below are straight-line selects, and on a value known to be uniform the compiler would turn them
// back into scalar branches, each a VALU -> SALU round trip.
T2R_DEV float vreg(float x) {
  float r;
  asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "v"(x));
  return r;
}

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
  const float r = a * b;
  const uint32_t rb = fb(r), m = rb & 0x7FFFFFFFu;
  const float r2 = (a * 0x1p64f) * (b * 0x1p64f);     // only looked at when |r| == 2^-126
  const bool zero = m < 0x00800000u || (m == 0x00800000u && fabsf(r2) < 4.0f);
  return zero ? fv(rb & 0x80000000u) : r;
}

// a * 2^n as an exponent-field add (llm/fp32.py:147-151): below the normal range a signed
// zero, above it a signed inf; zero and inf pass through, NaN gives the canonical NaN.
// (Straight-line selects, lowest precedence first: the SFU sequences run on latency chains.)
T2R_DEV float ldexp_ftz(float a, int n) {
  const uint32_t b = fb(a), e = (b >> 23) & 0xFFu, sg = b & 0x80000000u;
  const int e2 = (int)e + n;
  uint32_t r = (b & 0x807FFFFFu) | ((uint32_t)e2 << 23);
  r = e2 < 1 ? sg : r;
  r = e2 > 254 ? (sg | kPInf) : r;
  r = e == 0 ? sg : r;
  r = e == 255 ? ((b & 0x7FFFFFu) ? kQNaN : b) : r;
  return fv(r);
}

// floor, saturated to int32, NaN -> 0 (llm/fp32.py:169-189, mode "floor")
T2R_DEV int floor_sat(float t) {
  const float f = floorf(t);
  int r = (int)fminf(fmaxf(f, -2147483648.0f), 2147483520.0f);   // in range: defined conversion
  r = f >= 2147483648.0f ? 2147483647 : r;
  return t != t ? 0 : r;
}

// The three SFU functions below follow the reference's operation sequence. They use plain IEEE
// operations where the FTZ rule cannot change a result, and the FTZ helpers where it can. The
// rule only differs from IEEE on a result below 2^-126 (or, for a product, exactly 2^-126).
// After the input is flushed, every intermediate of these sequences is zero or at least 2^-126
// in magnitude:
//  - the table terms are in [2^-9, 2);
//  - a fraction times a slope is at least 2^-17 * 2^-9 for RECIP / RSQRT;
//  - EXP's slope term can be smaller, but it is then added to T >= 1 and vanishes either way.
// So only the final scaling by a power of two (ldexp_norm) can leave the normal range, and that
// step keeps the rule. Special inputs are selected at the end, never branched on.

// y * 2^n for a normal y, with the FTZ rule on the result
T2R_DEV float ldexp_norm(float y, int n) {
  const uint32_t b = fb(y), sg = b & 0x80000000u;
  const int e2 = (int)((b >> 23) & 0xFFu) + n;
  uint32_t r = (b & 0x807FFFFFu) | ((uint32_t)e2 << 23);
  r = e2 < 1 ? sg : r;
  return fv(e2 > 254 ? (sg | kPInf) : r);
}

// (frac & 0x1FFFF) / 2^17, exact
T2R_DEV float frac17(uint32_t frac) { return (float)(int)(frac & 0x1FFFFu) * 0x1p-17f; }

// EXP (llm/sfu.py:7-11, 69-82): the reference's steps, less what the input range makes redundant
// (the GPU self-check compares this form with the literal sequence over all 2^32 inputs):
//  - t = x log2(e) is clamped to [-160, 160] (NaN -> -160): every conversion stays defined, and no
//    result changes, since n = floor(t) then underflows (or overflows) the result's exponent on
//    exactly the inputs where the reference selects 0 (x <= -104) or +inf (x >= 89);
//  - u = 64 (t - floor(t)) lies in [0, 64] (64 where the difference rounds up to 1, for t just
//    below an integer), so the table index is min(trunc(u), 63);
//  - y = T + r S lies in [1, 2] (T = 2^(i/64), S > 0): no sign bit, and the result's exponent field
//    is y's plus n, 0 below 1 and +inf above 254.
T2R_DEV float sfu_exp(float xin, const float* tab = c_sfu) {
  const float x = ftz(vreg(xin));
  const float tc = fminf(fmaxf(x * (float)1.4426950408889634, -160.0f), 160.0f);
  const float tf = floorf(tc);
  const float u = (tc - tf) * 64.0f;
  const int i = min((int)u, 63);
  const float r = u - (float)i;
  const uint32_t b = fb(tab[kSfuExpT + i] + r * tab[kSfuExpS + i]);
  const int e2 = (int)(b >> 23) + (int)tf;
  uint32_t o = (b & 0x7FFFFFu) | ((uint32_t)e2 << 23);
  o = e2 < 1 ? 0u : o;
  o = e2 > 254 ? kPInf : o;
  return x != x ? fv(kQNaN) : fv(o);
}

// EXP of a softmax argument s - max: x <= 0, or NaN (a NaN score or maximum, or both infinite).
// Equal to sfu_exp on that domain (the GPU self-check compares it with the literal sequence over
// every such input); for x > 0 it returns EXP(0). Beyond sfu_exp's reductions:
//  - the entry flush is a select: x in (-2^-126, 0] gives 0, whose EXP is that of -0;
//  - only the lower clamp of t remains (t <= 0);
//  - n <= 0 and y in [1, 2]: n is added to y's bits as n 2^23; the sum never overflows, and the
//    result underflows (to +0) exactly where that integer is below 2^23 (as a signed value).
T2R_DEV float sfu_exp_np(float xin, const float* tab = c_sfu) {
  const float xr = vreg(xin);
  const float x = xr > -0x1p-126f ? 0.0f : xr;
  const float tc = fmaxf(x * (float)1.4426950408889634, -160.0f);
  const float tf = floorf(tc);
  const float u = (tc - tf) * 64.0f;
  const int i = min((int)u, 63);
  const float r = u - (float)i;
  const uint32_t b = fb(tab[kSfuExpT + i] + r * tab[kSfuExpS + i]);
  const int e = (int)(b + ((uint32_t)(int)tf << 23));
  const float out = e < 0x00800000 ? 0.0f : fv((uint32_t)e);
  return x != x ? fv(kQNaN) : out;
}

// The EXP table as 65 {T, S} pairs: entries 0..63 the table's, entry 64 {F(T[63] + S[63]), 0}.
constexpr int kSfuExpPairs = 65;
T2R_DEV float2 sfu_exp_pair(int i, const float* tab) {
  const int j = min(i, 63);                      // (both reads unconditional: no branch around a load)
  const float t = tab[kSfuExpT + j], s = tab[kSfuExpS + j];
  return i < 64 ? make_float2(t, s) : make_float2(t + s, 0.0f);
}

// EXP of a softmax argument x = s - max under a finite maximum: x <= 0 or -inf, never NaN. Equal to
// sfu_exp_np there (the GPU self-check compares it with the literal sequence over that whole domain)
// with fewer steps, given the table's F(T[63] + S[63]) = 2 and T[0] = 1 (checked by the library's
// init):
//  - i = trunc(u) and r = fract(u), both exact for u in [0, 64]: below 64 they are the reference's
//    index and remainder; at u = 64 the reference takes i = 63, r = 1, whose F(T[63] + 1 S[63]) is
//    pair 64's T (and 0 S[64] = 0);
//  - no entry flush: x in (-2^-126, 0) gives t in (-2^-125, 0), floor -1, F(t + 1) = 1, u = 64, y = 2,
//    and 2 2^-1 = 1 = T[0], the EXP of the flushed zero;
//  - no NaN select (x is never NaN);
//  - t clamped at -127 (not -160) and the power of two applied as a product, y F(2^n): with n >= -126
//    F(2^n) is normal and y 2^n (y in [1, 2]) exact and normal, the reference's result; n = -127 (t in
//    [-127, -126), and every t below, clamped to -127) gives F(2^n)'s bits 0, so y 0 = +0, the
//    reference's underflow there (its y < 2: u = 64 (t + 127) is exact, at most 64 - 2^-11, and
//    F(T[63] + F(r S[63])) stays below 2 for r <= 1 - 2^-11).
T2R_DEV float sfu_exp_sm(float x, const float2* et) {
  const float tc = fmaxf(x * (float)1.4426950408889634, -127.0f);
  const float tf = floorf(tc);
  const float u = (tc - tf) * 64.0f;
  const float2 ts = et[(int)u];
  const float y = ts.x + __builtin_amdgcn_fractf(u) * ts.y;
  return y * fv(((uint32_t)(int)tf << 23) + 0x3F800000u);
}

// RECIP (llm/sfu.py:12-15, 85-96)
// (the table pair {T[i], S[i]} from pair(i): sfu_recip's, or one that lanes hold in registers)
template <class P>
T2R_DEV float sfu_recip_by(float xin, P pair) {
  const uint32_t b = fb(ftz(vreg(xin)));
  const uint32_t s = b & 0x80000000u, e = (b >> 23) & 0xFFu, frac = b & 0x7FFFFFu;
  const int i = (int)(frac >> 17);
  const float m = fv(frac | 0x3F800000u);
  const float2 ts = pair(i);
  const float y0 = ts.x + frac17(frac) * ts.y;
  const float y1 = y0 * (2.0f - m * y0);
  uint32_t r = fb(ldexp_norm(y1, 127 - (int)e)) | s;
  r = e == 255 ? (frac ? kQNaN : s) : r;
  r = e == 0 ? (s | kPInf) : r;
  return fv(r);
}
T2R_DEV float sfu_recip(float xin, const float* tab = c_sfu) {
  return sfu_recip_by(xin, [tab](int i) { return make_float2(tab[kSfuRecT + i], tab[kSfuRecS + i]); });
}

// RECIP of a gate denominator F(1 + EXP(.)): x >= 1, +inf or NaN. Equal to sfu_recip on that domain
// (the GPU self-check compares it with the literal sequence over every such input). No flush, no
// sign, no zero; y1 lies in (0.5, 1], so (127 - e) is added to its bits as (127 - e) 2^23, and the
// result underflows to +0 exactly where that integer is below 2^23 (as a signed value) -- which also
// gives RECIP(+inf) = +0.
T2R_DEV float sfu_recip_ge1(float xin, const float* tab = c_sfu) {
  const float x = vreg(xin);
  const uint32_t b = fb(x), frac = b & 0x7FFFFFu;
  const int i = (int)(frac >> 17);
  const float m = fv(frac | 0x3F800000u);
  const float y0 = tab[kSfuRecT + i] + frac17(frac) * tab[kSfuRecS + i];
  const float y1 = y0 * (2.0f - m * y0);
  const int r = (int)(fb(y1) + ((uint32_t)(127 - (int)(b >> 23)) << 23));
  return x != x ? fv(kQNaN) : (r < 0x00800000 ? 0.0f : fv((uint32_t)r));
}

// RSQRT (llm/sfu.py:16-20, 99-114)
T2R_DEV float sfu_rsqrt(float xin, const float* tab = c_sfu) {
  const uint32_t b = fb(ftz(vreg(xin)));
  const uint32_t s = b >> 31, e = (b >> 23) & 0xFFu, frac = b & 0x7FFFFFu;
  const int E = (int)e - 127, odd = E & 1;
  const int j = odd * 64 + (int)(frac >> 17);
  const float m2 = fv(frac | ((uint32_t)(127 + odd) << 23));
  const float y0 = tab[kSfuRsqT + j] + frac17(frac) * tab[kSfuRsqS + j];
  const float d = 1.5f - (m2 * (y0 * y0)) * 0.5f;
  float r = ldexp_norm(y0 * d, -((E - odd) / 2));
  r = e == 255 ? 0.0f : r;
  r = s ? fv(kQNaN) : r;
  r = e == 0 ? fv(kPInf) : r;
  return (e == 255 && frac) ? fv(kQNaN) : r;
}

// The same three functions as the reference's literal sequence, the FTZ rule applied after every
// operation. Not used on the datapath: t2r_sfu_check compares the functions above with these on
// every one of the 2^32 inputs.
namespace seq {
T2R_DEV float frac17(uint32_t frac) { return ldexp_ftz((float)(int)(frac & 0x1FFFFu), -17); }
T2R_DEV float sfu_exp(float xin, const float* tab) {
  const float x = ftz(xin);
  const float t = fmul_ftz(x, (float)1.4426950408889634);
  const int n = floor_sat(t);
  const float f = fadd_ftz(t, -(float)n);
  const float u = fmul_ftz(f, 64.0f);
  const int i = min(max(floor_sat(u), 0), 63);
  const float r = fadd_ftz(u, -(float)i);
  const float y = fadd_ftz(tab[kSfuExpT + i], fmul_ftz(r, tab[kSfuExpS + i]));
  float out = ldexp_ftz(y, min(max(n, -300), 300));
  out = x <= -104.0f ? 0.0f : out;
  out = x >= 89.0f ? fv(kPInf) : out;
  return x != x ? fv(kQNaN) : out;
}
T2R_DEV float sfu_recip(float xin, const float* tab) {
  const uint32_t b = fb(ftz(xin));
  const uint32_t s = b & 0x80000000u, e = (b >> 23) & 0xFFu, frac = b & 0x7FFFFFu;
  if (e == 0) return fv(s | kPInf);
  if (e == 255) return frac ? fv(kQNaN) : fv(s);
  const int i = (int)(frac >> 17);
  const float m = fv(frac | 0x3F800000u);
  const float y0 = fadd_ftz(tab[kSfuRecT + i], fmul_ftz(frac17(frac), tab[kSfuRecS + i]));
  const float y1 = fmul_ftz(y0, fadd_ftz(2.0f, -fmul_ftz(m, y0)));
  return fv(fb(ldexp_ftz(y1, 127 - (int)e)) | s);
}
T2R_DEV float sfu_rsqrt(float xin, const float* tab) {
  const uint32_t b = fb(ftz(xin));
  const uint32_t s = b >> 31, e = (b >> 23) & 0xFFu, frac = b & 0x7FFFFFu;
  if (e == 255 && frac) return fv(kQNaN);
  if (e == 0) return fv(kPInf);
  if (s) return fv(kQNaN);
  if (e == 255) return 0.0f;
  const int E = (int)e - 127, odd = E & 1;
  const int j = odd * 64 + (int)(frac >> 17);
  const float m2 = fv(frac | ((uint32_t)(127 + odd) << 23));
  const float y0 = fadd_ftz(tab[kSfuRsqT + j], fmul_ftz(frac17(frac), tab[kSfuRsqS + j]));
  const float d = fadd_ftz(1.5f, -fmul_ftz(fmul_ftz(m2, fmul_ftz(y0, y0)), 0.5f));
  return ldexp_ftz(fmul_ftz(y0, d), -((E - odd) / 2));
}
}  // namespace seq

// fp32 -> int8: round half to even, saturate to +-127, NaN -> 0 (llm/ref_model.py:136-139)
T2R_DEV int to_i8(float y) {
  if (y != y) return 0;
  float r = rintf(y);
  r = fminf(fmaxf(r, -127.0f), 127.0f);
  return (int)r;
}

// max that propagates NaN (NumPy's np.max); selects only (early returns become exec-mask branches)
T2R_DEV float nanmax(float a, float b) {
  float r = a > b ? a : b;
  r = b != b ? b : r;
  return a != a ? a : r;
}
// The maximum with NaN winning, in one instruction (gfx950 v_maximum3_f32, IEEE 754-2019 maximum).
// It can differ from nanmax only in which NaN it returns and in the sign of a zero maximum (-0 < +0
// here); a softmax's EXP(s - max) sees neither (any NaN x gives the quiet NaN, s - (+-0) = s for
// s != 0, and +-0 - +-0 is a zero, whose EXP is that of 0).
T2R_DEV float smax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Bits of |x| for an order-free maximum of magnitudes: for values >= 0 the unsigned order of the
// bits is the numeric order, and every NaN (any payload, sign cleared) is above +inf, so the
// integer maximum propagates NaN as np.max does.
T2R_DEV uint32_t abs_bits(float x) { return fb(x) & 0x7FFFFFFFu; }


// int32 accumulator -> fp32 (RNE), times the row scale, times the activation scale:
// y = F(F(f32(acc) * s_w) * s_x) (llm/ref_model.py:198-202)
T2R_DEV float dequant(int acc, float s_w, float s_x) {
  float y = (float)acc * s_w;
  return y * s_x;
}

// SiLU gate: F(F(h1 * recip(F(1 + exp(F(h1 * -1))))) * h3) (llm/ref_model.py:249-250)
T2R_DEV float silu_mul(float h1, float h3, const float* tab = c_sfu) {
  float sig = sfu_recip_ge1(1.0f + sfu_exp(h1 * -1.0f, tab), tab);
  float a = h1 * sig;
  return a * h3;
}

// The gates' EXP and RECIP from {T, S} pair tables in LDS (one 8-byte read per lookup), for
// arguments that are not NaN; a NaN gate input makes the product NaN whatever these return (h1 * s
// with h1 NaN), so they need no NaN select.
// EXP of any non-NaN x, equal to sfu_exp there (the GPU self-check compares it with the literal
// sequence over every such input), with the 65-pair table of sfu_exp_sm:
//  - t is clamped to [-160, 128]: at 128 (x >= 88.7) the integer step below gives exactly the bits
//    of +inf (y = 1), the reference's result for every t >= 128, and no sum carries past them (for
//    t < 128, y <= 2 and n <= 127);
//  - i = trunc(u) and r = fract(u) are exact for u in [0, 64] (u = 64 takes pair 64, as in
//    sfu_exp_sm); a subnormal x needs no flush (its t is below 2^-25 in magnitude: y = 1 for x > 0,
//    and u = 64, y = 2, n = -1 for x < 0: EXP(0) = 1 either way);
//  - n is added to y's bits as n 2^23 and the result is +0 below 2^-126.
T2R_DEV float sfu_exp_g(float x, const float2* ep) {
  const float tc = fminf(fmaxf(x * (float)1.4426950408889634, -160.0f), 128.0f);
  const float tf = floorf(tc);
  const float u = (tc - tf) * 64.0f;
  const float2 ts = ep[(int)u];
  const uint32_t b = fb(ts.x + __builtin_amdgcn_fractf(u) * ts.y);
  const int e = (int)(b + ((uint32_t)(int)tf << 23));
  return e < 0x00800000 ? 0.0f : fv((uint32_t)e);
}

// RECIP of a gate denominator x >= 1 or +inf (not NaN), equal to sfu_recip_ge1 there (self-checked
// the same way), with a 64-pair {T, S} table: frac / 2^17 is fract(64 m) for the mantissa m in [1, 2)
// (exact: 64 m has 17 fraction bits), and (127 - e) 2^23 is 127 2^23 minus x's exponent field.
T2R_DEV float2 sfu_recip_pair(int i, const float* tab) { return make_float2(tab[kSfuRecT + i], tab[kSfuRecS + i]); }
T2R_DEV float sfu_recip_g1(float x, const float2* rp) {
  const uint32_t b = fb(x);
  const float m = fv((b & 0x7FFFFFu) | 0x3F800000u);
  const float2 ts = rp[(b >> 17) & 63u];
  const float y0 = ts.x + __builtin_amdgcn_fractf(m * 64.0f) * ts.y;
  const float y1 = y0 * (2.0f - m * y0);
  const int r = (int)(fb(y1) + 0x3F800000u - (b & 0x7F800000u));
  return r < 0x00800000 ? 0.0f : fv((uint32_t)r);
}

// silu_mul and gelu_mul (below) with those two forms: the same products for every input
T2R_DEV float silu_mul_p(float h1, float h3, const float2* ep, const float2* rp) {
  const float sig = sfu_recip_g1(1.0f + sfu_exp_g(h1 * -1.0f, ep), rp);
  const float a = h1 * sig;
  return a * h3;
}

// GELU-tanh gate (GeGLU; compiler/frontend/hf_generic.py:840-852): GELU's tanh approximation from EXP
// and RECIP, x * 0.5 (1 + tanh(u)) = x * RECIP(F(EXP(z) + 1)) with z = F(x * F(A + F(F(x * x) * B))),
// A = f32(-2 sqrt(2 / pi)), B = f32(-2 sqrt(2 / pi) 0.044715); then F(gelu * h3). Large negative x:
// EXP gives +inf, RECIP 0, the product a signed zero.
constexpr float kGeluA = -1.5957692f;     // the float32 values (shortest round-trip decimals)
constexpr float kGeluB = -0.071354814f;
T2R_DEV float gelu_mul(float h1, float h3, const float* tab = c_sfu) {
  const float z = h1 * (kGeluA + (h1 * h1) * kGeluB);
  const float a = h1 * sfu_recip_ge1(sfu_exp(z, tab) + 1.0f, tab);
  return a * h3;
}

// the FFN gate: act 0 SiLU (SwiGLU), 1 GELU-tanh (GeGLU); act is uniform over the launch
T2R_DEV float gate_mul(float h1, float h3, int act, const float* tab = c_sfu) {
  return act ? gelu_mul(h1, h3, tab) : silu_mul(h1, h3, tab);
}
T2R_DEV float gelu_mul_p(float h1, float h3, const float2* ep, const float2* rp) {
  const float z = h1 * (kGeluA + (h1 * h1) * kGeluB);
  const float a = h1 * sfu_recip_g1(sfu_exp_g(z, ep) + 1.0f, rp);
  return a * h3;
}
// the gate from the pair tables (LDS): ep 65 EXP pairs (sfu_exp_pair), rp 64 RECIP pairs
T2R_DEV float gate_mul_p(float h1, float h3, int act, const float2* ep, const float2* rp) {
  return act ? gelu_mul_p(h1, h3, ep, rp) : silu_mul_p(h1, h3, ep, rp);
}

// 16 int8 products of a 128-bit weight chunk with a 128-bit activation chunk, accumulated
T2R_DEV int dot16(int4 w, int4 x, int acc) {
  acc = __builtin_amdgcn_sdot4(w.x, x.x, acc, false);
  acc = __builtin_amdgcn_sdot4(w.y, x.y, acc, false);
  acc = __builtin_amdgcn_sdot4(w.z, x.z, acc, false);
  acc = __builtin_amdgcn_sdot4(w.w, x.w, acc, false);
  return acc;
}


// 16-byte streaming load (non-temporal hint: weights are read once per token)
T2R_DEV int4 load_nt16(const int8_t* p) {
  const v4i_t v = __builtin_nontemporal_load((const v4i_t*)p);
  return make_int4(v.x, v.y, v.z, v.w);
}

T2R_DEV int pack_i8x4(int a, int b, int c, int d) {
  return (a & 0xFF) | ((b & 0xFF) << 8) | ((c & 0xFF) << 16) | ((int)((unsigned)d << 24));
}

// ------------------------------------------------------------------ block-level helpers
// Wave-wide reductions over 64 lanes. Integer sums and maxima are order-free, so any tree works.
// DPP moves within 16-lane rows (no LDS round trip): xor 1 and xor 2 (quad permutes), then the
// half-row and row mirrors pair groups that already agree, so after the four steps every lane
// holds its row's result; the four rows are combined from lanes 0, 16, 32, 48.
template <int CTRL>
T2R_DEV int dpp_i(int v) { return __builtin_amdgcn_update_dpp(v, v, CTRL, 0xF, 0xF, false); }
template <int CTRL>
T2R_DEV float dpp_f(float v) { return __int_as_float(dpp_i<CTRL>(__float_as_int(v))); }
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;
// the same move for controls whose source lane is always inside the 16-lane row (quad permutes,
// mirrors): no old value to keep, so no copy of the source first
template <int CTRL>
T2R_DEV int dpp_mov_i(int v) { return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false); }

// every lane returns the sum over the wave (all 64 lanes active)
T2R_DEV int wave_sum_i32(int v) {
  v += dpp_i<kDppXor1>(v);
  v += dpp_i<kDppXor2>(v);
  v += dpp_i<kDppHalfMirror>(v);
  v += dpp_i<kDppMirror>(v);
  return (__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
         (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48));
}
// The wave sums of NV values at once (NV = 1, 2, 4 or 8; exact int32 in any order). Halving steps
// first: each sends half of the lane's values to its partner (lane bit 2, then 1, then 0) and keeps
// the other half, adding what the partner sent; then single-value steps over the remaining lane
// bits (row_ror:8 for bit 3, the gfx950 permlane swaps for bits 4 and 5, each swap of a register
// with itself leaving v(L) and v(L ^ 16) or v(L ^ 32) in the pair it returns). Lane L ends with the
// total of value (L >> (3 - log2 NV)) & (NV - 1).
template <int M, int CTRL>
T2R_DEV void wave_halve(int* c, int hi) {
#pragma unroll
  for (int j = 0; j < M / 2; ++j) {
    const int send = hi ? c[j] : c[j + M / 2];
    const int keep = hi ? c[j + M / 2] : c[j];
    c[j] = keep + dpp_i<CTRL>(send);
  }
}
template <int NV>
T2R_DEV int wave_sum_multi(const int (&v)[NV]) {
  static_assert(NV == 1 || NV == 2 || NV == 4 || NV == 8, "1, 2, 4 or 8 values");
  const int lane = threadIdx.x & 63;
  int c[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) c[j] = v[j];
  if constexpr (NV >= 2) wave_halve<NV, kDppHalfMirror>(c, (lane >> 2) & 1);   // partner lane ^ 7
  if constexpr (NV >= 4) wave_halve<NV / 2, kDppXor2>(c, (lane >> 1) & 1);
  if constexpr (NV >= 8) wave_halve<NV / 4, kDppXor1>(c, lane & 1);
  int t = c[0];
  if constexpr (NV < 8) t += dpp_i<kDppXor1>(t);
  if constexpr (NV < 4) t += dpp_i<kDppXor2>(t);
  if constexpr (NV < 2) t += dpp_i<kDppHalfMirror>(t);
  t += dpp_i<0x128>(t);                                                     // row_ror:8 = lane ^ 8
  {
    const auto r = __builtin_amdgcn_permlane16_swap((unsigned)t, (unsigned)t, false, false);
    t = (int)(r[0] + r[1]);
  }
  {
    const auto r = __builtin_amdgcn_permlane32_swap((unsigned)t, (unsigned)t, false, false);
    t = (int)(r[0] + r[1]);
  }
  return t;
}

// A workgroup barrier that orders LDS only: this wave's LDS accesses complete, then s_barrier. Unlike
// __syncthreads it leaves the wave's global loads in flight (no wait on their counter).
T2R_DEV void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);            // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// every lane returns the sum over its half-wave (lanes 0-31 or 32-63)
T2R_DEV int wave_half_sum_i32(int v) {
  v += dpp_i<kDppXor1>(v);
  v += dpp_i<kDppXor2>(v);
  v += dpp_i<kDppHalfMirror>(v);
  v += dpp_i<kDppMirror>(v);
  return v + __shfl_xor(v, 16);
}
// wave_max with smax: the maximum of the wave's 64 values, NaN winning, to every lane
T2R_DEV float wave_smax(float v) {
  v = smax(v, dpp_f<kDppXor1>(v));
  v = smax(v, dpp_f<kDppXor2>(v));
  v = smax(v, dpp_f<kDppHalfMirror>(v));
  v = smax(v, dpp_f<kDppMirror>(v));
  const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return smax(smax(a, b), smax(c, d));
}

T2R_DEV float wave_max(float v) {
  v = nanmax(v, dpp_f<kDppXor1>(v));
  v = nanmax(v, dpp_f<kDppXor2>(v));
  v = nanmax(v, dpp_f<kDppHalfMirror>(v));
  v = nanmax(v, dpp_f<kDppMirror>(v));
  const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return nanmax(nanmax(a, b), nanmax(c, d));
}

// The pairwise tree of the ordered sum over lanes [0, D) of a row (D <= 16 a power of two):
// lane l, l % 2s == 0, adds lane l + s; returns lane 0's total to every lane that calls it.
// lane_tree_sum's pairwise steps without the broadcast: the sum of lanes [r, r + D) ends in lane r of
// every 16-lane row r (D <= 16), so two half waves can sum two vectors at once (lanes 0 and 32)
T2R_DEV float lane_tree_rows(float acc, int D, int l) {
  float o = dpp_f<0x101>(acc);                                  // row_shl:1
  if (D > 1 && (l & 1) == 0) acc = acc + o;
  o = dpp_f<0x102>(acc);
  if (D > 2 && (l & 3) == 0) acc = acc + o;
  o = dpp_f<0x104>(acc);
  if (D > 4 && (l & 7) == 0) acc = acc + o;
  o = dpp_f<0x108>(acc);
  if (D > 8 && (l & 15) == 0) acc = acc + o;
  return acc;
}
T2R_DEV float lane_tree_sum(float acc, int D, int l) {
  float o = dpp_f<0x101>(acc);                                  // row_shl:1
  if (D > 1 && (l & 1) == 0) acc = acc + o;
  o = dpp_f<0x102>(acc);
  if (D > 2 && (l & 3) == 0) acc = acc + o;
  o = dpp_f<0x104>(acc);
  if (D > 4 && (l & 7) == 0) acc = acc + o;
  o = dpp_f<0x108>(acc);
  if (D > 8 && (l & 15) == 0) acc = acc + o;
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), 0));
}

// maximum of abs_bits values over the wave / the block (order-free, so any tree works); every
// thread gets the result. `red` holds >= 16 words.
T2R_DEV uint32_t wave_max_u32(uint32_t v) {
  v = max(v, (uint32_t)dpp_mov_i<kDppXor1>((int)v));
  v = max(v, (uint32_t)dpp_mov_i<kDppXor2>((int)v));
  v = max(v, (uint32_t)dpp_mov_i<kDppHalfMirror>((int)v));
  v = max(v, (uint32_t)dpp_mov_i<kDppMirror>((int)v));
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0), b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32), d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return max(max(a, b), max(c, d));
}
// ... over each half wave (lanes 0-31, 32-63): a lane gets its half's maximum
T2R_DEV uint32_t half_max_u32(uint32_t v, int half) {
  v = max(v, (uint32_t)dpp_mov_i<kDppXor1>((int)v));
  v = max(v, (uint32_t)dpp_mov_i<kDppXor2>((int)v));
  v = max(v, (uint32_t)dpp_mov_i<kDppHalfMirror>((int)v));
  v = max(v, (uint32_t)dpp_mov_i<kDppMirror>((int)v));
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0), b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32), d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return half ? max(c, d) : max(a, b);
}
T2R_DEV float block_absmax(uint32_t v, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
  uint32_t* r = (uint32_t*)red;
  v = wave_max_u32(v);
  __syncthreads();
  if (lane == 0) r[wave] = v;
  __syncthreads();
  uint32_t m = r[0];
  for (int i = 1; i < nw; ++i) m = max(m, r[i]);
  return fv(m);
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
// (0+1, 2+3, ...) until one value is left. Run by lanes [0, D) of one wave, vals readable by them
// (LDS); returns the sum on every one of those lanes. `sq`: sum the squares F(v * v) instead
// (RMSNorm). A lane's chain starts from its first value (no +0 in front).
template <bool SQ>
T2R_DEV float ordered_sum(const float* vals, int n, int D, int l) {
  const int groups = n > 0 ? (n + D - 1) / D : 1;
  auto val = [&](int g) {
    const int i = g * D + l;
    float v = i < n ? vals[i] : 0.0f;
    return SQ ? v * v : v;
  };
  float acc = val(0);
  int g = 1;
  // 8 groups at a time: the loads are independent, the adds stay one chain in group order
  for (; g + 8 <= groups; g += 8) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = val(g + j);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc = acc + v[j];
  }
  for (; g < groups; ++g) acc = acc + val(g);
  return lane_tree_sum(acc, D, l);
}

// The same sum over a lane-major copy: value i is at osum_index(i) = (i % D) * P + i / D, with
// P = osum_stride(n, D) >= the group count, a multiple of 4 (16-byte aligned runs). Lane l's
// chain is then contiguous: its values are read 16 at a time with 128-bit loads, the next 16
// requested before the current 16 are added, so the loads stay off the chain of adds. The writer
// stores +0 at the padding positions i in [n, groups * D).
__host__ __device__ inline int osum_stride(int n, int D) {
  const int G = n > 0 ? (n + D - 1) / D : 1;
  return ((G + 3) & ~3) + 4;
}
__host__ __device__ inline int osum_index(int i, int D, int P) {
  return (i & (D - 1)) * P + (i >> __builtin_ctz((unsigned)D));   // D a power of two
}

template <bool SQ>
T2R_DEV float ordered_sum_t(const float* buf, int n, int D, int P, int l) {
  const int G = n > 0 ? (n + D - 1) / D : 1;
  const float* row = buf + l * P;
  float acc;
  int g;
  if (G >= 16) {
    float4 c0 = *(const float4*)(row), c1 = *(const float4*)(row + 4);
    float4 c2 = *(const float4*)(row + 8), c3 = *(const float4*)(row + 12);
    for (g = 0; g + 16 <= G; g += 16) {
      const bool more = g + 32 <= G;
      float4 n0 = c0, n1 = c1, n2 = c2, n3 = c3;
      if (more) {
        n0 = *(const float4*)(row + g + 16);
        n1 = *(const float4*)(row + g + 20);
        n2 = *(const float4*)(row + g + 24);
        n3 = *(const float4*)(row + g + 28);
      }
      float v[16] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w, c2.x, c2.y, c2.z, c2.w, c3.x, c3.y, c3.z, c3.w};
      if (SQ) {
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = v[j] * v[j];
      }
      if (g == 0) {
        acc = v[0];
#pragma unroll
        for (int j = 1; j < 16; ++j) acc = acc + v[j];
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) acc = acc + v[j];
      }
      c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    }
  } else {
    acc = SQ ? row[0] * row[0] : row[0];
    g = 1;
  }
  for (; g < G; ++g) {
    float v = row[g];
    if (SQ) v = v * v;
    acc = acc + v;
  }
  return lane_tree_sum(acc, D, l);
}

// ordered_sum_t for a lane whose chain is the only work of its wave: all 16-value batches of the
// chain requested at once (G <= 16 * NB, NB x 16 registers), then the adds in order.
template <bool SQ, int NB>
T2R_DEV float ordered_sum_t_all(const float* buf, int n, int D, int P, int l) {
  const int G = n > 0 ? (n + D - 1) / D : 1;
  if (G < 16 || G > 16 * NB) return ordered_sum_t<SQ>(buf, n, D, P, l);
  const float* row = buf + l * P;
  const int nb = G / 16;
  float4 c[NB][4];
#pragma unroll
  for (int b = 0; b < NB; ++b)
    if (b < nb)
#pragma unroll
      for (int q = 0; q < 4; ++q) c[b][q] = *(const float4*)(row + 16 * b + 4 * q);
  float acc = 0.0f;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if (b < nb) {
      float v[16] = {c[b][0].x, c[b][0].y, c[b][0].z, c[b][0].w, c[b][1].x, c[b][1].y, c[b][1].z, c[b][1].w,
                     c[b][2].x, c[b][2].y, c[b][2].z, c[b][2].w, c[b][3].x, c[b][3].y, c[b][3].z, c[b][3].w};
      if (SQ) {
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = v[j] * v[j];
      }
      acc = b == 0 ? v[0] : acc + v[0];
#pragma unroll
      for (int j = 1; j < 16; ++j) acc = acc + v[j];
    }
  }
  for (int g = 16 * nb; g < G; ++g) {
    float v = row[g];
    if (SQ) v = v * v;
    acc = acc + v;
  }
  return lane_tree_sum(acc, D, l);
}

}  // namespace t2r
