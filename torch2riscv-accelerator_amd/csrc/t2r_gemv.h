// W8A8 GEMV for decode: int8 weight rows streamed from HBM with 128-bit loads, int8 dot
// products (v_dot4) into exact int32 accumulators, wave reductions, and the dequantisation
// y = F(F(f32(acc) * s_w[n]) * s_x) fused with what surrounds the linear layer in the
// reference's op list (llm/compile_model.py:147-171, 295-331):
//
//  prologue  PRO_XQ          the int8 activations and their scale are given
//            PRO_QUANT       quant_act of an fp32 vector (llm/ref_model.py:191-196)
//            PRO_NORM_QUANT  RMSNorm then quant_act (llm/ref_model.py:204-207)
//  epilogue  EPI_STORE       y[n]
//            EPI_RESID       y[n] = F(res[n] + y)           (the residual add)
//            EPI_SWIGLU      two weight matrices W1, W3 with the same input:
//                            u[n] = F(F(h1 * sigmoid(h1)) * h3) (llm/ref_model.py:246-250)
//            + optional argmax: the first index of the largest output (greedy selection)
//
// Every workgroup recomputes the prologue on the whole input vector (at most 8192 values,
// a few microseconds of L2 reads), so no cross-workgroup communication is needed: the maximum
// |x| that quant_act needs is order-free and every workgroup gets the same bits. Weights are
// row-major (N, K), K contiguous; one wave covers 1024 bytes of a row per load step, each lane
// 16 bytes, and keeps its slice of the int8 activations in registers.
#pragma once
#include "t2r_device.h"

namespace t2r {

enum { PRO_XQ = 0, PRO_QUANT = 1, PRO_NORM_QUANT = 2 };
enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2 };
constexpr int kMaxK = 8192;
constexpr int kGemvThreads = 256;

struct GemvArgs {
  const int8_t* w;
  const float* s_w;          // [N, K], [N]
  const int8_t* w3;
  const float* s_w3;         // EPI_SWIGLU second matrix
  const float* x;            // PRO_QUANT / PRO_NORM_QUANT input rows (stride x_stride)
  const float* g;            // RMSNorm gain [K]
  const int8_t* xq;          // PRO_XQ input rows (stride xq_stride)
  const float* s_x;          // PRO_XQ scale per row
  float inv_n, eps;
  int D;
  int N, K;
  long long x_stride, xq_stride, y_stride, res_stride;
  float* y;                  // output rows (stride y_stride)
  const float* res;          // EPI_RESID residual rows (may alias y)
  int32_t* acc_out;          // optional int32 accumulators [rows, N] (SWIGLU: [rows, 2N])
  unsigned long long* argmax_key;  // optional: atomic max of (value, -index) per row
  int8_t* xq_out;            // optional: the quantised input (block 0 of each row writes it)
  float* sx_out;
  const int32_t* ids;        // optional row indirection (MoE experts): output row r reads weight row
  int rows_per_id;           //   ids[row * ids_stride + r / rows_per_id] * rows_per_id + r % rows_per_id
  int ids_stride;
};

T2R_DEV long long weight_row(const GemvArgs& a, int row_in, int row) {
  if (a.ids == nullptr) return row;
  const int j = row / a.rows_per_id;
  return (long long)a.ids[row_in * a.ids_stride + j] * a.rows_per_id + (row - j * a.rows_per_id);
}

// orderable 64-bit key of (value, index): larger value first, then the smaller index; NaN above
// everything (np.argmax returns the first NaN), -0 equal to +0
T2R_DEV unsigned long long argmax_key(float v, int idx) {
  uint32_t b = fb(v);
  if (v != v) {
    b = 0xFFFFFFFFu;
  } else {
    if ((b & 0x7FFFFFFFu) == 0) b = 0;
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  }
  return ((unsigned long long)b << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)idx);
}

// The prologue: fills xq_lds[0..K) with the int8 activations of row `row`, returns s_x.
// xf_lds: K floats of scratch.
template <int PRO>
T2R_DEV float gemv_prologue(const GemvArgs& a, int row, int8_t* xq_lds, float* xf_lds, float* red) {
  const int tid = threadIdx.x, K = a.K;
  if (PRO == PRO_XQ) {
    const int8_t* src = a.xq + row * a.xq_stride;
    for (int i = tid * 16; i < K; i += kGemvThreads * 16) *(int4*)(xq_lds + i) = *(const int4*)(src + i);
    __syncthreads();
    return a.s_x[row];
  }
  const float* x = a.x + row * a.x_stride;
  for (int i = tid; i < K; i += kGemvThreads) xf_lds[i] = x[i];
  __syncthreads();
  float r = 1.0f;
  if (PRO == PRO_NORM_QUANT) {
    if (tid < a.D) {
      float ss = ordered_sum<true>(xf_lds, K, a.D, tid);
      if (tid == 0) red[32] = sfu_rsqrt(ss * a.inv_n + a.eps);
    }
    __syncthreads();
    r = red[32];
  }
  float amax = 0.0f;
  for (int i = tid; i < K; i += kGemvThreads) {
    float v = xf_lds[i];
    if (PRO == PRO_NORM_QUANT) {
      v = (v * r) * a.g[i];
      xf_lds[i] = v;
    }
    amax = nanmax(amax, fabsf(v));
  }
  amax = block_max(amax, red);
  const float s_x = amax * kInv127;
  const float inv = sfu_recip(s_x);
  for (int i = tid; i < K; i += kGemvThreads) xq_lds[i] = (int8_t)to_i8(xf_lds[i] * inv);
  __syncthreads();
  return s_x;
}

// NCB: 1024-byte column chunks per row covered by the register slice (K <= NCB * 1024);
// RU: rows per wave iteration.
template <int PRO, int EPI, int NCB, int RU>
__global__ __launch_bounds__(kGemvThreads) void k_gemv(GemvArgs a) {
  __shared__ __align__(16) int8_t xq_lds[kMaxK];
  __shared__ float xf_lds[PRO == PRO_XQ ? 1 : kMaxK];
  __shared__ float red[64];
  const int row_in = blockIdx.y;                  // activation row (prefill runs rows on grid y)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int N = a.N, K = a.K;
  const float s_x = gemv_prologue<PRO>(a, row_in, xq_lds, xf_lds, red);
  if (a.xq_out != nullptr && blockIdx.x == 0) {
    for (int i = threadIdx.x; i < K; i += kGemvThreads) a.xq_out[row_in * a.xq_stride + i] = xq_lds[i];
    if (threadIdx.x == 0) a.sx_out[row_in] = s_x;
  }
  int4 xr[NCB];
#pragma unroll
  for (int c = 0; c < NCB; ++c) {
    const int col = lane * 16 + c * 1024;
    xr[c] = col < K ? *(const int4*)(xq_lds + col) : make_int4(0, 0, 0, 0);
  }
  float* y = a.y + row_in * a.y_stride;
  const float* res = a.res ? a.res + row_in * a.res_stride : nullptr;
  unsigned long long best = 0;
  const int nwaves = gridDim.x * (kGemvThreads / 64);
  for (int r0 = (blockIdx.x * (kGemvThreads / 64) + wave) * RU; r0 < N; r0 += nwaves * RU) {
    int4 wv[RU][NCB];
    int4 wv3[EPI == EPI_SWIGLU ? RU : 1][NCB];
    long long wrow[RU];
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const int row = r0 + u;
      wrow[u] = row < N ? weight_row(a, row_in, row) : 0;
#pragma unroll
      for (int c = 0; c < NCB; ++c) {
        const int col = lane * 16 + c * 1024;
        const bool ok = row < N && col < K;
        wv[u][c] = ok ? load_nt16(a.w + wrow[u] * K + col) : make_int4(0, 0, 0, 0);
        if (EPI == EPI_SWIGLU)
          wv3[u][c] = ok ? load_nt16(a.w3 + wrow[u] * K + col)
                         : make_int4(0, 0, 0, 0);
      }
    }
    int acc[RU], acc3[RU];
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      acc[u] = 0;
      acc3[u] = 0;
#pragma unroll
      for (int c = 0; c < NCB; ++c) {
        acc[u] = dot16(wv[u][c], xr[c], acc[u]);
        if (EPI == EPI_SWIGLU) acc3[u] = dot16(wv3[u][c], xr[c], acc3[u]);
      }
      acc[u] = wave_sum_i32(acc[u]);
      if (EPI == EPI_SWIGLU) acc3[u] = wave_sum_i32(acc3[u]);
    }
    if (lane == 0) {
#pragma unroll
      for (int u = 0; u < RU; ++u) {
        const int row = r0 + u;
        if (row >= N) break;
        float v = dequant(acc[u], a.s_w[wrow[u]], s_x);
        if (EPI == EPI_SWIGLU) v = silu_mul(v, dequant(acc3[u], a.s_w3[wrow[u]], s_x));
        if (EPI == EPI_RESID) v = res[row] + v;
        y[row] = v;
        if (a.acc_out != nullptr) {
          const long long base = (long long)row_in * N * (EPI == EPI_SWIGLU ? 2 : 1);
          a.acc_out[base + row] = acc[u];
          if (EPI == EPI_SWIGLU) a.acc_out[base + N + row] = acc3[u];
        }
        if (a.argmax_key != nullptr) {
          unsigned long long k = argmax_key(v, row);
          best = k > best ? k : best;
        }
      }
    }
  }
  if (a.argmax_key != nullptr && lane == 0 && best != 0) atomicMax(a.argmax_key + row_in, best);
}

}  // namespace t2r
