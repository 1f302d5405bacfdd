// W8A8 GEMV for decode: int8 weight rows streamed from HBM with 128-bit loads, int8 dot
// products (v_dot4) into exact int32 accumulators, wave reductions, and the dequantisation
// y = F(F(f32(acc) * s_w[n]) * s_x) fused with what surrounds the linear layer in the
// reference's op list (llm/compile_model.py:147-171, 295-331):
//
//  prologue  PRO_XQ          the int8 activations and their scale are given
//            PRO_QUANT       quant_act of an fp32 vector (llm/ref_model.py:191-196)
//            PRO_NORM_QUANT  RMSNorm then quant_act (llm/ref_model.py:204-207)
//            PRO_SPLITQ      quant_act of x = F(f32(p0 + p1 + p2 + p3) * xs_scale) from four int32
//                            partial vectors (the split decode attention's P.V sums)
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

enum { PRO_XQ = 0, PRO_QUANT = 1, PRO_NORM_QUANT = 2, PRO_SPLITQ = 3 };
enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2 };
constexpr int kMaxK = 8192;
constexpr int kOsumLds = kMaxK + 16 * 8;   // D * osum_stride(kMaxK, D) floats, D <= 16
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
  const float* tab;          // the SFU tables (kSfuWords floats, 16-byte aligned) in device memory
  const int32_t* xs;         // PRO_SPLITQ: four int32 partial vectors [4][xs_stride] (16-byte aligned)
  long long xs_stride;
  float xs_scale;
  int act;                   // EPI_SWIGLU gate: 0 SiLU, 1 GELU-tanh (gate_mul)
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
  float r = 1.0f;
  float* ot = xf_lds + kMaxK;                      // lane-major copy for the ordered sum
  if (PRO == PRO_NORM_QUANT) {
    const int P = osum_stride(K, a.D), pad = ((K + a.D - 1) / a.D) * a.D;
    for (int i = tid; i < pad; i += kGemvThreads) ot[osum_index(i, a.D, P)] = i < K ? x[i] : 0.0f;
  }
  for (int i = tid; i < K; i += kGemvThreads) xf_lds[i] = x[i];
  __syncthreads();
  if (PRO == PRO_NORM_QUANT) {
    if (tid < a.D) {
      const float ss = ordered_sum_t<true>(ot, K, a.D, osum_stride(K, a.D), tid);
      if (tid == 0) red[32] = sfu_rsqrt(ss * a.inv_n + a.eps);
    }
    __syncthreads();
    r = red[32];
  }
  uint32_t am = 0;
  for (int i = tid; i < K; i += kGemvThreads) {
    float v = xf_lds[i];
    if (PRO == PRO_NORM_QUANT) {
      v = (v * r) * a.g[i];
      xf_lds[i] = v;
    }
    am = max(am, abs_bits(v));
  }
  const float amax = block_absmax(am, red);
  const float s_x = amax * kInv127;
  const float inv = sfu_recip(s_x);
  for (int i = tid; i < K; i += kGemvThreads) xq_lds[i] = (int8_t)to_i8(xf_lds[i] * inv);
  __syncthreads();
  return s_x;
}

// One wave's tile: RU rows x NCB 1024-byte chunks of weights (16 bytes per lane per chunk), and the
// rows' scales and residuals, so the epilogue needs no load of its own.
template <int EPI, int NCB, int RU>
struct WTile {
  int4 w[RU][NCB];
  int4 w3[EPI == EPI_SWIGLU ? RU : 1][NCB];
  float sw[RU], sw3[EPI == EPI_SWIGLU ? RU : 1], res[EPI == EPI_RESID ? RU : 1];
};

// Branch-free: every lane issues every load. A row past N reads row N - 1 (its result is never
// stored) and a column past K reads the row's last 16 bytes (the activations there are +0, so the
// products vanish). Loads under branches would cost more than the wasted bytes: the compiler
// could no longer count them, and would wait for all of them before the prologue's first use of
// its own (earlier) loads. IDX: weight rows through the MoE id table, looked up first.
template <int EPI, int NCB, int RU, bool IDX>
T2R_DEV void load_tile(WTile<EPI, NCB, RU>& t, const GemvArgs& a, const float* res, int row_in, int r0, int lane) {
  long long wr[RU];
  int rc[RU];
#pragma unroll
  for (int u = 0; u < RU; ++u) {
    rc[u] = min(r0 + u, a.N - 1);
    wr[u] = IDX ? weight_row(a, row_in, rc[u]) : rc[u];
  }
#pragma unroll
  for (int u = 0; u < RU; ++u) {
#pragma unroll
    for (int c = 0; c < NCB; ++c) {
      const int col = min(lane * 16 + c * 1024, a.K - 16);
      t.w[u][c] = load_nt16(a.w + wr[u] * a.K + col);
      if (EPI == EPI_SWIGLU) t.w3[u][c] = load_nt16(a.w3 + wr[u] * a.K + col);
    }
    t.sw[u] = a.s_w[wr[u]];
    if (EPI == EPI_SWIGLU) t.sw3[u] = a.s_w3[wr[u]];
    if (EPI == EPI_RESID) t.res[u] = res[rc[u]];
  }
}

// The prologue's inputs, loaded into registers before the first weight tile is requested (the
// wait for them then does not wait for the tile): K <= 1024 * NCB. NORM/QUANT inputs are read as
// float4 (thread t holds elements 4 (t + NT j) .. + 3), int8 inputs as int4; the SFU tables travel
// with them when the kernel looks anything up.
template <int PRO, int EPI, int NCB, int NT>
struct XStage {
  static constexpr int NX = (256 * NCB) / NT > 0 ? (256 * NCB) / NT : 1;   // float4 per thread
  static constexpr int NQ = (64 * NCB) / NT > 0 ? (64 * NCB) / NT : 1;     // int4 per thread
  static constexpr bool SFU = PRO != PRO_XQ || EPI == EPI_SWIGLU;
  float4 x[PRO == PRO_XQ || PRO == PRO_SPLITQ ? 1 : NX];
  v4i_t xs[PRO == PRO_SPLITQ ? 4 * NX : 1];
  float4 g[PRO == PRO_NORM_QUANT ? NX : 1];
  v4i_t q[PRO == PRO_XQ ? NQ : 1];
  v4f_t tab;
};

template <int PRO, int EPI, int NCB, int NT>
T2R_DEV void stage_load(XStage<PRO, EPI, NCB, NT>& st, const GemvArgs& a, int row) {
  typedef XStage<PRO, EPI, NCB, NT> S;
  const int tid = threadIdx.x, K = a.K;
  // unconditional loads at clamped addresses (see load_tile); elements past K are never used
  if (S::SFU) st.tab = ((const v4f_t*)a.tab)[tid & (kSfuWords / 4 - 1)];
  if (PRO == PRO_XQ) {
    const int8_t* src = a.xq + row * a.xq_stride;
#pragma unroll
    for (int j = 0; j < S::NQ; ++j) st.q[j] = *(const v4i_t*)(src + min((tid + j * NT) * 16, K - 16));
  } else if (PRO == PRO_SPLITQ) {
#pragma unroll
    for (int j = 0; j < S::NX; ++j) {
      const int i = min((tid + j * NT) * 4, K - 4);
#pragma unroll
      for (int z = 0; z < 4; ++z) st.xs[4 * j + z] = *(const v4i_t*)(a.xs + z * a.xs_stride + i);
    }
  } else {
    const float* x = a.x + row * a.x_stride;
#pragma unroll
    for (int j = 0; j < S::NX; ++j) {
      const int i = min((tid + j * NT) * 4, K - 4);
      st.x[j] = *(const float4*)(x + i);
      if (PRO == PRO_NORM_QUANT) st.g[j] = *(const float4*)(a.g + i);
    }
  }
}

// RMSNorm / quant_act from the staged registers (same numerics as gemv_prologue); leaves the int8
// activations in xq_lds and the SFU tables in tab_lds, returns s_x
template <int PRO, int EPI, int NCB, int NT, bool DEEP = false>
T2R_DEV float stage_finish(const XStage<PRO, EPI, NCB, NT>& st, const GemvArgs& a, int row, int8_t* xq_lds,
                           float* xf_lds, float* tab_lds, float* red) {
  typedef XStage<PRO, EPI, NCB, NT> S;
  const int tid = threadIdx.x, K = a.K;
  if (S::SFU) sfu_store(tab_lds, st.tab);
  if (PRO == PRO_XQ) {
#pragma unroll
    for (int j = 0; j < S::NQ; ++j) {
      const int i = (tid + j * NT) * 16;
      if (i < K) *(v4i_t*)(xq_lds + i) = st.q[j];
    }
    __syncthreads();
    return a.s_x[row];
  }
  constexpr int NV = 4 * S::NX;
  float xv[NV];
  if constexpr (PRO == PRO_SPLITQ) {
    // the four partial sums (exact int32), then x = F(f32(sum) * xs_scale)
#pragma unroll
    for (int j = 0; j < S::NX; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        xv[4 * j + e] = (float)(((st.xs[4 * j][e] + st.xs[4 * j + 1][e]) + st.xs[4 * j + 2][e]) + st.xs[4 * j + 3][e]) *
                        a.xs_scale;
  } else {
#pragma unroll
    for (int j = 0; j < S::NX; ++j) {
      xv[4 * j] = st.x[j].x; xv[4 * j + 1] = st.x[j].y; xv[4 * j + 2] = st.x[j].z; xv[4 * j + 3] = st.x[j].w;
    }
  }
  float r = 1.0f;
  if (PRO == PRO_NORM_QUANT) {
    // the squares F(x * x), lane-major for the ordered sum (K % D == 0: no padding)
    const int P = osum_stride(K, a.D);
#pragma unroll
    for (int j = 0; j < S::NX; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = (tid + j * NT) * 4 + e;
        if (i < K) xf_lds[osum_index(i, a.D, P)] = xv[4 * j + e] * xv[4 * j + e];
      }
    __syncthreads();
    if (tid < a.D) {
      // DEEP: the chain's values requested at once (K / D <= 128)
      const float ss = DEEP ? ordered_sum_t_all<false, 8>(xf_lds, K, a.D, P, tid) : ordered_sum_t<false>(xf_lds, K, a.D, P, tid);
      if (tid == 0) red[32] = sfu_rsqrt(ss * a.inv_n + a.eps, tab_lds);
    }
    __syncthreads();
    r = red[32];
#pragma unroll
    for (int j = 0; j < S::NX; ++j) {
      xv[4 * j] = (xv[4 * j] * r) * st.g[j].x;
      xv[4 * j + 1] = (xv[4 * j + 1] * r) * st.g[j].y;
      xv[4 * j + 2] = (xv[4 * j + 2] * r) * st.g[j].z;
      xv[4 * j + 3] = (xv[4 * j + 3] * r) * st.g[j].w;
    }
  }
  uint32_t am = 0;
#pragma unroll
  for (int j = 0; j < S::NX; ++j)
    if ((tid + j * NT) * 4 < K)
#pragma unroll
      for (int e = 0; e < 4; ++e) am = max(am, abs_bits(xv[4 * j + e]));
  const float amax = block_absmax(am, red);
  const float s_x = amax * kInv127;
  const float inv = sfu_recip(s_x, tab_lds);
#pragma unroll
  for (int j = 0; j < S::NX; ++j) {
    const int i = (tid + j * NT) * 4;
    if (i < K)
      *(int*)(xq_lds + i) = pack_i8x4(to_i8(xv[4 * j] * inv), to_i8(xv[4 * j + 1] * inv), to_i8(xv[4 * j + 2] * inv),
                                      to_i8(xv[4 * j + 3] * inv));
  }
  __syncthreads();
  return s_x;
}

// The tile walk of one wave: dot products of the wave's tile with the int8 activations in xq_lds,
// the next tile requested right after them, the tile's row sums in one multi-value reduction, and
// the dequant epilogue. Returns the wave's largest argmax key (0: none). WALK false: the grid covers
// every row in one tile per wave, so no next tile is ever requested (nor held in registers).
template <int EPI, int NCB, int RU, bool IDX, bool WALK = true>
T2R_DEV unsigned long long gemv_tiles(const GemvArgs& a, WTile<EPI, NCB, RU>& t, const float* res, int row_in, int r0,
                                      int nwaves, float s_x, const int8_t* xq_lds, const float* tab_lds, int lane) {
  const int N = a.N, K = a.K;
  int4 xr[NCB];
#pragma unroll
  for (int c = 0; c < NCB; ++c) {
    const int col = lane * 16 + c * 1024;
    xr[c] = col < K ? *(const int4*)(xq_lds + col) : make_int4(0, 0, 0, 0);
  }
  float* y = a.y + row_in * a.y_stride;
  unsigned long long best = 0;
  for (; r0 < N; r0 += nwaves * RU) {
    int acc[RU], acc3[RU];
    float sw[RU], sw3[RU], rs[RU];
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      acc[u] = 0;
      acc3[u] = 0;
#pragma unroll
      for (int c = 0; c < NCB; ++c) {
        acc[u] = dot16(t.w[u][c], xr[c], acc[u]);
        if (EPI == EPI_SWIGLU) acc3[u] = dot16(t.w3[u][c], xr[c], acc3[u]);
      }
      sw[u] = t.sw[u];
      sw3[u] = EPI == EPI_SWIGLU ? t.sw3[u] : 0.0f;
      rs[u] = EPI == EPI_RESID ? t.res[u] : 0.0f;
    }
    if (WALK && r0 + nwaves * RU < N) load_tile<EPI, NCB, RU, IDX>(t, a, res, row_in, r0 + nwaves * RU, lane);
    // the tile's RU row sums (and W3's) in one multi-value reduction: lane L ends with sum
    // (L >> SH) & (NV - 1) of vv; the lanes holding W1's sum of row u (and, beside them, W3's)
    // finish row r0 + u
    constexpr int NV = EPI == EPI_SWIGLU ? 2 * RU : RU;
    constexpr int SH = NV == 8 ? 0 : NV == 4 ? 1 : NV == 2 ? 2 : 3;
    int vv[NV];
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      if (EPI == EPI_SWIGLU) {
        vv[2 * u] = acc[u];
        vv[2 * u + 1] = acc3[u];
      } else {
        vv[u] = acc[u];
      }
    }
    const int tot = wave_sum_multi<NV>(vv);
    int tot3 = 0;                                   // W3's sum: the lane holding value idx + 1
    if constexpr (EPI == EPI_SWIGLU) tot3 = dpp_i<SH == 0 ? kDppXor1 : SH == 1 ? kDppXor2 : kDppHalfMirror>(tot);
    const int idx = (lane >> SH) & (NV - 1);
    const int ul = EPI == EPI_SWIGLU ? idx >> 1 : idx;
    if (lane < 8 && (lane & ((1 << SH) - 1)) == 0 && (EPI != EPI_SWIGLU || (idx & 1) == 0)) {
      int ac = tot, ac3 = tot3;
      float w1s = sw[0], w3s = sw3[0], rr = rs[0];
#pragma unroll
      for (int u = 1; u < RU; ++u)
        if (ul == u) {
          w1s = sw[u]; w3s = sw3[u]; rr = rs[u];
        }
      const int row = r0 + ul;
      if (row < N) {
        float v = dequant(ac, w1s, s_x);
        if (EPI == EPI_SWIGLU) v = gate_mul(v, dequant(ac3, w3s, s_x), a.act, tab_lds);
        if (EPI == EPI_RESID) v = rr + v;
        y[row] = v;
        if (a.acc_out != nullptr) {
          const long long base = (long long)row_in * N * (EPI == EPI_SWIGLU ? 2 : 1);
          a.acc_out[base + row] = ac;
          if (EPI == EPI_SWIGLU) a.acc_out[base + N + row] = ac3;
        }
        if (a.argmax_key != nullptr) {
          const unsigned long long k = argmax_key(v, row);
          best = k > best ? k : best;
        }
      }
    }
    if (!WALK) break;
  }
  return best;
}

// greedy argmax over the block's NW waves: one atomic per block at most, skipped when the key
// already holds a larger one. Every wave of the block calls it (it has a barrier).
template <int NW>
T2R_DEV void gemv_argmax(const GemvArgs& a, unsigned long long best, int row_in, int lane, int wave) {
  __shared__ unsigned long long bk[NW];
  for (int o = 1; o < 64; o <<= 1) {
    const unsigned long long other = __shfl_xor(best, o);
    best = other > best ? other : best;
  }
  if (lane == 0) bk[wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long b = bk[0];
    for (int w = 1; w < NW; ++w) b = bk[w] > b ? bk[w] : b;
    unsigned long long* key = a.argmax_key + row_in;
    if (b != 0 && b > __atomic_load_n(key, __ATOMIC_RELAXED)) atomicMax(key, b);
  }
}

// NCB: 1024-byte column chunks per row covered by the register slice (K <= NCB * 1024);
// RU: rows per wave tile; NT: threads per block. A wave's first tile is requested right after the
// prologue's inputs and before the prologue runs, and each next tile right after the current one's
// dot products, so HBM stays busy while the prologue, the reductions and the epilogues run.
template <int PRO, int EPI, int NCB, int RU, int NT, bool IDX>
__global__ __launch_bounds__(NT) void k_gemv(GemvArgs a) {
  __shared__ __align__(16) int8_t xq_lds[kMaxK];
  __shared__ __align__(16) float xf_lds[PRO == PRO_NORM_QUANT ? kOsumLds : 1];
  __shared__ __align__(16) float tab_lds[XStage<PRO, EPI, NCB, NT>::SFU ? kSfuWords : 1];
  __shared__ float red[64];
  const int row_in = blockIdx.y;                  // activation row (MoE prefill runs rows on grid y)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int K = a.K;
  const int nwaves = gridDim.x * (NT / 64);
  const float* res = a.res ? a.res + row_in * a.res_stride : nullptr;
  const int r0 = (blockIdx.x * (NT / 64) + wave) * RU;
  XStage<PRO, EPI, NCB, NT> st;
  stage_load(st, a, row_in);
  // keep the issue order: the prologue's loads strictly before the tile's (waits count in order)
  __builtin_amdgcn_sched_barrier(0);
  WTile<EPI, NCB, RU> t;
  load_tile<EPI, NCB, RU, IDX>(t, a, res, row_in, r0, lane);
  __builtin_amdgcn_sched_barrier(0);
  const float s_x = stage_finish(st, a, row_in, xq_lds, xf_lds, tab_lds, red);
  if (a.xq_out != nullptr && blockIdx.x == 0) {
    for (int i = threadIdx.x; i < K; i += NT) a.xq_out[row_in * a.xq_stride + i] = xq_lds[i];
    if (threadIdx.x == 0) a.sx_out[row_in] = s_x;
  }
  const unsigned long long best = gemv_tiles<EPI, NCB, RU, IDX>(a, t, res, row_in, r0, nwaves, s_x, xq_lds, tab_lds, lane);
  if (a.argmax_key != nullptr) gemv_argmax<NT / 64>(a, best, row_in, lane, wave);
}

// RMSNorm + quant_act of row `row` by one wave (the block's wave 0), with the numerics of
// stage_finish<PRO_NORM_QUANT>: squares F(x * x) in the lane-major layout, the ordered sum by
// lanes [0, D), RSQRT, x F(x r) g, max |x| over the row, RECIP of s_x, to_i8. Writes the SFU
// tables to tab_lds, the int8 row to xq_lds and s_x to *sx_lds. Only this wave's own LDS writes are
// read back before the block's barrier: a wave's LDS accesses complete in program order.
// where pw_prologue parks x in its LDS scratch: past the lane-major squares (at most D * P = 2080
// floats for K <= 2048), with room for K <= 2048 values of its own
constexpr int kPwXNat = 4096;
static_assert(kPwXNat + 2048 <= kOsumLds, "pw_prologue's LDS scratch");

template <int NCB>
T2R_DEV void pw_prologue(const GemvArgs& a, int row, int8_t* xq_lds, float* xf_lds, float* tab_lds, float* sx_lds,
                         int lane) {
  static_assert(NCB <= 2, "pw_prologue holds K <= 2048");
  constexpr int NX = 4 * NCB;                     // float4 per lane: K <= 1024 NCB
  constexpr int NTB = kSfuWords / 256;            // table float4 per lane
  const int K = a.K;
  const float* x = a.x + row * a.x_stride;
  v4f_t tb[NTB];
  float4 xv4[NX], g4[NX];
#pragma unroll
  for (int s = 0; s < NTB; ++s) tb[s] = ((const v4f_t*)a.tab)[lane + 64 * s];
#pragma unroll
  for (int j = 0; j < NX; ++j) {
    const int i = min((lane + 64 * j) * 4, K - 4);  // clamped: elements past K are never used
    xv4[j] = *(const float4*)(x + i);
    g4[j] = *(const float4*)(a.g + i);
  }
#pragma unroll
  for (int s = 0; s < NTB; ++s) ((v4f_t*)tab_lds)[lane + 64 * s] = tb[s];
  // the squares in the lane-major layout of the ordered sum, and x itself parked in LDS (at
  // kPwXNat, past the squares) so that its registers are free during the chain
  const int P = osum_stride(K, a.D);
  float* xnat = xf_lds + kPwXNat;
#pragma unroll
  for (int j = 0; j < NX; ++j) {
    const float e4[4] = {xv4[j].x, xv4[j].y, xv4[j].z, xv4[j].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = (lane + 64 * j) * 4 + e;
      if (i < K) xf_lds[osum_index(i, a.D, P)] = e4[e] * e4[e];
    }
    *(float4*)(xnat + (lane + 64 * j) * 4) = xv4[j];
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  float rr = 0.0f;
  if (lane < a.D) {
    // the chain's values requested at once (K / D <= 128; C4 decode 1,903 -> 1,909 tok/s)
    const float ss = ordered_sum_t_all<false, 8>(xf_lds, K, a.D, P, lane);
    rr = sfu_rsqrt(ss * a.inv_n + a.eps, tab_lds);
  }
  const float r = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rr), 0));
  float xv[4 * NX];
#pragma unroll
  for (int j = 0; j < NX; ++j) {
    const float4 v = *(const float4*)(xnat + (lane + 64 * j) * 4);
    xv[4 * j] = v.x; xv[4 * j + 1] = v.y; xv[4 * j + 2] = v.z; xv[4 * j + 3] = v.w;
  }
  uint32_t am = 0;
#pragma unroll
  for (int j = 0; j < NX; ++j) {
    xv[4 * j] = (xv[4 * j] * r) * g4[j].x;
    xv[4 * j + 1] = (xv[4 * j + 1] * r) * g4[j].y;
    xv[4 * j + 2] = (xv[4 * j + 2] * r) * g4[j].z;
    xv[4 * j + 3] = (xv[4 * j + 3] * r) * g4[j].w;
    if ((lane + 64 * j) * 4 < K)
#pragma unroll
      for (int e = 0; e < 4; ++e) am = max(am, abs_bits(xv[4 * j + e]));
  }
  const float s_x = fv(wave_max_u32(am)) * kInv127;
  const float inv = sfu_recip(s_x, tab_lds);
#pragma unroll
  for (int j = 0; j < NX; ++j) {
    const int i = (lane + 64 * j) * 4;
    if (i < K)
      *(int*)(xq_lds + i) = pack_i8x4(to_i8(xv[4 * j] * inv), to_i8(xv[4 * j + 1] * inv), to_i8(xv[4 * j + 2] * inv),
                                      to_i8(xv[4 * j + 3] * inv));
  }
  if (lane == 0) *sx_lds = s_x;
}

// The RMSNorm GEMV with a prologue wave: wave 0 of each block loads the row, the gain and the SFU
// tables and runs the whole prologue (pw_prologue); waves 1..WS issue their weight tiles at once and
// wait at the block's barrier. The prologue's instructions then never sit behind a tile's load
// issue (a wave issues in order, and a CU accepts new loads only as its outstanding ones drain), and
// the chain of the ordered sum runs while the weights stream. Same results as k_gemv<PRO_NORM_QUANT>.
// Bounded to three waves per SIMD (<= 168 VGPRs), so that a 9-wave block fits on one CU beside
// another kernel's tail. The grid covers the N rows in one tile per streaming wave.
template <int EPI, int NCB, int RU, int WS>
__global__ __launch_bounds__(64 * (WS + 1), 3) void k_gemv_pw(GemvArgs a) {
  static_assert(EPI != EPI_RESID, "the prologue-wave GEMV has no residual operand");
  __shared__ __align__(16) int8_t xq_lds[kMaxK];
  __shared__ __align__(16) float xf_lds[kOsumLds];
  __shared__ __align__(16) float tab_lds[kSfuWords];
  __shared__ float sx_lds;
  const int row_in = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int K = a.K;
  const int nwaves = gridDim.x * WS;
  const int r0 = (blockIdx.x * WS + wave - 1) * RU;
  WTile<EPI, NCB, RU> t;
  if (wave == 0) pw_prologue<NCB>(a, row_in, xq_lds, xf_lds, tab_lds, &sx_lds, lane);
  else load_tile<EPI, NCB, RU, false>(t, a, nullptr, row_in, r0, lane);
  __syncthreads();
  const float s_x = sx_lds;
  if (a.xq_out != nullptr && blockIdx.x == 0) {
    for (int i = threadIdx.x; i < K; i += 64 * (WS + 1)) a.xq_out[row_in * a.xq_stride + i] = xq_lds[i];
    if (threadIdx.x == 0) a.sx_out[row_in] = s_x;
  }
  unsigned long long best = 0;
  if (wave > 0) best = gemv_tiles<EPI, NCB, RU, false, false>(a, t, nullptr, row_in, r0, nwaves, s_x, xq_lds, tab_lds, lane);
  if (a.argmax_key != nullptr) gemv_argmax<WS + 1>(a, best, row_in, lane, wave);
}

}  // namespace t2r
