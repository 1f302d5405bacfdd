// Row kernels around the linear layers and attention: embedding, RMSNorm / quant_act rows,
// RoPE, KV append, the MoE router / expert combine, argmax, and the element-wise hooks that let
// the tests see the SFU and the flush-to-zero primitives bit for bit.
#pragma once
#include "t2r_gemm.h"
#include "t2r_gemv.h"

namespace t2r {

// x[r] = F(f32(emb_q[tok[r]]) * emb_s[tok[r]]) (llm/ref_model.py:221); block 0 also clears the
// argmax keys of the step (one per row) when given.
__global__ __launch_bounds__(256) void k_embed(const int8_t* emb_q, const float* emb_s, const int32_t* tokens,
                                               int dim, int vocab, float* x, long long x_stride,
                                               unsigned long long* keys, int nkeys, int32_t* status) {
  const int r = blockIdx.x;
  int t = tokens[r];
  if (t < 0 || t >= vocab) {
    if (threadIdx.x == 0 && status) atomicOr(status, 1);   // out-of-range token: row 0 of the table instead
    t = 0;
  }
  const float s = emb_s[t];
  const int8_t* e = emb_q + (long long)t * dim;
  float* xr = x + r * x_stride;
  int done = 0;
  if (dim % 16 == 0 && ((uintptr_t)e & 15) == 0 && ((uintptr_t)xr & 15) == 0) {
    // 16 bytes a thread and pass, every pass's load issued (from a clamped address) before the first
    // conversion: one memory round trip for the row instead of one per pass
    constexpr int NP = 4;
    const int span = 16 * (int)blockDim.x;
    v4i_t q[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) q[p] = *(const v4i_t*)(e + min(16 * (int)threadIdx.x + span * p, dim - 16));
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int i = 16 * (int)threadIdx.x + span * p;
      if (i < dim) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int v = q[p][w];
          *(float4*)(xr + i + 4 * w) = make_float4((float)(int8_t)v * s, (float)(int8_t)(v >> 8) * s,
                                                   (float)(int8_t)(v >> 16) * s, (float)(int8_t)(v >> 24) * s);
        }
      }
    }
    done = min(dim, NP * span);
  }
  for (int i = done + threadIdx.x; i < dim; i += blockDim.x) xr[i] = (float)e[i] * s;
  if (keys && r == 0)
    for (int i = threadIdx.x; i < nkeys; i += blockDim.x) keys[i] = 0;
}

// The prefill row kernels over rows of more than 1024 values request their norm chain's values at once
// (C4's 512 rows: prefill 1.86 -> 1.83 ms); over shorter rows, with thousands of rows, the registers
// that takes cost more occupancy than it saves (C3 measured slower).
template <int NCB>
constexpr bool rows_deep() { return NCB == 2; }
// RMSNorm and / or quant_act of rows (prefill inputs of the MFMA GEMM; the op-level ABI).
// out_f: normalised rows (optional), xq / s_x: quantised rows (optional).
__global__ __launch_bounds__(kGemvThreads) void k_rows_norm_quant(GemvArgs a, int norm, float* out_f, long long out_stride) {
  __shared__ __align__(16) int8_t xq_lds[kMaxK];
  __shared__ __align__(16) float xf_lds[kMaxK + kOsumLds];
  __shared__ float red[64];
  const int row = blockIdx.x;
  float s_x;
  if (norm) s_x = gemv_prologue<PRO_NORM_QUANT>(a, row, xq_lds, xf_lds, red);
  else s_x = gemv_prologue<PRO_QUANT>(a, row, xq_lds, xf_lds, red);
  for (int i = threadIdx.x; i < a.K; i += kGemvThreads) {
    if (out_f) out_f[row * out_stride + i] = xf_lds[i];
    if (a.xq_out) a.xq_out[row * a.xq_stride + i] = xq_lds[i];
  }
  if (threadIdx.x == 0 && a.sx_out) a.sx_out[row] = s_x;
}

// Prefill rows: RMSNorm (PRO_NORM_QUANT) or quant_act alone (PRO_QUANT) of row blockIdx.x into the
// int8 rows the MFMA GEMM reads (K <= 1024 NCB): the decode GEMV's staged prologue (inputs in
// registers, lane-major squares for the one ordered chain, block max), same numerics.
template <int PRO, int NCB>
__global__ __launch_bounds__(kGemvThreads) void k_rows_quant(GemvArgs a) {
  __shared__ __align__(16) int8_t xq_lds[1024 * NCB];
  __shared__ __align__(16) float xf_lds[PRO == PRO_NORM_QUANT ? 1024 * NCB + 128 : 1];
  __shared__ __align__(16) float tab_lds[kSfuWords];
  __shared__ float red[64];
  const int row = blockIdx.x;
  XStage<PRO, EPI_STORE, NCB, kGemvThreads> st;
  stage_load(st, a, row);
  const float s_x = stage_finish<PRO, EPI_STORE, NCB, kGemvThreads, rows_deep<NCB>()>(st, a, row, xq_lds, xf_lds, tab_lds, red);
  int8_t* out = a.xq_out + row * a.xq_stride;
  for (int i = threadIdx.x * 16; i < a.K; i += kGemvThreads * 16) *(v4i_t*)(out + i) = *(const v4i_t*)(xq_lds + i);
  if (threadIdx.x == 0) a.sx_out[row] = s_x;
}

// The split-K finish of a residual linear fused with the row RMSNorm / quant_act that reads its
// output: x[row] = F(res + F(F(f32(sum_z part[z, row]) * s_w) * s_x_in[row])) (the residual epilogue,
// llm/ref_model.py:198-202 and :229-230; the int32 sum is exact in any order) is stored back into the
// residual rows, then normalised and quantised as k_rows_quant<PRO_NORM_QUANT> does. The partials are
// [nz, rows, K] (K = the linear's output width). s_x_in may be a.sx_out: each row's scale is read
// before its new one is written.
struct FinArgs {
  const int32_t* part;
  long long zstride;                 // rows * K
  int nz;
  const float* s_w;                  // [K] the linear's row scales
  const float* s_x;                  // [rows] its input scales
  float* x;                          // the residual rows (a.x, writable)
};

template <int NCB>
__global__ __launch_bounds__(kGemvThreads) void k_rows_fin_quant(GemvArgs a, FinArgs f) {
  __shared__ __align__(16) int8_t xq_lds[1024 * NCB];
  __shared__ __align__(16) float xf_lds[1024 * NCB + 128];
  __shared__ __align__(16) float tab_lds[kSfuWords];
  __shared__ float red[64];
  typedef XStage<PRO_NORM_QUANT, EPI_STORE, NCB, kGemvThreads> S;
  const int row = blockIdx.x, tid = threadIdx.x, K = a.K;
  S st;
  st.tab = ((const v4f_t*)a.tab)[tid & (kSfuWords / 4 - 1)];
  const float sx = f.s_x[row];
  float* xr = f.x + row * a.x_stride;
  const int32_t* pr = f.part + (long long)row * K;
  v4i_t acc[S::NX];
  float4 sw[S::NX];
#pragma unroll
  for (int j = 0; j < S::NX; ++j) {                // loads first (clamped, unconditional), then arithmetic
    const int i = min((tid + j * kGemvThreads) * 4, K - 4);
    st.x[j] = *(const float4*)(xr + i);
    st.g[j] = *(const float4*)(a.g + i);
    sw[j] = *(const float4*)(f.s_w + i);
    acc[j] = *(const v4i_t*)(pr + i);
  }
  // the other splits' partials (nz is 1, 2 or 4), requested together from clamped splits and added
  // where they exist (a loop over nz would wait for each split's load before the next)
  v4i_t pz[3][S::NX];
#pragma unroll
  for (int z = 1; z < 4; ++z)
#pragma unroll
    for (int j = 0; j < S::NX; ++j)
      pz[z - 1][j] = *(const v4i_t*)(pr + min(z, f.nz - 1) * f.zstride + min((tid + j * kGemvThreads) * 4, K - 4));
#pragma unroll
  for (int z = 1; z < 4; ++z)
#pragma unroll
    for (int j = 0; j < S::NX; ++j)
      if (z < f.nz) acc[j] += pz[z - 1][j];
  for (int z = 4; z < f.nz; ++z)                   // (more splits than the launcher makes: in order)
#pragma unroll
    for (int j = 0; j < S::NX; ++j) acc[j] += *(const v4i_t*)(pr + z * f.zstride + min((tid + j * kGemvThreads) * 4, K - 4));
#pragma unroll
  for (int j = 0; j < S::NX; ++j) {
    float4 v = st.x[j];
    v.x = v.x + dequant(acc[j].x, sw[j].x, sx);
    v.y = v.y + dequant(acc[j].y, sw[j].y, sx);
    v.z = v.z + dequant(acc[j].z, sw[j].z, sx);
    v.w = v.w + dequant(acc[j].w, sw[j].w, sx);
    st.x[j] = v;
    const int i = (tid + j * kGemvThreads) * 4;
    if (i < K) *(float4*)(xr + i) = v;
  }
  const float s_x = stage_finish<PRO_NORM_QUANT, EPI_STORE, NCB, kGemvThreads, rows_deep<NCB>()>(st, a, row, xq_lds, xf_lds, tab_lds, red);
  int8_t* out = a.xq_out + row * a.xq_stride;
  for (int i = tid * 16; i < K; i += kGemvThreads * 16) *(v4i_t*)(out + i) = *(const v4i_t*)(xq_lds + i);
  if (tid == 0) a.sx_out[row] = s_x;
}

// RMSNorm alone (no quantisation): out = F(F(x * r) * g), r = RSQRT(F(F(ss * F(1/n)) + F(eps)))
__global__ __launch_bounds__(256) void k_rmsnorm(const float* x, const float* g, int n, float inv_n, float eps, int D,
                                                 float* out) {
  __shared__ float xs[kMaxK];
  __shared__ __align__(16) float ot[kOsumLds];
  __shared__ float rr;
  const int row = blockIdx.x;
  x += (long long)row * n;
  out += (long long)row * n;
  const int P = osum_stride(n, D), pad = ((n + D - 1) / D) * D;
  for (int i = threadIdx.x; i < pad; i += blockDim.x) {
    const float v = i < n ? x[i] : 0.0f;
    if (i < n) xs[i] = v;
    ot[osum_index(i, D, P)] = v;
  }
  __syncthreads();
  if (threadIdx.x < D) {
    const float ss = ordered_sum_t<true>(ot, n, D, P, threadIdx.x);
    if (threadIdx.x == 0) rr = sfu_rsqrt(ss * inv_n + eps);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = (xs[i] * rr) * g[i];
}

// RoPE of rows v[rows, n] in place at positions pos[rows]; the tables are [S, half] (pairs of a
// head), n a multiple of 2 * half (the heads of a row).
__global__ __launch_bounds__(256) void k_rope(float* v, const float* cos_t, const float* sin_t, const int32_t* pos,
                                              int n, int half, int S) {
  const int row = blockIdx.x;
  float* r = v + (long long)row * n;
  const int p = pos[row];
  if (p < 0 || p >= S) return;
  for (int i = threadIdx.x; i < n / 2; i += blockDim.x) {
    const int k = i % half;
    const float c = cos_t[(long long)p * half + k], s = sin_t[(long long)p * half + k];
    const float v0 = r[2 * i], v1 = r[2 * i + 1];
    const float o0 = (v0 * c) + ((-v1) * s), o1 = (v1 * c) + (v0 * s);
    r[2 * i] = o0;
    r[2 * i + 1] = o1;
  }
}

// kc[pos[r]] = to_i8(F(k[r] * inv_sk)), vc[pos[r]] = to_i8(F(v[r] * inv_sv)); per channel c with
// inv_sk_ch[c] / inv_sv_ch[c] when given
__global__ __launch_bounds__(256) void k_kv_append(const float* k, const float* v, float inv_sk, float inv_sv,
                                                   const float* inv_sk_ch, const float* inv_sv_ch, int8_t* kc,
                                                   int8_t* vc, const int32_t* pos, int kv_dim, int S) {
  const int row = blockIdx.x;
  const long long p = pos[row];
  if (p < 0 || p >= S) return;
  for (int i = threadIdx.x; i < kv_dim; i += blockDim.x) {
    const float isk = inv_sk_ch ? inv_sk_ch[i] : inv_sk, isv = inv_sv_ch ? inv_sv_ch[i] : inv_sv;
    kc[p * kv_dim + i] = (int8_t)to_i8(k[(long long)row * kv_dim + i] * isk);
    vc[p * kv_dim + i] = (int8_t)to_i8(v[(long long)row * kv_dim + i] * isv);
  }
}

// Top-k of a score vector in device order (compiler/tests/oracle.py:558-585): descending value,
// an equal value before a larger id; NaN scores after every number. Then the route weights
// e = EXP(F(v - v0)), w = F(e * RECIP(red_sum(e))) (compiler/frontend/hf_generic.py:641-646).
// Run by lanes [0, 64) of wave 0; sc in LDS.
T2R_DEV bool route_before(float a, int ia, float b, int ib) {
  const bool na = a != a, nb = b != b;
  if (na || nb) return nb && (!na || ia < ib);
  if (a != b) return a > b;
  return ia < ib;
}

T2R_DEV void route_topk(const float* sc, int E, int k, int D, int lane, int32_t* ids, float* w, float* ev,
                        const float* tab = c_sfu) {
  // lane e's rank: how many experts come before it under route_before (a total order: ids differ)
  const float v = lane < E ? sc[lane] : 0.0f;
  int rank = 0;
  for (int j = 0; j < E; ++j) rank += route_before(sc[j], j, v, lane) ? 1 : 0;
  const bool sel = lane < E && rank < k;
  if (sel && rank == 0) ev[8] = v;                 // the top score v0
  __builtin_amdgcn_wave_barrier();
  const float v0 = ev[8];
  if (sel) {
    ids[rank] = lane;
    ev[rank] = sfu_exp(v - v0, tab);
  }
  __builtin_amdgcn_wave_barrier();
  float s = 0.0f;
  if (lane < D) s = ordered_sum<false>(ev, k, D, lane);
  s = __shfl(s, 0);
  const float r = sfu_recip(s, tab);
  if (lane < k) w[lane] = ev[lane] * r;
}

// The MoE router of rows: RMSNorm + quant_act of x (the activations every expert shares), the
// router's W8A8 scores, top-k and weights. One block per row; K <= 1024 * NCB. The prologue's inputs
// and the router's first 1024 columns are requested together, before the prologue runs, and the SFU
// tables are read from LDS (the decode GEMV's staged prologue).
struct RouteArgs {
  GemvArgs a;                 // x, g, inv_n, eps, D, router weights (w, s_w; N = E, K = dim), tab
  int k;
  int32_t* ids;               // [rows, k]
  float* wts;                 // [rows, k]
  float* scores;              // optional [rows, E]
};
template <int NCB>
__global__ __launch_bounds__(kGemvThreads) void k_moe_route(RouteArgs ra) {
  constexpr int NT = kGemvThreads, kWaves = NT / 64, kPerWave = 64 / kWaves;   // E <= 64 over the waves
  __shared__ __align__(16) int8_t xq_lds[NCB * 1024];
  __shared__ __align__(16) float xf_lds[kOsumLds];
  __shared__ __align__(16) float tab_lds[kSfuWords];
  __shared__ float red[64];
  __shared__ float sc[64];
  __shared__ float ev[16];
  const GemvArgs& a = ra.a;
  const int row = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  XStage<PRO_NORM_QUANT, EPI_STORE, NCB, NT> st;
  stage_load(st, a, row);
  __builtin_amdgcn_sched_barrier(0);
  const int col0 = lane * 16;
  int4 w0[kPerWave];
#pragma unroll
  for (int i = 0; i < kPerWave; ++i) {
    const int e = min(wave + kWaves * i, a.N - 1);
    w0[i] = load_nt16(a.w + (long long)e * a.K + min(col0, a.K - 16));
  }
  const float sw = a.s_w[min(lane, a.N - 1)];
  __builtin_amdgcn_sched_barrier(0);
  const float s_x = stage_finish(st, a, row, xq_lds, xf_lds, tab_lds, red);
  if (a.xq_out) {
    for (int i = threadIdx.x; i < a.K; i += NT) a.xq_out[row * a.xq_stride + i] = xq_lds[i];
    if (threadIdx.x == 0) a.sx_out[row] = s_x;
  }
  const int4 x0 = col0 < a.K ? *(const int4*)(xq_lds + col0) : make_int4(0, 0, 0, 0);
#pragma unroll
  for (int i = 0; i < kPerWave; ++i) {
    const int e = wave + kWaves * i;
    if (e >= a.N) break;
    int acc = dot16(w0[i], x0, 0);
    for (int col = col0 + 1024; col < a.K; col += 1024)
      acc = dot16(load_nt16(a.w + (long long)e * a.K + col), *(const int4*)(xq_lds + col), acc);
    acc = wave_sum_i32(acc);
    const float s_e = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sw), e));
    if (lane == 0) sc[e] = dequant(acc, s_e, s_x);
  }
  __syncthreads();
  if (ra.scores)
    for (int e = threadIdx.x; e < a.N; e += NT) ra.scores[row * a.N + e] = sc[e];
  if (wave == 0) route_topk(sc, a.N, ra.k, a.D, lane, ra.ids + row * ra.k, ra.wts + row * ra.k, ev, tab_lds);
}

// The router fused with the selected experts' gate / up GEMV (rows on grid y): every block repeats
// its row's routing (the router's staged prologue, the E scores, top-k and weights: the same bits in
// every block, with the same numerics as k_moe_route) and then computes its waves' tiles of the k Fe
// selected W1 / W3 rows with the SwiGLU gate (k_gemv's int8-input path: the tile rows through the ids
// in LDS). One launch instead of the router's single block followed by the GEMV, whose weight
// requests had to wait for the router kernel to end. Block 0 of the row writes the ids and weights
// for the down projections (and the int8 activations when xq_out is set).
struct MoeUpArgs {
  RouteArgs r;                // the router (r.a: x, g, inv_n, eps, D, w / s_w with N = E, K = dim, tab)
  GemvArgs up;                // gate / up: w, s_w, w3, s_w3, N = k Fe, K = dim, y, y_stride, act, rows_per_id = Fe
};
template <int NCB, int RU>
__global__ __launch_bounds__(kGemvThreads) void k_moe_up(MoeUpArgs m) {
  constexpr int NT = kGemvThreads, kWaves = NT / 64, kPerWave = 64 / kWaves;   // E <= 64 over the waves
  __shared__ __align__(16) int8_t xq_lds[NCB * 1024];
  __shared__ __align__(16) float xf_lds[kOsumLds];
  __shared__ __align__(16) float tab_lds[kSfuWords];
  __shared__ float red[64];
  __shared__ float sc[64];
  __shared__ float ev[16];
  __shared__ int32_t ids_l[16];
  __shared__ float wts_l[16];
  const GemvArgs& ra = m.r.a;
  const GemvArgs& a = m.up;
  const int row = blockIdx.y, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int k = m.r.k, Fe = a.rows_per_id, N = a.N, K = a.K;
  // ---- routing (k_moe_route's steps)
  XStage<PRO_NORM_QUANT, EPI_STORE, NCB, NT> st;
  stage_load(st, ra, row);
  __builtin_amdgcn_sched_barrier(0);
  const int col0 = lane * 16;
  int4 w0[kPerWave];
#pragma unroll
  for (int i = 0; i < kPerWave; ++i) {
    const int e = min(wave + kWaves * i, ra.N - 1);
    w0[i] = load_nt16(ra.w + (long long)e * ra.K + min(col0, ra.K - 16));
  }
  const float sw_r = ra.s_w[min(lane, ra.N - 1)];
  __builtin_amdgcn_sched_barrier(0);
  const float s_x = stage_finish(st, ra, row, xq_lds, xf_lds, tab_lds, red);
  if (ra.xq_out && blockIdx.x == 0) {
    for (int i = threadIdx.x; i < ra.K; i += NT) ra.xq_out[row * ra.xq_stride + i] = xq_lds[i];
    if (threadIdx.x == 0) ra.sx_out[row] = s_x;
  }
  const int4 x0 = col0 < ra.K ? *(const int4*)(xq_lds + col0) : make_int4(0, 0, 0, 0);
#pragma unroll
  for (int i = 0; i < kPerWave; ++i) {
    const int e = wave + kWaves * i;
    if (e >= ra.N) break;
    int acc = dot16(w0[i], x0, 0);
    for (int col = col0 + 1024; col < ra.K; col += 1024)
      acc = dot16(load_nt16(ra.w + (long long)e * ra.K + col), *(const int4*)(xq_lds + col), acc);
    acc = wave_sum_i32(acc);
    const float s_e = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sw_r), e));
    if (lane == 0) sc[e] = dequant(acc, s_e, s_x);
  }
  __syncthreads();
  if (wave == 0) route_topk(sc, ra.N, k, ra.D, lane, ids_l, wts_l, ev, tab_lds);
  __syncthreads();
  if (blockIdx.x == 0 && threadIdx.x < k) {
    m.r.ids[row * k + threadIdx.x] = ids_l[threadIdx.x];
    m.r.wts[row * k + threadIdx.x] = wts_l[threadIdx.x];
  }
  // ---- the gate / up rows of the selected experts: tile row r reads weight row ids[r / Fe] Fe + r % Fe
  const int nwaves = gridDim.x * (NT / 64);
  int r0 = (blockIdx.x * (NT / 64) + wave) * RU;
  WTile<EPI_SWIGLU, NCB, RU> t;
  auto tile = [&](int rb) {
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const int rc = min(rb + u, N - 1), j = rc / Fe;
      const long long wr = (long long)ids_l[j] * Fe + (rc - j * Fe);
#pragma unroll
      for (int c = 0; c < NCB; ++c) {
        const int col = min(lane * 16 + c * 1024, K - 16);
        t.w[u][c] = load_nt16(a.w + wr * K + col);
        t.w3[u][c] = load_nt16(a.w3 + wr * K + col);
      }
      t.sw[u] = a.s_w[wr];
      t.sw3[u] = a.s_w3[wr];
    }
  };
  tile(r0);
  int4 xr[NCB];
#pragma unroll
  for (int c = 0; c < NCB; ++c) {
    const int col = lane * 16 + c * 1024;
    xr[c] = col < K ? *(const int4*)(xq_lds + col) : make_int4(0, 0, 0, 0);
  }
  float* y = a.y + row * a.y_stride;
  for (; r0 < N; r0 += nwaves * RU) {
    int acc[RU], acc3[RU];
    float sw[RU], sw3[RU];
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      acc[u] = 0;
      acc3[u] = 0;
#pragma unroll
      for (int c = 0; c < NCB; ++c) {
        acc[u] = dot16(t.w[u][c], xr[c], acc[u]);
        acc3[u] = dot16(t.w3[u][c], xr[c], acc3[u]);
      }
      sw[u] = t.sw[u];
      sw3[u] = t.sw3[u];
    }
    if (r0 + nwaves * RU < N) tile(r0 + nwaves * RU);
    // the RU row sums and W3's in one multi-value reduction (as in k_gemv): lane L holds sum
    // (L >> SH) & (NV - 1) of vv, W3's beside it; the lanes holding W1's sum of row u finish it
    constexpr int NV = 2 * RU;
    constexpr int SH = NV == 8 ? 0 : NV == 4 ? 1 : 2;
    int vv[NV];
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      vv[2 * u] = acc[u];
      vv[2 * u + 1] = acc3[u];
    }
    const int tot = wave_sum_multi<NV>(vv);
    const int tot3 = dpp_i<SH == 0 ? kDppXor1 : SH == 1 ? kDppXor2 : kDppHalfMirror>(tot);
    const int idx = (lane >> SH) & (NV - 1), ul = idx >> 1;
    if (lane < 8 && (lane & ((1 << SH) - 1)) == 0 && (idx & 1) == 0) {
      float w1s = sw[0], w3s = sw3[0];
#pragma unroll
      for (int u = 1; u < RU; ++u)
        if (ul == u) {
          w1s = sw[u]; w3s = sw3[u];
        }
      const int r = r0 + ul;
      if (r < N) y[r] = gate_mul(dequant(tot, w1s, s_x), dequant(tot3, w3s, s_x), a.act, tab_lds);
    }
  }
}

// ---- MoE over many rows (prefill): the experts' linears grouped by expert. The per-row kernels
// (k_moe_up, k_moe_down) stream each row's k experts for that row alone; here the step's routes
// (row r, slot j: entry r k + j) are listed per expert and every expert's weights are read once per
// 32 routes by an int8 MFMA tile (k_bgemv's main loop with the activation rows gathered through the
// list). The int32 sums are exact, and every float step is the per-row kernels' own, in their order.

// list[off[e] .. off[e + 1]) = the entries routed to expert e (in no particular order: each entry's
// result is computed on its own). One workgroup; E <= 64.
__global__ __launch_bounds__(256) void k_moe_lists(const int32_t* ids, int n, int E, int32_t* off, int32_t* list) {
  __shared__ int cnt[64], fill[64];
  const int tid = threadIdx.x;
  if (tid < 64) cnt[tid] = 0;
  __syncthreads();
  for (int i = tid; i < n; i += 256) atomicAdd(&cnt[min(max(ids[i], 0), E - 1)], 1);
  __syncthreads();
  if (tid == 0) {
    int o = 0;
    for (int e = 0; e < E; ++e) {
      off[e] = o;
      fill[e] = o;
      o += cnt[e];
    }
    off[E] = o;
  }
  __syncthreads();
  for (int i = tid; i < n; i += 256) list[atomicAdd(&fill[min(max(ids[i], 0), E - 1)], 1)] = i;
}

// quant_act of every route's expert output u_j (one wave per entry; k_moe_down's prologue): hq [n, F]
// int8, s_h [n]. F <= 1024.
__global__ __launch_bounds__(256) void k_moe_hq(const float* u, int n, int F, int8_t* hq, float* s_h) {
  const int lane = threadIdx.x & 63, ent = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (ent >= n) return;                           // (wave-uniform)
  const float* ur = u + (long long)ent * F;
  float4 uv[4];
  uint32_t am = 0;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int i = c * 256 + lane * 4;
    uv[c] = i < F ? *(const float4*)(ur + i) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    am = max(am, max(max(abs_bits(uv[c].x), abs_bits(uv[c].y)), max(abs_bits(uv[c].z), abs_bits(uv[c].w))));
  }
  const float sj = fv(wave_max_u32(am)) * kInv127, inv = sfu_recip(sj);
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int i = c * 256 + lane * 4;
    if (i < F)
      *(int*)(hq + (long long)ent * F + i) = pack_i8x4(to_i8(uv[c].x * inv), to_i8(uv[c].y * inv),
                                                       to_i8(uv[c].z * inv), to_i8(uv[c].w * inv));
  }
  if (lane == 0) s_h[ent] = sj;
}

// The grouped expert linear. Block b = (expert e, weight tile, route group g) takes the routes
// list[off[e] + 32 g ..] (at most 32; a group past the expert's routes ends at once):
//   MOE_GU (gate / up): X = mxq[r] (K = dim), tiles of 16 gate + the same 16 up rows of expert e,
//          u[r][j F + n] = gate(F(F(f32(s1) s_wg) s_x[r]), F(F(f32(s3) s_wu) s_x[r]))
//   MOE_DN (down): X = hq[r k + j] (K = F), tiles of 32 rows of wd[e] (dim x F),
//          t[r k + j][n] = F(w[r k + j] F(F(f32(s) s_wd) s_h[r k + j]))
enum { MOE_GU = 0, MOE_DN = 1 };
struct MoeGemmArgs {
  const int32_t* off;
  const int32_t* list;
  const int8_t* xq;           // GU: mxq [rows, dim] (row r = entry / k); DN: hq [rows k, F] (row = entry)
  const float* s_x;           // GU: msx [rows]; DN: s_h [rows k]
  const int8_t* w;            // GU: wg [E, F, dim]; DN: wd [E, dim, F]
  const float* s_w;           // [E, N]
  const int8_t* w3;           // GU: wu [E, F, dim]
  const float* s_w3;
  const float* wts;           // DN: route weights [rows k]
  float* y;                   // GU: u [rows, k F]; DN: t [rows k, dim]
  const float* tab;           // SFU tables (GU's gate)
  int act;
  int k, N, K;                // N: weight rows per expert (GU: F; DN: dim), K: their length
  int ntile, ngrp;            // weight tiles per expert, route groups per expert
};
template <int MODE, int KW>
__global__ __launch_bounds__(64 * KW) void k_moe_gemm(MoeGemmArgs a) {
  extern __shared__ __align__(16) int8_t lds[];    // KW x kBgWaveLds
  __shared__ __align__(16) float tab_lds[MODE == MOE_GU ? kSfuWords : 4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 31, kh = lane >> 5;
  const int per_e = a.ntile * a.ngrp;
  const int e = blockIdx.x / per_e, tile = (blockIdx.x % per_e) / a.ngrp, grp = blockIdx.x % a.ngrp;
  const int beg = a.off[e] + 32 * grp, cnt = min(32, a.off[e + 1] - beg);
  if (cnt <= 0) return;                           // (block-uniform: before any barrier)
  constexpr int NT = MODE == MOE_GU ? 16 : 32;    // output columns per tile
  const int n0 = tile * NT, K = a.K, N = a.N;
  const int nwin = cdiv_i(K, kBgWin);
  int8_t* wl = lds + wave * kBgWaveLds;
  if (MODE == MOE_GU && tid < kSfuWords / 4) ((v4f_t*)tab_lds)[tid] = ((const v4f_t*)a.tab)[tid];
  const int8_t* we = a.w + (long long)e * N * K;
  const int8_t* we3 = MODE == MOE_GU ? a.w3 + (long long)e * N * K : we;
  const int8_t* rowp[8];
  int qo[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 4 * i + (lane >> 4);
    qo[i] = 16 * ((lane & 15) ^ (r & 15));
    if (MODE == MOE_GU) rowp[i] = (r < 16 ? we : we3) + (long long)min(n0 + (r & 15), N - 1) * K;
    else rowp[i] = we + (long long)min(n0 + r, N - 1) * K;
  }
  // lane lr's activation row: route lr of the group (routes past cnt repeat the last one, unused)
  const int ent = a.list[beg + min(lr, cnt - 1)];
  const int8_t* xrow = a.xq + (long long)(MODE == MOE_GU ? ent / a.k : ent) * K + 16 * kh;
  v16i_t acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0;
  for (int w = wave; w < nwin; w += KW) {
    const int k0 = w * kBgWin, nst = min(kBgWin, K - k0) >> 5;
    asm volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < 8; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(rowp[i] + min(k0 + qo[i], K - 16)), (void*)(wl + 1024 * i), 16, 0, 0);
    v4i_t xv[8];
#pragma unroll
    for (int st = 0; st < 8; ++st) xv[st] = *(const v4i_t*)(xrow + min(k0 + 32 * st, K - 32));
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    asm volatile("" ::: "memory");
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      if (st < nst) {
        const v4i_t wv = *(const v4i_t*)(wl + 256 * lr + 16 * ((2 * st + kh) ^ (lr & 15)));
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(xv[st], wv, acc, 0, 0, 0);
      }
    }
  }
  asm volatile("" ::: "memory");
  int* red = (int*)wl;
#pragma unroll
  for (int r = 0; r < 16; ++r) red[((r >> 2) * 8 + kh * 4 + (r & 3)) * 33 + lr] = acc[r];
  __syncthreads();
  constexpr int OPT = (32 * NT + 64 * KW - 1) / (64 * KW);
#pragma unroll
  for (int i = 0; i < OPT; ++i) {
    const int o = tid + i * 64 * KW, m = o / NT, j = o % NT, n = n0 + j;
    if (m >= cnt || n >= N) continue;
    int s1 = 0, s3 = 0;
#pragma unroll
    for (int v = 0; v < KW; ++v) {
      const int* rv = (const int*)(lds + v * kBgWaveLds);
      s1 += rv[m * 33 + j];
      if (MODE == MOE_GU) s3 += rv[m * 33 + 16 + j];
    }
    const int em = a.list[beg + m];
    if constexpr (MODE == MOE_GU) {
      const int r = em / a.k, slot = em - r * a.k;
      const float sx = a.s_x[r];
      a.y[((long long)r * a.k + slot) * N + n] =
          gate_mul(dequant(s1, a.s_w[(long long)e * N + n], sx), dequant(s3, a.s_w3[(long long)e * N + n], sx), a.act, tab_lds);
    } else {
      a.y[(long long)em * N + n] = a.wts[em] * dequant(s1, a.s_w[(long long)e * N + n], a.s_x[em]);
    }
  }
}

// x[r][n] = F(x[r][n] + y), y = +0 then y = F(y + t[r k + j][n]) for j = 0..k-1 in route order
// (k_moe_down's combine). Grid (dim / 256 blocks, rows).
__global__ __launch_bounds__(256) void k_moe_combine(const float* t, int k, int dim, float* x, long long x_stride) {
  const int r = blockIdx.y, n = blockIdx.x * 256 + threadIdx.x;
  if (n >= dim) return;
  float y = 0.0f;
  for (int j = 0; j < k; ++j) y = y + t[((long long)r * k + j) * dim + n];
  float* xr = x + (long long)r * x_stride + n;
  *xr = *xr + y;
}

// top-k + weights from given scores (the op-level ABI)
__global__ __launch_bounds__(64) void k_route_scores(const float* scores, int E, int k, int D, int32_t* ids, float* wts) {
  __shared__ float sc[64];
  __shared__ float ev[16];
  const int row = blockIdx.x;
  for (int e = threadIdx.x; e < E; e += 64) sc[e] = scores[row * E + e];
  __syncthreads();
  route_topk(sc, E, k, D, threadIdx.x, ids + row * k, wts + row * k, ev);
}

// MoE down projections and the ordered combine of one row (compiler/frontend/hf_generic.py:648-657):
//   hq_j, s_j = quant_act(u_j)                           per selected expert j
//   y_j[n]    = F(F(f32(wd[id_j][n] . hq_j) * s_wd) * s_j)
//   y[n] = +0; y[n] = F(y[n] + F(w_j * y_j[n])) for j = 0..k-1 in order; x[n] = F(x[n] + y[n])
// One wave per output row n (the grid covers dim); u rows [k, F] (F <= 1024, F % 16 == 0).
struct MoeDownArgs {
  const float* u;             // [rows, k, F]
  const int8_t* wd;           // [E, dim, F]
  const float* s_wd;          // [E, dim]
  const int32_t* ids;         // [rows, k]
  const float* wts;           // [rows, k]
  float* x;                   // [rows, dim] residual stream, updated in place
  int k, F, dim;
  long long x_stride;
};
__global__ __launch_bounds__(256) void k_moe_down(MoeDownArgs m) {
  __shared__ __align__(16) int8_t hq[8 * 1024];
  __shared__ float s_h[8];
  const int row = blockIdx.y, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int k = m.k, F = m.F;
  const int n = blockIdx.x * 4 + wave;
  const bool live = n < m.dim;
  const int32_t* idr = m.ids + row * k;
  // everything this wave's row needs, requested at once: the k weight rows (16 columns a lane), lane j's
  // expert scale and route weight, and x[n]
  const int col = lane * 16;
  int4 wv[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int id = j < k ? idr[j] : 0;
    wv[j] = (j < k && live && col < F) ? load_nt16(m.wd + ((long long)id * m.dim + n) * F + col)
                                       : make_int4(0, 0, 0, 0);
  }
  float swd = 0.0f, wj = 0.0f;
  if (lane < k && live) {
    swd = m.s_wd[(long long)idr[lane] * m.dim + n];
    wj = m.wts[row * k + lane];
  }
  float* xr = m.x + row * m.x_stride;
  const float x_old = live ? xr[n] : 0.0f;
  // quant_act of each selected expert's u (one wave per expert, the values kept in registers)
  const float* u = m.u + (long long)row * k * F;
  for (int j = wave; j < k; j += 4) {
    float4 uv[4];
    uint32_t am = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int i = c * 256 + lane * 4;
      uv[c] = i < F ? *(const float4*)(u + j * F + i) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      am = max(am, max(max(abs_bits(uv[c].x), abs_bits(uv[c].y)), max(abs_bits(uv[c].z), abs_bits(uv[c].w))));
    }
    const float sj = fv(wave_max_u32(am)) * kInv127, inv = sfu_recip(sj);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int i = c * 256 + lane * 4;
      if (i < F)
        *(int*)(hq + j * 1024 + i) = pack_i8x4(to_i8(uv[c].x * inv), to_i8(uv[c].y * inv), to_i8(uv[c].z * inv),
                                               to_i8(uv[c].w * inv));
    }
    if (lane == 0) s_h[j] = sj;
  }
  __syncthreads();
  if (!live) return;
  int acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int4 xq = (j < k && col < F) ? *(const int4*)(hq + j * 1024 + col) : make_int4(0, 0, 0, 0);
    acc[j] = dot16(wv[j], xq, 0);
  }
  // the 8 sums in one multi-value reduction: lane j (< 8) holds expert j's;
  // lane j: F(w_j * y_j), y_j the dequantised expert output; then the sum in route order
  const int aj = wave_sum_multi<8>(acc);
  const float t = lane < k ? wj * dequant(aj, swd, s_h[lane < k ? lane : 0]) : 0.0f;
  float y = 0.0f;
  for (int j = 0; j < k; ++j) y = y + __shfl(t, j);
  if (lane == 0) xr[n] = x_old + y;
}

// argmax of rows (first index of the largest value; NaN counts as the largest): one block per row
__global__ __launch_bounds__(256) void k_argmax(const float* x, int n, int32_t* idx) {
  __shared__ unsigned long long red[4];
  const int row = blockIdx.x;
  unsigned long long best = 0;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const unsigned long long kk = argmax_key(x[(long long)row * n + i], i);
    best = kk > best ? kk : best;
  }
  for (int o = 32; o > 0; o >>= 1) {
    const unsigned long long other = __shfl_xor(best, o);
    best = other > best ? other : best;
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long b = red[0];
    for (int w = 1; w < 4; ++w) b = red[w] > b ? red[w] : b;
    idx[row] = (int32_t)(0xFFFFFFFFu - (uint32_t)(b & 0xFFFFFFFFu));
  }
}

// End of a decode step: the greedy token from the argmax key; optionally pos += 1.
// positions start .. start + n - 1 (t2r_prefill_at)
__global__ __launch_bounds__(256) void k_iota(int32_t* out, int start, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = start + i;
}

// the greedy tokens of n rows from their argmax keys
__global__ void k_keys_tokens(const unsigned long long* key, int32_t* next_tokens, int n) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r < n) next_tokens[r] = (int32_t)(0xFFFFFFFFu - (uint32_t)(key[r] & 0xFFFFFFFFu));
}

__global__ void k_finish(const unsigned long long* key, int32_t* next_token, int32_t* pos, int advance) {
  if (threadIdx.x == 0) {
    if (next_token) *next_token = (int32_t)(0xFFFFFFFFu - (uint32_t)(*key & 0xFFFFFFFFu));
    if (advance) *pos = *pos + 1;
  }
}

// ---- test hooks: the SFU and the flush-to-zero primitives on bit patterns
// Every input in [first, first + count) through the datapath SFU and through the literal
// sequence (namespace seq): out[0] counts the inputs whose bits differ, out[1] keeps the smallest
// such input (initialised by k_sfu_check_init).
__global__ void k_sfu_check_init(uint32_t* out) {
  if (threadIdx.x == 0) {
    out[0] = 0;
    out[1] = 0xFFFFFFFFu;
  }
}
__global__ void k_sfu_check(int fn, unsigned long long first, unsigned long long count, uint32_t* out) {
  __shared__ float2 et[kSfuExpPairs], rt[64];
  if (threadIdx.x < kSfuExpPairs) et[threadIdx.x] = sfu_exp_pair(threadIdx.x, c_sfu);
  if (threadIdx.x < 64) rt[threadIdx.x] = sfu_recip_pair(threadIdx.x, c_sfu);
  __syncthreads();
  uint32_t bad = 0, lowest = 0xFFFFFFFFu;
  for (unsigned long long k = blockIdx.x * (unsigned long long)blockDim.x + threadIdx.x; k < count;
       k += (unsigned long long)gridDim.x * blockDim.x) {
    const uint32_t xb = (uint32_t)(first + k);
    const float v = fv(xb);
    uint32_t a, b;
    if (fn == 0) {
      a = fb(sfu_exp(v)); b = fb(seq::sfu_exp(v, c_sfu));
    } else if (fn == 3) {                       // the softmax form, on its domain (x <= 0, NaN)
      if (v > 0.0f) continue;
      a = fb(sfu_exp_np(v)); b = fb(seq::sfu_exp(v, c_sfu));
    } else if (fn == 5) {                       // the finite-maximum softmax form (x <= 0, not NaN)
      if (!(v <= 0.0f)) continue;
      a = fb(sfu_exp_sm(v, et)); b = fb(seq::sfu_exp(v, c_sfu));
    } else if (fn == 6) {                       // the gates' pair-table EXP (x not NaN)
      if (v != v) continue;
      a = fb(sfu_exp_g(v, et)); b = fb(seq::sfu_exp(v, c_sfu));
    } else if (fn == 7) {                       // the gates' pair-table RECIP (x >= 1 or +inf)
      if (!(v >= 1.0f)) continue;
      a = fb(sfu_recip_g1(v, rt)); b = fb(seq::sfu_recip(v, c_sfu));
    } else if (fn == 4) {                       // the gate form, on its domain (x >= 1, NaN)
      if (v < 1.0f) continue;
      a = fb(sfu_recip_ge1(v)); b = fb(seq::sfu_recip(v, c_sfu));
    } else if (fn == 1) {
      a = fb(sfu_recip(v)); b = fb(seq::sfu_recip(v, c_sfu));
    } else {
      a = fb(sfu_rsqrt(v)); b = fb(seq::sfu_rsqrt(v, c_sfu));
    }
    if (a != b) {
      ++bad;
      lowest = min(lowest, xb);
    }
  }
  if (bad) {
    atomicAdd(out, bad);
    atomicMin(out + 1, lowest);
  }
}

__global__ void k_sfu(int fn, const uint32_t* x, uint32_t* y, long long n) {
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x) {
    const float v = fv(x[i]);
    float r;
    switch (fn) {
      case 0: r = sfu_exp(v); break;
      case 1: r = sfu_recip(v); break;
      case 2: r = sfu_rsqrt(v); break;
      default: r = fv(x[i] & 0x7FFFFFFFu); break;
    }
    y[i] = fb(r);
  }
}

// op: 0 add, 1 sub, 2 mul, 3 ldexp (b = exponent as int32), 4 floor to int32, 5 to_i8, 6 from_int
// (a as int32), 7 IEEE mul (the vector-step multiply), 8 IEEE add
__global__ void k_fp32op(int op, const uint32_t* a, const uint32_t* b, uint32_t* y, long long n) {
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x) {
    const float x0 = ftz(fv(a[i])), x1 = ftz(fv(b[i]));
    uint32_t r;
    switch (op) {
      case 0: r = fb(fadd_ftz(x0, x1)); break;
      case 1: r = fb(fadd_ftz(x0, -x1)); break;
      case 2: r = fb(fmul_ftz(x0, x1)); break;
      case 3: r = fb(ldexp_ftz(x0, (int)b[i])); break;
      case 4: r = (uint32_t)floor_sat(x0); break;
      case 5: r = (uint32_t)to_i8(fv(a[i])); break;
      case 6: r = fb((float)(int)a[i]); break;
      case 7: r = fb(fv(a[i]) * fv(b[i])); break;
      default: r = fb(fv(a[i]) + fv(b[i])); break;
    }
    if (op <= 3 && (r & 0x7F800000u) == 0x7F800000u && (r & 0x7FFFFFu)) r = kQNaN;
    y[i] = r;
  }
}

// Integer REQUANT of the vector engine (llm/sa_funcsim.py:265-274):
// q = clamp(((r * scale + 2^(shift-1)) >> shift) + zp, lo, hi), saturated to int8.
__global__ void k_requant(const int32_t* r, long long n, int scale, int shift, int zp, int lo, int hi, int8_t* out) {
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x) {
    long long q = ((long long)r[i] * scale + (shift ? (1LL << (shift - 1)) : 0)) >> shift;
    q += zp;
    q = q < lo ? lo : (q > hi ? hi : q);
    q = q < -128 ? -128 : (q > 127 ? 127 : q);
    out[i] = (int8_t)q;
  }
}

}  // namespace t2r
