// Attention over the int8 KV cache, one workgroup per (KV head, query row): the KV head's G
// query heads share every K / V row it reads (grouped-query attention).
//
// Per query head h (llm/ref_model.py:230-243; QK-norm and q_dim != dim as
// compiler/frontend/qhf.py:304-353):
//   qq, s_q = quant_act(q_h)                                  int8 q per head
//   sc[t]   = F(F(f32(sum_j K[t, j] qq[j]) * s_q) * a_k)       exact int32 dot products
//   m = max(sc); e = EXP(F(sc - m)); r = RECIP(red_sum(e))     red_sum in the D-lane order
//   pq[t]   = to_i8(F(F(e[t] * r) * 127))                      int8 probabilities
//   att_h   = F(f32(sum_t pq[t] V[t, :]) * a_v)                exact int32 P.V
// The stages before it, per row at its position (llm/ref_model.py:224-229):
//   k, q: per-head RMSNorm (QK-norm models), RoPE on the interleaved pairs
//   kc[pos] = to_i8(F(k * (1/s_k))), vc[pos] = to_i8(F(v * (1/s_v)))
// Modes: ATTN_FUSED (decode: the stages, then attention; the new row is used from LDS),
// ATTN_PREP (prefill: the stages for every row, q rotated in place), ATTN_ONLY (prefill:
// attention of rows whose q is rotated and whose KV rows are all in the cache).
#pragma once
#include "t2r_device.h"

namespace t2r {

enum { ATTN_FUSED = 0, ATTN_PREP = 1, ATTN_ONLY = 2 };
constexpr int kAttnThreads = 256;
constexpr int kMaxG = 8;
constexpr int kMaxHd = 128;
constexpr int kMaxGS = 8192;          // G * S scores in LDS (32 KB), with the int8 probabilities 40 KB

struct AttnArgs {
  float* qkv;                // rows of [q | k | v] projections (stride qkv_stride)
  long long qkv_stride;
  int8_t* kc;                // this layer's K cache [S, kv_dim]
  int8_t* vc;                // this layer's V cache [S, kv_dim]
  const int32_t* pos;        // position of every row
  const float* qn;           // QK-norm gains [hd] (nullptr: no QK-norm)
  const float* kn;
  const float* cos_t;        // [S, hd / 2]
  const float* sin_t;
  float inv_sk, inv_sv, a_k, a_v, eps, inv_hd;
  int H, Hk, hd, D, S;
  float* att;                // [rows, q_dim] (stride att_stride)
  long long att_stride;
};

// RMSNorm (optional) and RoPE of one head vector v[0..hd) in LDS, by the threads of one wave
// (wave-local: lanes l < hd / 2 rotate pair l; D lanes run the ordered sum).
T2R_DEV void head_norm_rope(float* v, const float* gain, const AttnArgs& a, int pos, int lane) {
  const int hd = a.hd;
  if (gain != nullptr) {
    float ss = 0.0f;
    if (lane < a.D) ss = ordered_sum<true>(v, hd, a.D, lane);
    const float r = sfu_rsqrt(__shfl(ss, 0) * a.inv_hd + a.eps);
    float nv[2];
    for (int k = 0; k < 2; ++k) {
      const int j = lane + 64 * k;
      if (j < hd) nv[k] = (v[j] * r) * gain[j];
    }
    __builtin_amdgcn_wave_barrier();
    for (int k = 0; k < 2; ++k) {
      const int j = lane + 64 * k;
      if (j < hd) v[j] = nv[k];
    }
    __builtin_amdgcn_wave_barrier();
  }
  const float* cs = a.cos_t + (long long)pos * (hd / 2);
  const float* sn = a.sin_t + (long long)pos * (hd / 2);
  float o0 = 0.0f, o1 = 0.0f, o2 = 0.0f, o3 = 0.0f;
  const int i0 = lane, i1 = lane + 64;
  if (i0 < hd / 2) {
    const float v0 = v[2 * i0], v1 = v[2 * i0 + 1], c = cs[i0], s = sn[i0];
    o0 = (v0 * c) + ((-v1) * s);
    o1 = (v1 * c) + (v0 * s);
  }
  if (i1 < hd / 2) {
    const float v0 = v[2 * i1], v1 = v[2 * i1 + 1], c = cs[i1], s = sn[i1];
    o2 = (v0 * c) + ((-v1) * s);
    o3 = (v1 * c) + (v0 * s);
  }
  __builtin_amdgcn_wave_barrier();
  if (i0 < hd / 2) { v[2 * i0] = o0; v[2 * i0 + 1] = o1; }
  if (i1 < hd / 2) { v[2 * i1] = o2; v[2 * i1 + 1] = o3; }
  __builtin_amdgcn_wave_barrier();
}

template <int MODE>
__global__ __launch_bounds__(kAttnThreads) void k_attn(AttnArgs a) {
  extern __shared__ __align__(16) float dyn[];   // [G * S] scores / exps, then P.V partial sums
  __shared__ float s_q[kMaxG][kMaxHd];
  __shared__ float s_k[kMaxHd], s_v[kMaxHd];
  __shared__ int s_qq[kMaxG][kMaxHd / 4];
  __shared__ int s_kq[kMaxHd / 4], s_vq[kMaxHd / 4];
  __shared__ float s_sq[kMaxG], s_m[kMaxG], s_r[kMaxG];
  __shared__ float red[64];

  const int g = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int hd = a.hd, G = a.H / a.Hk, S = a.S;
  const int q_dim = a.H * hd, kv_dim = a.Hk * hd;
  const int pos = a.pos[row];
  if (pos < 0 || pos >= S) return;               // a position outside the cache: nothing is read or written
  const int T = pos + 1;
  float* qkv = a.qkv + row * a.qkv_stride;

  // ---- the row's k / v: norm, RoPE, int8, append to the cache
  if (MODE != ATTN_ONLY) {
    for (int j = tid; j < hd; j += kAttnThreads) {
      s_k[j] = qkv[q_dim + g * hd + j];
      s_v[j] = qkv[q_dim + kv_dim + g * hd + j];
    }
    __syncthreads();
    if (wave == 0) head_norm_rope(s_k, a.kn, a, pos, lane);
    __syncthreads();
    for (int j = tid; j < hd / 4; j += kAttnThreads) {
      int k4[4], v4[4];
      for (int b = 0; b < 4; ++b) {
        k4[b] = to_i8(s_k[4 * j + b] * a.inv_sk);
        v4[b] = to_i8(s_v[4 * j + b] * a.inv_sv);
      }
      const int kw = pack_i8x4(k4[0], k4[1], k4[2], k4[3]), vw = pack_i8x4(v4[0], v4[1], v4[2], v4[3]);
      s_kq[j] = kw;
      s_vq[j] = vw;
      *(int*)(a.kc + (long long)pos * kv_dim + g * hd + 4 * j) = kw;
      *(int*)(a.vc + (long long)pos * kv_dim + g * hd + 4 * j) = vw;
    }
  }
  // ---- the group's query heads
  for (int i = tid; i < G * hd; i += kAttnThreads) s_q[i / hd][i % hd] = qkv[(g * G + i / hd) * hd + i % hd];
  __syncthreads();
  if (MODE != ATTN_ONLY) {
    for (int hh = wave; hh < G; hh += kAttnThreads / 64) head_norm_rope(s_q[hh], a.qn, a, pos, lane);
    __syncthreads();
    if (MODE == ATTN_PREP) {
      for (int i = tid; i < G * hd; i += kAttnThreads) qkv[(g * G + i / hd) * hd + i % hd] = s_q[i / hd][i % hd];
      return;
    }
  }
  // quant_act per head (one wave per head)
  for (int hh = wave; hh < G; hh += kAttnThreads / 64) {
    float m = 0.0f;
    for (int j = lane; j < hd; j += 64) m = nanmax(m, fabsf(s_q[hh][j]));
    m = wave_max(m);
    const float sq = m * kInv127;
    const float inv = sfu_recip(sq);
    for (int j = lane; j < hd / 4; j += 64) {
      const float* q = &s_q[hh][4 * j];
      s_qq[hh][j] = pack_i8x4(to_i8(q[0] * inv), to_i8(q[1] * inv), to_i8(q[2] * inv), to_i8(q[3] * inv));
    }
    if (lane == 0) s_sq[hh] = sq;
  }
  __syncthreads();

  // ---- scores: one thread per cache row
  float* sc = dyn;                                   // [G][S]
  const int nw = hd / 4;
  for (int t = tid; t < T; t += kAttnThreads) {
    int dots[kMaxG];
    for (int hh = 0; hh < G; ++hh) dots[hh] = 0;
    const bool fresh = MODE == ATTN_FUSED && t == pos;
    const int8_t* krow = a.kc + (long long)t * kv_dim + g * hd;
    for (int w = 0; w < nw; w += 4) {
      int kw[4];
      if (fresh) {
        for (int b = 0; b < 4; ++b) kw[b] = w + b < nw ? s_kq[w + b] : 0;
      } else if (w + 4 <= nw) {
        const int4 k4 = *(const int4*)(krow + 4 * w);
        kw[0] = k4.x; kw[1] = k4.y; kw[2] = k4.z; kw[3] = k4.w;
      } else {
        for (int b = 0; b < 4; ++b) kw[b] = w + b < nw ? *(const int*)(krow + 4 * (w + b)) : 0;
      }
      for (int hh = 0; hh < G; ++hh)
        for (int b = 0; b < 4; ++b)
          if (w + b < nw) dots[hh] = __builtin_amdgcn_sdot4(kw[b], s_qq[hh][w + b], dots[hh], false);
    }
    for (int hh = 0; hh < G; ++hh) sc[hh * S + t] = ((float)dots[hh] * s_sq[hh]) * a.a_k;
  }
  __syncthreads();
  // max per head (order-free), then EXP
  for (int hh = 0; hh < G; ++hh) {
    float m = -__builtin_inff();
    for (int t = tid; t < T; t += kAttnThreads) m = nanmax(m, sc[hh * S + t]);
    m = block_max(m, red);
    if (tid == 0) s_m[hh] = m;
  }
  __syncthreads();
  for (int i = tid; i < G * T; i += kAttnThreads) {
    const int hh = i / T, t = i % T;
    sc[hh * S + t] = sfu_exp(sc[hh * S + t] - s_m[hh]);
  }
  __syncthreads();
  // the ordered sum of e per head (D lanes of one wave each), RECIP
  for (int hh = wave; hh < G; hh += kAttnThreads / 64) {
    if (lane < a.D) {
      const float s = ordered_sum<false>(sc + hh * S, T, a.D, lane);
      if (lane == 0) s_r[hh] = sfu_recip(s);
    }
  }
  __syncthreads();
  // int8 probabilities
  int8_t* pq = (int8_t*)(dyn + (G * S > 1024 * G ? G * S : 1024 * G));   // [G][S]
  for (int i = tid; i < G * T; i += kAttnThreads) {
    const int hh = i / T, t = i % T;
    pq[hh * S + t] = (int8_t)to_i8((sc[hh * S + t] * s_r[hh]) * 127.0f);
  }
  __syncthreads();
  // ---- P.V: thread = (column word cw, row slice ts); exact int32 partial sums, then a sum over slices
  const int CW = nw, TS = kAttnThreads / CW;
  const int cw = tid % CW, ts = tid / CW;
  int acc[kMaxG][4];
  for (int hh = 0; hh < G; ++hh)
    for (int b = 0; b < 4; ++b) acc[hh][b] = 0;
  if (ts < TS) {
    for (int t = ts; t < T; t += TS) {
      const int vw = (MODE == ATTN_FUSED && t == pos) ? s_vq[cw] : *(const int*)(a.vc + (long long)t * kv_dim + g * hd + 4 * cw);
      const int v0 = (int)(int8_t)(vw & 0xFF), v1 = (int)(int8_t)((vw >> 8) & 0xFF);
      const int v2 = (int)(int8_t)((vw >> 16) & 0xFF), v3 = vw >> 24;
      for (int hh = 0; hh < G; ++hh) {
        const int p = pq[hh * S + t];
        acc[hh][0] += p * v0;
        acc[hh][1] += p * v1;
        acc[hh][2] += p * v2;
        acc[hh][3] += p * v3;
      }
    }
  }
  __syncthreads();                                   // sc is dead: reuse it for the partial sums
  int* part = (int*)dyn;                             // [TS][G][hd]
  if (ts < TS)
    for (int hh = 0; hh < G; ++hh)
      for (int b = 0; b < 4; ++b) part[(ts * G + hh) * hd + 4 * cw + b] = acc[hh][b];
  __syncthreads();
  float* out = a.att + row * a.att_stride;
  for (int i = tid; i < G * hd; i += kAttnThreads) {
    const int hh = i / hd, j = i % hd;
    int s = 0;
    for (int k = 0; k < TS; ++k) s += part[(k * G + hh) * hd + j];
    out[(g * G + hh) * hd + j] = (float)s * a.a_v;
  }
}

// dynamic LDS bytes of k_attn
inline size_t attn_lds_bytes(int G, int S) {
  const size_t f = (size_t)(G * S > 1024 * G ? G * S : 1024 * G);
  return f * 4 + (size_t)G * S;
}

}  // namespace t2r
