// Attention over the int8 KV cache, one 512-thread workgroup per (query head, query row).
//
// Per query head h with KV head g = h / G (llm/ref_model.py:230-243; QK-norm and q_dim != dim as
// compiler/frontend/qhf.py:304-353):
//   qq, s_q = quant_act(q_h)                                  int8 q per head
//   sc[t]   = F(F(f32(sum_j K[t, j] qq[j]) * s_q) * a_k)       exact int32 dot products
//   m = max(sc); e = EXP(F(sc - m)); r = RECIP(red_sum(e))     red_sum in the D-lane order
//   pq[t]   = to_i8(F(F(e[t] * r) * 127))                      int8 probabilities
//   att_h   = F(f32(sum_t pq[t] V[t, :]) * a_v)                exact int32 P.V (any summation order)
// The stages before it, per row at its position (llm/ref_model.py:224-229):
//   k, q: per-head RMSNorm (QK-norm models), RoPE on the interleaved pairs
//   kc[pos] = to_i8(F(k * (1/s_k))), vc[pos] = to_i8(F(v * (1/s_v)))
// Every workgroup of a KV head's group computes that head's new row (identical bits); the first
// one of the group writes it to the cache, and each uses it from LDS, so no workgroup reads a
// row another one writes.
// Modes: ATTN_FUSED (decode: the stages, then attention), ATTN_PREP (prefill: the stages for every
// row, q rotated in place: k_attn_prep), ATTN_ONLY (prefill: attention of rows whose q is rotated
// and whose KV rows are all in the cache).
// The HF path's options (compiler/frontend/hf_generic.py:153-187, 265-292), off by default:
//   qsum:          pq[t] = to_i8(F(e[t] * 127)), att_h = F(F(f32(sum_t pq V) * rq) * a_v) with
//                  rq = F(RECIP(f32(sum_t pq[t])) * 127) (an exact integer sum)
//   K per channel: q = F(q * s_k[c]) before its quant_act; kc = to_i8(F(k * inv_sk[c]))
//   V per channel: vc = to_i8(F(v * inv_sv[c])); att = F(... * a_v[c]) per output channel
// (channel c = g hd + j of the cache row). The specialised kernels take them in a separate
// instantiation (template flag OPT), so the default one is unchanged.
#pragma once
#include "t2r_device.h"

namespace t2r {

enum { ATTN_FUSED = 0, ATTN_PREP = 1, ATTN_ONLY = 2 };
constexpr int kAttnThreads = 512;
constexpr int kAttnWaves = kAttnThreads / 64;
constexpr int kMaxG = 8;
constexpr int kMaxHd = 128;
constexpr int kMaxS = 8192;           // cache rows: scores and int8 probabilities in LDS (40 KB)

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
  const float* tab;          // the SFU tables in device memory (k_attn_dec)
  long long kv_row_stride;   // bytes between the caches of consecutive rows (batched decode: one
                             // sequence per row); 0: every row uses the one cache (prefill rows)
  int t_cap;                 // prefill attention: every row attends to <= t_cap positions (sizes the
                             // score rows in LDS); 0: S
  // k_attn_prep: the Wqkv linear's split-K partials [part_nz, rows, qkv_stride] when part_nz > 1
  // (then column c of a row is F(F(f32(sum_z part) * part_sw[c]) * part_sx[row]), the store
  // epilogue, instead of qkv[c])
  const int32_t* part;
  long long part_zstride;
  int part_nz;
  const float* part_sw;
  const float* part_sx;
  // the HF path's options (see above); nullptr / 0: off
  int qsum;
  const float* ch_sk;        // K per channel [kv_dim]: the q multiplier s_k
  const float* ch_isk;       //   and 1 / s_k for the cache row
  const float* ch_isv;       // V per channel [kv_dim]: 1 / s_v for the cache row
  const float* ch_av;        //   and a_v per output channel
  // batch-1 decode with a head's keys split over nsplit workgroups (grid y; k_attn_dec's SPLIT forms,
  // nsplit > 1): the scores published [H, S]; SPLIT 2's per-split int32 P.V sums [nsplit, H HD] for
  // the next linear's prologue (written and read within one step); SPLIT 1's P.V sums met as
  // [H, kMaxHd] (zero between launches); per head two counters [H, 2]: the arrivals (every launch
  // adds nsplit, so a launch's target is the next multiple of nsplit: never cleared) and SPLIT 1's
  // finish count (zero between launches)
  float* sp_s;
  int32_t* sp_o;
  int32_t* sp_acc;
  uint32_t* sp_sync;
  int nsplit;
  // the model's status word (nullptr: none): bit 1 a split's bounded wait ran out, bit 2 a row's
  // position was outside the cache (the row is then neither read nor written)
  int32_t* status;
  // prefill at head dims 64 / 128: the prep kernels' quant_act of each q head vector, the int8 rows
  // [rows, q8_stride] and the scales [rows, H], written instead of the fp32 q and read by the
  // 32-row attention (k_attn_pw's Q8I form); nullptr: q stays fp32 in qkv
  int8_t* q8;
  long long q8_stride;
  float* q8s;
};

// a row whose position is outside the cache: its kernels end at once and flag it (bit 2)
T2R_DEV void flag_bad_pos(int32_t* status) {
  if (status) atomicOr(status, 4);
}

// Every vector memory operation of this wave (the stores and atomics that a release by another wave
// of the workgroup is about to publish) completed before the wave passes on: a release at agent
// scope waits only for its own wave's operations. The fence keeps the compiler from moving this
// wave's accesses past the wait.
T2R_DEV void wave_mem_done() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_s_waitcnt(0x0F70);           // vmcnt(0): gfx9 encoding, expcnt / lgkmcnt untouched
}

// A bounded wait for *p to reach want (modulo 2^32) at device scope (one lane polls); on running out
// it sets bit 1 of *status and returns, so every workgroup reaches its end whatever happens.
T2R_DEV void split_wait(uint32_t* p, uint32_t want, int32_t* status) {
  for (int it = 0; it < (1 << 20); ++it) {
    if ((int32_t)(__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - want) >= 0) {
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      return;
    }
    __builtin_amdgcn_s_sleep(2);
  }
  if (status) atomicOr(status, 2);
}

inline bool attn_opt(const AttnArgs& a) { return a.qsum || a.ch_sk || a.ch_isk || a.ch_isv || a.ch_av; }

// qsum's output scale rq = F(RECIP(f32(sum of the int8 probabilities)) * 127)
T2R_DEV float qsum_scale(int sum, const float* tab) { return sfu_recip((float)sum, tab) * 127.0f; }

// The per-lane operands of head_norm_rope, loadable before the head vector is: the norm gains of
// elements lane + 64 k and the RoPE cos / sin of pairs lane + 64 k at the row's position (0 past
// the vector).
struct NormRopeOps {
  float g[2], c[2], s[2];
};
T2R_DEV NormRopeOps norm_rope_ops(const float* gain, const AttnArgs& a, int pos, int lane) {
  NormRopeOps o;
  const int hd = a.hd;
  const float* cs = a.cos_t + (long long)pos * (hd / 2);
  const float* sn = a.sin_t + (long long)pos * (hd / 2);
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int j = lane + 64 * k;
    o.g[k] = gain != nullptr && j < hd ? gain[j] : 0.0f;
    o.c[k] = j < hd / 2 ? cs[j] : 0.0f;
    o.s[k] = j < hd / 2 ? sn[j] : 0.0f;
  }
  return o;
}

// RMSNorm (optional) and RoPE of one head vector v[0..hd) in LDS, by one wave.
T2R_DEV void head_norm_rope(float* v, bool norm, const NormRopeOps& p, const AttnArgs& a, int lane) {
  const int hd = a.hd;
  if (norm) {
    float ss = 0.0f;
    if (lane < a.D) ss = ordered_sum<true>(v, hd, a.D, lane);
    const float r = sfu_rsqrt(__shfl(ss, 0) * a.inv_hd + a.eps);
    float nv[2];
    for (int k = 0; k < 2; ++k) {
      const int j = lane + 64 * k;
      if (j < hd) nv[k] = (v[j] * r) * p.g[k];
    }
    __builtin_amdgcn_wave_barrier();
    for (int k = 0; k < 2; ++k) {
      const int j = lane + 64 * k;
      if (j < hd) v[j] = nv[k];
    }
    __builtin_amdgcn_wave_barrier();
  }
  float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int k = 0; k < 2; ++k) {
    const int i = lane + 64 * k;
    if (i < hd / 2) {
      const float v0 = v[2 * i], v1 = v[2 * i + 1], c = p.c[k], s = p.s[k];
      o[2 * k] = (v0 * c) + ((-v1) * s);
      o[2 * k + 1] = (v1 * c) + (v0 * s);
    }
  }
  __builtin_amdgcn_wave_barrier();
  for (int k = 0; k < 2; ++k) {
    const int i = lane + 64 * k;
    if (i < hd / 2) {
      v[2 * i] = o[2 * k];
      v[2 * i + 1] = o[2 * k + 1];
    }
  }
  __builtin_amdgcn_wave_barrier();
}
T2R_DEV void head_norm_rope(float* v, const float* gain, const AttnArgs& a, int pos, int lane) {
  head_norm_rope(v, gain != nullptr, norm_rope_ops(gain, a, pos, lane), a, lane);
}

// 8 or 16 int8 of a cache row as int32 words (hd % 16 == 0: one 16-byte load)
template <int CB>
T2R_DEV void load_chunk(const int8_t* p, int* w) {
  if (CB == 16) {
    const int4 v = *(const int4*)p;
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else {
    const int2 v = *(const int2*)p;
    w[0] = v.x; w[1] = v.y;
  }
}

T2R_DEV int sext8(int w, int b) { return (int)(int8_t)((w >> (8 * b)) & 0xFF); }

// CB: bytes per cache-row chunk a thread handles (16 when hd % 16 == 0, else 8)
template <int MODE, int CB>
__global__ __launch_bounds__(kAttnThreads) void k_attn(AttnArgs a) {
  extern __shared__ __align__(16) float dyn[];   // sc[S] scores / exps, then pq[S] int8
  __shared__ float s_q[kMaxHd], s_k[kMaxHd], s_v[kMaxHd];
  __shared__ int s_qq[kMaxHd / 4], s_kq[kMaxHd / 4], s_vq[kMaxHd / 4];
  __shared__ int part[kAttnWaves][kMaxHd];
  __shared__ float red[64];
  __shared__ float s_sq, s_r;
  __shared__ int s_qs[kAttnWaves];

  const int h = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int hd = a.hd, G = a.H / a.Hk, S = a.S, g = h / G;
  const int q_dim = a.H * hd, kv_dim = a.Hk * hd;
  a.kc += row * a.kv_row_stride;                 // this row's sequence cache
  a.vc += row * a.kv_row_stride;
  const int pos = a.pos[row];
  if (pos < 0 || pos >= S) {                     // a position outside the cache: nothing is read or written
    if (tid == 0) flag_bad_pos(a.status);
    return;
  }
  const int T = pos + 1;
  float* qkv = a.qkv + row * a.qkv_stride;
  constexpr int CW = CB / 4;                     // int32 words per chunk

  // ---- the row's k / v (wave 0) and this head's q (wave 1): norm, RoPE; k / v to int8
  if (MODE != ATTN_ONLY && wave == 0) {
    for (int j = lane; j < hd; j += 64) {
      s_k[j] = qkv[q_dim + g * hd + j];
      s_v[j] = qkv[q_dim + kv_dim + g * hd + j];
    }
    __builtin_amdgcn_wave_barrier();
    head_norm_rope(s_k, a.kn, a, pos, lane);
    for (int j = lane; j < hd / 4; j += 64) {
      int k4[4], v4[4];
      for (int b = 0; b < 4; ++b) {
        const int ch = g * hd + 4 * j + b;
        k4[b] = to_i8(s_k[4 * j + b] * (a.ch_isk ? a.ch_isk[ch] : a.inv_sk));
        v4[b] = to_i8(s_v[4 * j + b] * (a.ch_isv ? a.ch_isv[ch] : a.inv_sv));
      }
      const int kw = pack_i8x4(k4[0], k4[1], k4[2], k4[3]), vw = pack_i8x4(v4[0], v4[1], v4[2], v4[3]);
      s_kq[j] = kw;
      s_vq[j] = vw;
      if (h % G == 0) {
        *(int*)(a.kc + (long long)pos * kv_dim + g * hd + 4 * j) = kw;
        *(int*)(a.vc + (long long)pos * kv_dim + g * hd + 4 * j) = vw;
      }
    }
  }
  if (wave == 1) {
    for (int j = lane; j < hd; j += 64) s_q[j] = qkv[h * hd + j];
    __builtin_amdgcn_wave_barrier();
    if (MODE != ATTN_ONLY) head_norm_rope(s_q, a.qn, a, pos, lane);
    if (a.ch_sk) {                               // K per channel: its scales folded into q
      for (int j = lane; j < hd; j += 64) s_q[j] = s_q[j] * a.ch_sk[g * hd + j];
      __builtin_amdgcn_wave_barrier();
    }
    // quant_act of the head
    float m = 0.0f;
    for (int j = lane; j < hd; j += 64) m = nanmax(m, fabsf(s_q[j]));
    m = wave_max(m);
    const float sq = m * kInv127;
    const float inv = sfu_recip(sq);
    for (int j = lane; j < hd / 4; j += 64)
      s_qq[j] = pack_i8x4(to_i8(s_q[4 * j] * inv), to_i8(s_q[4 * j + 1] * inv), to_i8(s_q[4 * j + 2] * inv),
                          to_i8(s_q[4 * j + 3] * inv));
    if (lane == 0) s_sq = sq;
  }
  __syncthreads();

  // ---- scores: one thread per cache row, the row in chunks of CB bytes. sc is kept in the
  // lane-major layout of the ordered sum (row t at osum_index(t)).
  float* sc = dyn;
  const int D = a.D, P = osum_stride(S, D);
  const int nch = hd / CB;
  const int8_t* kbase = a.kc + g * hd;
  const float sq = s_sq;
  float mloc = -__builtin_inff();
  for (int t = tid; t < T; t += kAttnThreads) {
    int dot = 0;
    if (MODE == ATTN_FUSED && t == pos) {
      for (int w = 0; w < hd / 4; ++w) dot = __builtin_amdgcn_sdot4(s_kq[w], s_qq[w], dot, false);
    } else {
      const int8_t* kr = kbase + (long long)t * kv_dim;
      int kw[kMaxHd / 4];
#pragma unroll
      for (int c = 0; c < kMaxHd / CB; ++c)
        if (c < nch) load_chunk<CB>(kr + c * CB, kw + c * CW);
#pragma unroll
      for (int w = 0; w < kMaxHd / 4; ++w)
        if (w < hd / 4) dot = __builtin_amdgcn_sdot4(kw[w], s_qq[w], dot, false);
    }
    const float s = ((float)dot * sq) * a.a_k;
    sc[osum_index(t, D, P)] = s;
    mloc = nanmax(mloc, s);
  }
  const float m = block_max(mloc, red);
  const int Tpad = ((T + D - 1) / D) * D;
  for (int t = tid; t < Tpad; t += kAttnThreads) {
    const int i = osum_index(t, D, P);
    sc[i] = t < T ? sfu_exp_np(sc[i] - m) : 0.0f;
  }
  __syncthreads();
  if (wave == 0) {
    float s = 0.0f;
    if (lane < D) s = ordered_sum_t<false>(sc, T, D, P, lane);
    s = __shfl(s, 0);
    if (lane == 0) s_r = a.qsum ? 1.0f : sfu_recip(s);   // qsum: pq = to_i8(F(F(e * 1) * 127)), e * 1 = e
  }
  __syncthreads();
  int8_t* pq = (int8_t*)(dyn + D * P);
  const float r = s_r;
  int qs = 0;
  for (int t = tid; t < T; t += kAttnThreads) {
    const int p = to_i8((sc[osum_index(t, D, P)] * r) * 127.0f);
    pq[t] = (int8_t)p;
    qs += p;
  }
  if (a.qsum) {
    qs = wave_sum_i32(qs);
    if (lane == 0) s_qs[wave] = qs;
  }
  __syncthreads();

  // ---- P.V: thread = (chunk slot c of CB columns, row slice ts); int32 partial sums, 4 rows in flight.
  // Chunk slots are padded to a power of two (NCHP) so that the lanes of one chunk are an xor class.
  const int NCH = hd / CB;                       // chunks per row
  int NCHP = 1;
  while (NCHP < NCH) NCHP <<= 1;
  const int TS = kAttnThreads / NCHP;
  const int c = tid & (NCHP - 1), ts = tid / NCHP;
  int acc[CB];
#pragma unroll
  for (int b = 0; b < CB; ++b) acc[b] = 0;
  if (c < NCH) {
    const int8_t* vbase = a.vc + g * hd + c * CB;
    int t = ts;
    for (; t + 3 * TS < T; t += 4 * TS) {
      int vw[4][CW];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int tt = t + u * TS;
        if (MODE == ATTN_FUSED && tt == pos) {
          for (int w = 0; w < CW; ++w) vw[u][w] = s_vq[c * CW + w];
        } else {
          load_chunk<CB>(vbase + (long long)tt * kv_dim, vw[u]);
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int p = pq[t + u * TS];
#pragma unroll
        for (int w = 0; w < CW; ++w)
#pragma unroll
          for (int b = 0; b < 4; ++b) acc[4 * w + b] += p * sext8(vw[u][w], b);
      }
    }
    for (; t < T; t += TS) {
      int vw[CW];
      if (MODE == ATTN_FUSED && t == pos) {
        for (int w = 0; w < CW; ++w) vw[w] = s_vq[c * CW + w];
      } else {
        load_chunk<CB>(vbase + (long long)t * kv_dim, vw);
      }
      const int p = pq[t];
#pragma unroll
      for (int w = 0; w < CW; ++w)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[4 * w + b] += p * sext8(vw[w], b);
    }
  }
  // lanes of a wave with the same chunk: xor-shuffle over the row-slice bits, then one partial per wave
  for (int o = NCHP; o < 64; o <<= 1)
#pragma unroll
    for (int b = 0; b < CB; ++b) acc[b] += __shfl_xor(acc[b], o);
  if (lane < NCH)
    for (int b = 0; b < CB; ++b) part[wave][lane * CB + b] = acc[b];
  __syncthreads();
  float* out = a.att + row * a.att_stride;
  float rq = 1.0f;
  if (a.qsum) {
    int tot = 0;
    for (int w = 0; w < kAttnWaves; ++w) tot += s_qs[w];
    rq = qsum_scale(tot, c_sfu);
  }
  for (int j = tid; j < hd; j += kAttnThreads) {
    int s = 0;
    for (int w = 0; w < kAttnWaves; ++w) s += part[w][j];
    float o = (float)s;
    if (a.qsum) o = o * rq;
    out[h * hd + j] = o * (a.ch_av ? a.ch_av[g * hd + j] : a.a_v);
  }
}

// ------------------------------------------------------------------ decode attention
// Same numerics as k_attn<ATTN_FUSED>, organised around memory latency and instruction count.
// Every thread owns one 16-byte chunk (slot c of the NCHP slots per row) of R rows
// t = ts + TS i, for both K and V. The position is requested first and with it what does not
// depend on it (the SFU tables, the row's k / v or q, the norm gains); the RoPE inputs and the K and
// V chunks follow once it has arrived. K and V go through buffer loads whose range ends at row pos: rows past it read as zero
// without a memory access, so the loads stay unconditional (exact in-order wait counts) and cost
// nothing when the sequence is short. Per row, the slot lanes' partial dot products meet by DPP.
// Each lane exps one row in NCHP; the exps go to the lane-major copy for the D-lane ordered sum,
// and are read back from it. P.V packs four rows' int8 probabilities into one word and the V
// chunks, transposed 4 x 4 bytes with v_perm, into words of four rows: one v_dot4 per column per
// four rows.
T2R_DEV __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// the same from wave-uniform inputs, taken from the first lane: a descriptor must sit in scalar
// registers, and one built from a uniform value that the compiler keeps in vector registers turns
// every load through it into a waterfall loop
T2R_DEV __amdgpu_buffer_rsrc_t buffer_rsrc_u(const void* base, uint32_t bytes) {
  const uint64_t p = (uint64_t)base;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)p);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(p >> 32));
  return buffer_rsrc((const void*)(((uint64_t)hi << 32) | lo), (uint32_t)__builtin_amdgcn_readfirstlane((int)bytes));
}
T2R_DEV v4i_t buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

// 4 x 4 byte transpose: in r0..r3 (four rows, four columns each), out k = column k of the four rows
T2R_DEV void transpose4x4(int r0, int r1, int r2, int r3, int* out) {
  const int a = __builtin_amdgcn_perm(r1, r0, 0x05010400);   // r0.b0 r1.b0 r0.b1 r1.b1
  const int b = __builtin_amdgcn_perm(r1, r0, 0x07030602);   // r0.b2 r1.b2 r0.b3 r1.b3
  const int c = __builtin_amdgcn_perm(r3, r2, 0x05010400);
  const int d = __builtin_amdgcn_perm(r3, r2, 0x07030602);
  out[0] = __builtin_amdgcn_perm(c, a, 0x05040100);          // a.b0 a.b1 c.b0 c.b1
  out[1] = __builtin_amdgcn_perm(c, a, 0x07060302);          // a.b2 a.b3 c.b2 c.b3
  out[2] = __builtin_amdgcn_perm(d, b, 0x05040100);
  out[3] = __builtin_amdgcn_perm(d, b, 0x07060302);
}

// sum over the NCHP lanes of a slot group (consecutive lanes)
template <int NCHP>
T2R_DEV int slot_group_sum(int v) {
  if (NCHP >= 2) v += dpp_i<kDppXor1>(v);
  if (NCHP >= 4) v += dpp_i<kDppXor2>(v);
  if (NCHP >= 8) v += dpp_i<kDppHalfMirror>(v);
  return v;
}

// SPLIT (batch-1 decode of long caches): grid y splits a head's keys, workgroup j taking passes
// j, j + n, ... (n = min(nsplit, passes); the others end at once). One CU streams a head's K and V
// at most ~95 GB/s (522 KB at head dim 128 and T = 2048), so more CUs per head shorten that part.
// Each split publishes its scores with device-coherent stores and arrives once; after one bounded
// wait every split reads all T scores and forms the max, the EXPs, the ordered sum and RECIP itself
// (the same bits in each), then the probabilities and P.V of its own passes. The splits past the
// passes arrive too, so each launch adds exactly nsplit arrivals and waits for the next multiple.
// SPLIT 1: the P.V sums meet as exact int32 device atomics, and the head's last split to finish
// writes the output and clears the sums and its counter for the next launch. SPLIT 2 (no HF
// options): each split stores its own int32 sums (splits past the passes store zeros) and the next
// linear's prologue adds the four and scales them (F(f32(sum) a_v), the output's own formula).
template <int NCH, bool OPT = false, int SPLIT = 0>   // 16-byte chunks per head row: hd = 16 NCH; OPT: the HF options
__global__ __launch_bounds__(kAttnThreads) void k_attn_dec(AttnArgs a) {
  constexpr int HD = 16 * NCH;
  constexpr int NCHP = NCH <= 1 ? 1 : (NCH <= 2 ? 2 : (NCH <= 4 ? 4 : 8));
  constexpr int TS = kAttnThreads / NCHP;                   // row slices
  // rows per thread per pass (R % 4 == 0): 8 keeps the unconditional loads cheap (each costs the
  // CU's load pipeline ~16 clocks whether or not its rows exist); longer contexts take more passes
  constexpr int R = 8;
  constexpr int NV = HD > 64 ? 2 : 1;                       // head-vector floats per lane
  extern __shared__ __align__(16) float dyn[];              // sc (lane-major)
  __shared__ __align__(16) float tab[kSfuWords];
  __shared__ __align__(16) float s_k[HD], s_q[HD], s_v[HD];
  __shared__ __align__(16) int s_qq[HD / 4], s_kq[HD / 4], s_vq[HD / 4];
  __shared__ int part[kAttnWaves * 4][HD];
  __shared__ float red[16];
  __shared__ float s_sq, s_r;
  __shared__ int s_qs[kAttnWaves];
  __shared__ int s_last;

  const int h = blockIdx.x, row = SPLIT ? 0 : blockIdx.y, tid = threadIdx.x;
  const int sj = SPLIT ? blockIdx.y : 0;         // this workgroup's split
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // (uniform: scalar selects by wave)
  const int G = a.H / a.Hk, g = h / G, S = a.S;
  a.kc += row * a.kv_row_stride;                 // this row's sequence cache
  a.vc += row * a.kv_row_stride;
  const long long q_dim = (long long)a.H * HD;
  const int kv_dim = a.Hk * HD;
  // ---- issue: the position, then what does not depend on it (SFU tables, head vectors, gains), then
  // the RoPE rows and K chunks at the position. The position comes by a vector load, counted in order
  // with the loads after it, so that waiting for it waits for nothing issued later; the loads before
  // that wait are unconditional and no branch precedes it in the default kernels (a branch lets the
  // compiler sink them below the wait). A position outside the cache runs as position 0 and writes
  // nothing: no cache row, no output (SPLIT 2: no sums; SPLIT 1 clears its sums as after any launch),
  // the status bit at the end.
  const int pos_v = (int)__builtin_amdgcn_raw_buffer_load_b32(buffer_rsrc_u(a.pos + row, 4), 0, 0, 0);
  const float* qkv = a.qkv + row * a.qkv_stride;
  v4f_t tb[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) tb[k] = ((const v4f_t*)a.tab)[(lane + 64 * k) & (kSfuWords / 4 - 1)];
  const float* va = wave == 0 ? qkv + q_dim + (long long)g * HD : qkv + (long long)h * HD;
  const float* vb = wave == 0 ? qkv + q_dim + kv_dim + (long long)g * HD : va;
  const float* gn = wave == 0 ? a.kn : a.qn;
  const bool norm = gn != nullptr;
  if (!norm) gn = va;                            // any readable address: the values are unused
  float xa[NV], xb[NV], xg[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int j = min(lane + 64 * k, HD - 1);
    xa[k] = va[j];
    xb[k] = vb[j];
    xg[k] = gn[j];
  }
  // OPT: per-channel scales of this KV head (wave 0: 1 / s_k, 1 / s_v; wave 1: the q multiplier s_k),
  // loaded unconditionally from a readable address when absent
  float xc1[NV], xc2[NV];
  if constexpr (OPT) {
    const float* c1 = wave == 0 ? a.ch_isk : a.ch_sk;
    c1 = c1 ? c1 + (long long)g * HD : va;
    const float* c2 = wave == 0 && a.ch_isv ? a.ch_isv + (long long)g * HD : va;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int j = min(lane + 64 * k, HD - 1);
      xc1[k] = c1[j];
      xc2[k] = c2[j];
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  const int pos_in = __builtin_amdgcn_readfirstlane(pos_v);
  const bool pos_ok = pos_in >= 0 && pos_in < S;
  const int pos = pos_ok ? pos_in : 0;
  const int T = pos + 1;
  const int nsp = SPLIT ? min(a.nsplit, (T + TS * R - 1) / (TS * R)) : 1;   // splits with passes
  const int c = tid & (NCHP - 1), ts = tid / NCHP;
  const bool cok = c < NCH;
  // cache rows [0, pos): byte range of this KV head's columns up to row pos
  const __amdgpu_buffer_rsrc_t krs = buffer_rsrc_u(a.kc + (long long)g * HD, (uint32_t)pos * kv_dim);
  const __amdgpu_buffer_rsrc_t vrs = buffer_rsrc_u(a.vc + (long long)g * HD, (uint32_t)pos * kv_dim);
  auto chunk_off = [&](int t) -> uint32_t { return cok ? (uint32_t)t * kv_dim + 16 * c : 0xFFFFFFF0u; };
  float cs[NV], sn[NV];                          // RoPE of element j = lane + 64 k: pair j / 2
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const long long ip = (long long)pos * (HD / 2) + min((lane + 64 * k) >> 1, HD / 2 - 1);
    cs[k] = a.cos_t[ip];
    sn[k] = a.sin_t[ip];
  }
  __builtin_amdgcn_sched_barrier(0);
  // unconditional: a branch around a load would make the compiler's wait counts path-dependent
  // (it then waits for every later load too); rows past pos read as zero
  // (the V rows follow after the first barrier: nothing before P.V needs them, and the barriers up to
  // P.V order LDS only, so they stay in flight meanwhile)
  v4i_t kw[R], vw[R];
#pragma unroll
  for (int i = 0; i < R; ++i) kw[i] = buffer_load16(krs, chunk_off(sj * TS * R + ts + TS * i));
  __builtin_amdgcn_sched_barrier(0);

  // ---- tables to LDS; wave 0: k (norm, RoPE), k / v to int8 (+ cache row); wave 1: q to int8.
  // Lane j holds element j (and j + 64); the RoPE partner of element j is element j ^ 1 (DPP).
#pragma unroll
  for (int k = 0; k < 2; ++k) ((v4f_t*)tab)[lane + 64 * k] = tb[k];
  if (wave <= 1) {
    __builtin_amdgcn_s_waitcnt(0xc07f);          // lgkmcnt(0): this wave's table stores are done
    __builtin_amdgcn_wave_barrier();
    if (norm) {
      float* vec = wave == 0 ? s_k : s_q;
#pragma unroll
      for (int k = 0; k < NV; ++k)
        if (lane + 64 * k < HD) vec[lane + 64 * k] = xa[k];
      __builtin_amdgcn_s_waitcnt(0xc07f);
      __builtin_amdgcn_wave_barrier();
      float ss = 0.0f;
      if (lane < a.D) ss = ordered_sum<true>(vec, HD, a.D, lane);
      const float r = sfu_rsqrt(__shfl(ss, 0) * a.inv_hd + a.eps, tab);
#pragma unroll
      for (int k = 0; k < NV; ++k) xa[k] = (xa[k] * r) * xg[k];
    }
    float xr[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const float partner = dpp_f<kDppXor1>(xa[k]);
      xr[k] = (lane & 1) ? (xa[k] * cs[k]) + (partner * sn[k]) : (xa[k] * cs[k]) + ((-partner) * sn[k]);
    }
    int8_t* kq8 = (int8_t*)s_kq;
    int8_t* vq8 = (int8_t*)s_vq;
    int8_t* qq8 = (int8_t*)s_qq;
    if (wave == 0) {
      const long long crow = (long long)pos * kv_dim + (long long)g * HD;
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const int j = lane + 64 * k;
        float isk = a.inv_sk, isv = a.inv_sv;
        if constexpr (OPT) {
          if (a.ch_isk) isk = xc1[k];
          if (a.ch_isv) isv = xc2[k];
        }
        const int8_t kb = (int8_t)to_i8(xr[k] * isk), vb8 = (int8_t)to_i8(xb[k] * isv);
        if (j < HD) {
          kq8[j] = kb;
          vq8[j] = vb8;
          if (h % G == 0 && sj == 0 && pos_ok) {
            a.kc[crow + j] = kb;
            a.vc[crow + j] = vb8;
          }
        }
      }
    } else {
      if constexpr (OPT) {
        if (a.ch_sk) {                           // K per channel: its scales folded into q
#pragma unroll
          for (int k = 0; k < NV; ++k) xr[k] = xr[k] * xc1[k];
        }
      }
      uint32_t am = 0;
#pragma unroll
      for (int k = 0; k < NV; ++k)
        if (lane + 64 * k < HD) am = max(am, abs_bits(xr[k]));       // lanes past HD hold no element
      const float sq = fv(wave_max_u32(am)) * kInv127;
      const float inv = sfu_recip(sq, tab);
#pragma unroll
      for (int k = 0; k < NV; ++k)
        if (lane + 64 * k < HD) qq8[lane + 64 * k] = (int8_t)to_i8(xr[k] * inv);
      if (lane == 0) s_sq = sq;
    }
  }
  __syncthreads();
  // SPLIT: splits past the number of passes end here (all of a launch's workgroups agree on it; not
  // before the head vectors' first use, so that no branch lets the compiler sink their loads below
  // the position's wait); SPLIT 2: with zero sums
  if (SPLIT && sj >= nsp) {
    if (SPLIT == 2)
      for (int j = tid; j < HD; j += kAttnThreads) a.sp_o[(long long)sj * q_dim + (long long)h * HD + j] = 0;
    if (tid == 0) __hip_atomic_fetch_add(a.sp_sync + 2 * h, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
#pragma unroll
  for (int i = 0; i < R; ++i) vw[i] = buffer_load16(vrs, chunk_off(sj * TS * R + ts + TS * i));

  // ---- scores: slot c's partial dot products of the thread's rows, summed over the slot group
  float* sc = dyn;
  const int D = a.D, P = osum_stride(S, D);
  const float sq = s_sq;
  const int cc = cok ? c : 0;
  int qw[4], kpos[4], vpos[4];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    qw[w] = cok ? s_qq[4 * cc + w] : 0;
    kpos[w] = s_kq[4 * cc + w];
    vpos[w] = s_vq[4 * cc + w];
  }
  const int npass = (T + TS * R - 1) / (TS * R);
  constexpr int RM = R / NCHP;                   // rows a lane keeps per pass: i = j NCHP + c
  const int dummy = D * P + lane;                // per-lane LDS slot for stores that keep nothing
  float mloc = -__builtin_inff();
  // row pos lies past the buffer range (its K and V chunks load as zero); its slot's dot product comes
  // from the LDS copy of the new row, formed once
  int dpos = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) dpos = __builtin_amdgcn_sdot4(kpos[w], qw[w], dpos, false);
  for (int pass = sj; pass < npass; pass += nsp) {
    const int base = pass * TS * R;
    if (pass > sj) {
#pragma unroll
      for (int i = 0; i < R; ++i) kw[i] = buffer_load16(krs, chunk_off(base + ts + TS * i));
    }
    int dots[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
      int dot = 0;
#pragma unroll
      for (int w = 0; w < 4; ++w) dot = __builtin_amdgcn_sdot4(kw[i][w], qw[w], dot, false);
      dots[i] = base + ts + TS * i == pos ? dpos : dot;
    }
    // the slot group's partial sums, the DPP steps of all rows interleaved
    if (NCHP >= 2) {
#pragma unroll
      for (int i = 0; i < R; ++i) dots[i] += dpp_i<kDppXor1>(dots[i]);
    }
    if (NCHP >= 4) {
#pragma unroll
      for (int i = 0; i < R; ++i) dots[i] += dpp_i<kDppXor2>(dots[i]);
    }
    if (NCHP >= 8) {
#pragma unroll
      for (int i = 0; i < R; ++i) dots[i] += dpp_i<kDppHalfMirror>(dots[i]);
    }
    // every lane of a slot group now holds its rows' sums; lane c keeps rows i = j NCHP + c
#pragma unroll
    for (int j = 0; j < RM; ++j) {
      int dk = dots[j * NCHP];
#pragma unroll
      for (int q = 1; q < NCHP; ++q) dk = c == q ? dots[j * NCHP + q] : dk;
      const int t = base + ts + TS * (j * NCHP + c);
      const float sv = ((float)dk * sq) * a.a_k;
      const bool ok = t < T;
      sc[ok ? osum_index(t, D, P) : dummy] = sv;
      mloc = smax(mloc, ok ? sv : -__builtin_inff());
      if (SPLIT && ok) __hip_atomic_store(a.sp_s + (long long)h * S + t, sv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if constexpr (SPLIT) {
    // every split's scores published (every wave's stores complete before the barrier, so thread 0's
    // release covers all of them), then all T of them into sc from the published copy (the own ones
    // read back unchanged); the max over them
    wave_mem_done();
    __syncthreads();
    uint32_t* arrive = a.sp_sync + 2 * h;
    if (tid == 0) {
      const uint32_t old = __hip_atomic_fetch_add(arrive, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
      const uint32_t ns = (uint32_t)a.nsplit;
      split_wait(arrive, old - old % ns + ns, a.status);
    }
    __syncthreads();
    mloc = -__builtin_inff();
    const float* pub = a.sp_s + (long long)h * S;
    for (int t0 = 0; t0 < T; t0 += 4 * kAttnThreads) {   // four loads in flight per thread
      float sv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        sv[u] = __hip_atomic_load(pub + min(t0 + u * kAttnThreads + tid, T - 1), __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int t = t0 + u * kAttnThreads + tid;
        if (t < T) {
          sc[osum_index(t, D, P)] = sv[u];
          mloc = smax(mloc, sv[u]);
        }
      }
    }
  }
  mloc = wave_smax(mloc);
  if (lane == 0) red[wave] = mloc;
  lds_barrier();
  float m = red[0];
#pragma unroll
  for (int w = 1; w < kAttnWaves; ++w) m = smax(m, red[w]);

  // ---- e = EXP(s - m) by the row's keeping lane (+0 padding to a multiple of D), ordered sum, RECIP
  // over the lane-major copy itself: wave w takes its rows d = w, w + 8 of it (D is 8 or 16),
  // lanes the groups g < Tpad / D (row t = g D + d; +0 at t >= T), conflict-free runs of words
  const int Gt = (T + D - 1) / D;
  const bool two = D > kAttnWaves;
  for (int g0 = 0; g0 < Gt; g0 += 64) {
    const int gg = g0 + lane;
    if (gg < Gt) {
      float* p0 = sc + wave * P + gg;
      float* p1 = p0 + kAttnWaves * P;
      const float v0 = *p0, v1 = two ? *p1 : 0.0f;
      const float e0 = sfu_exp_np(v0 - m, tab);
      *p0 = gg * D + wave < T ? e0 : 0.0f;
      if (two) {
        const float e1 = sfu_exp_np(v1 - m, tab);
        *p1 = gg * D + wave + kAttnWaves < T ? e1 : 0.0f;
      }
    }
  }
  lds_barrier();
  if (wave == 0) {
    float ssum = 0.0f;
    if (lane < D) ssum = ordered_sum_t<false>(sc, T, D, P, lane);
    if (lane == 0) s_r = (OPT && a.qsum) ? 1.0f : sfu_recip(ssum, tab);   // qsum: to_i8(F(F(e * 1) * 127))
  }
  lds_barrier();
  const float rr = s_r;
  // int8 probabilities, once per row (not once per slot lane), in the order P.V reads them: word
  // (pass R / 4 + i / 4) TS + ts holds rows base + ts + TS (i - i % 4 + u), u = 0..3; +0 past T
  // (a thread forms one word, its four rows; SPLIT: the split's own passes, or all of them for
  // qsum's total)
  int8_t* pq = (int8_t*)(dyn + D * P + 64);
  int qs = 0;                                    // qsum: the probabilities of the rows this thread forms
  {
    constexpr int WP = (R / 4) * TS;             // words per pass
    const bool all = !SPLIT || (OPT && a.qsum);
    const int p0 = all ? 0 : sj, pst = all ? 1 : nsp;
    const int nw = ((npass - p0 + pst - 1) / pst) * WP;
    for (int q = tid; q < nw; q += kAttnThreads) {
      const int ps = p0 + (q / WP) * pst, r = q % WP;
      const int t0 = ps * TS * R + r % TS + 4 * TS * (r / TS);
      float sv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) sv[u] = sc[t0 + TS * u < T ? osum_index(t0 + TS * u, D, P) : dummy];
      int word = 0;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int p8 = t0 + TS * u < T ? to_i8((sv[u] * rr) * 127.0f) : 0;
        if (OPT) qs += p8;
        word |= (p8 & 0xFF) << (8 * u);
      }
      ((int*)pq)[ps * WP + r] = word;
    }
  }
  lds_barrier();

  // ---- P.V over the thread's rows, four at a time: int8 p of the four rows against V transposed
  int acc[16];
#pragma unroll
  for (int b = 0; b < 16; ++b) acc[b] = 0;
  for (int pass = sj; pass < npass; pass += nsp) {
    const int base = pass * TS * R;
    if (pass > sj) {
#pragma unroll
      for (int i = 0; i < R; ++i) vw[i] = buffer_load16(vrs, chunk_off(base + ts + TS * i));
    }
#pragma unroll
    for (int i4 = 0; i4 < R; i4 += 4) {
      if (base + TS * i4 >= T) break;
      int rw[4][4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int w = 0; w < 4; ++w) rw[u][w] = vw[i4 + u][w];     // row pos: zero here, added below
      const int pp = ((const int*)pq)[(pass * (R / 4) + (i4 >> 2)) * TS + ts];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        int col[4];
        transpose4x4(rw[0][w], rw[1][w], rw[2][w], rw[3][w], col);
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[4 * w + k] = __builtin_amdgcn_sdot4(col[k], pp, acc[4 * w + k], false);
      }
    }
  }
  // row pos's term, p(pos) times the new V row (from LDS), in the threads whose slot holds row pos
  // (exact int32 either way)
  if (ts == pos % TS && cok && (pos / (TS * R)) % nsp == sj) {
    const int ppos = to_i8((sc[osum_index(pos, D, P)] * rr) * 127.0f);
#pragma unroll
    for (int w = 0; w < 4; ++w)
#pragma unroll
      for (int k = 0; k < 4; ++k) acc[4 * w + k] += ppos * (int)(int8_t)(vpos[w] >> (8 * k));
  }
  // ---- partial sums: lanes of a 16-lane row with the same slot rotate-and-add over the row-slice
  // bits, then one partial per row of lanes and wave meets in LDS
#pragma unroll
  for (int b = 0; b < 16; ++b) {
    int v = acc[b];
    if (NCHP <= 1) v += dpp_i<0x121>(v);                      // row_ror:1
    if (NCHP <= 2) v += dpp_i<0x122>(v);                      // row_ror:2
    if (NCHP <= 4) v += dpp_i<0x124>(v);                      // row_ror:4
    if (NCHP <= 8) v += dpp_i<0x128>(v);                      // row_ror:8
    acc[b] = v;
  }
  if (OPT && a.qsum) {
    qs = wave_sum_i32(qs);
    if (lane == 0) s_qs[wave] = qs;
  }
  if ((lane & 15) < NCHP && cok) {
#pragma unroll
    for (int b = 0; b < 16; ++b) part[wave * 4 + (lane >> 4)][16 * c + b] = acc[b];
  }
  __syncthreads();
  float* out = a.att + row * a.att_stride;
  float rq = 1.0f;
  if (OPT && a.qsum) {
    int tot = 0;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) tot += s_qs[w];
    rq = qsum_scale(tot, tab);
  }
  if constexpr (SPLIT == 2) {
    // this split's sums for the next linear's prologue; the counters cleared by the last split
    for (int j = tid; j < HD; j += kAttnThreads) {
      int ssum = 0;
#pragma unroll
      for (int w = 0; w < kAttnWaves * 4; ++w) ssum += part[w][j];
      if (pos_ok) a.sp_o[(long long)sj * q_dim + (long long)h * HD + j] = ssum;
    }
    if (!pos_ok && tid == 0) flag_bad_pos(a.status);
    return;
  }
  if constexpr (SPLIT == 1) {
    // this split's sums into the head's (exact int32 device atomics, every wave's complete before the
    // barrier); the last split to arrive finishes the output from them and clears them and the
    // counters for the next launch
    for (int j = tid; j < HD; j += kAttnThreads) {
      int ssum = 0;
#pragma unroll
      for (int w = 0; w < kAttnWaves * 4; ++w) ssum += part[w][j];
      __hip_atomic_fetch_add(a.sp_acc + (long long)h * kMaxHd + j, ssum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    wave_mem_done();
    __syncthreads();
    if (tid == 0)
      s_last = __hip_atomic_fetch_add(a.sp_sync + 2 * h + 1, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) ==
               (uint32_t)(nsp - 1);
    __syncthreads();
    if (!s_last) return;
  }
  if (!pos_ok && tid == 0) flag_bad_pos(a.status);   // (SPLIT 1 still clears its sums below)
  for (int j = tid; j < HD; j += kAttnThreads) {
    int ssum = 0;
    if constexpr (SPLIT) {
      int* o = a.sp_acc + (long long)h * kMaxHd + j;
      ssum = __hip_atomic_load(o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(o, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
#pragma unroll
      for (int w = 0; w < kAttnWaves * 4; ++w) ssum += part[w][j];
    }
    if (!pos_ok) continue;
    if constexpr (OPT) {
      float o = (float)ssum;
      if (a.qsum) o = o * rq;
      out[(long long)h * HD + j] = o * (a.ch_av ? a.ch_av[(long long)g * HD + j] : a.a_v);
    } else {
      out[(long long)h * HD + j] = (float)ssum * a.a_v;
    }
  }
  if (SPLIT && tid == 0) __hip_atomic_store(a.sp_sync + 2 * h + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- prefill prep (ATTN_PREP): one wave per head vector of a row (the H query heads, then the Hk
// KV heads): QK-norm and RoPE by head_norm_rope, the decode kernels' numerics; q back into qkv
// (fp32), k and v to int8 into the cache row at the row's position. Each KV head's row is formed
// once, by its own wave. With Wqkv's split-K partials pending, the wave finishes its columns first.
constexpr int kPrepWaves = 4;

__global__ __launch_bounds__(64 * kPrepWaves) void k_attn_prep(AttnArgs a) {
  __shared__ float sv[kPrepWaves][2][kMaxHd];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = blockIdx.y, vi = blockIdx.x * kPrepWaves + wave;
  const int hd = a.hd;
  if (vi >= a.H + a.Hk) return;                  // (wave-uniform; the kernel has no block barrier)
  const int pos = a.pos[row];
  if (pos < 0 || pos >= a.S) {                   // a position outside the cache: nothing is written
    if (lane == 0) flag_bad_pos(a.status);
    return;
  }
  const int q_dim = a.H * hd, kv_dim = a.Hk * hd;
  float* qkv = a.qkv + row * a.qkv_stride;
  const int32_t* pr = a.part + row * a.qkv_stride;
  const float sx = a.part_nz > 1 ? a.part_sx[row] : 0.0f;
  auto col = [&](int c) {                        // column c of the row's [q | k | v]
    if (a.part_nz <= 1) return qkv[c];
    int acc = 0;
    for (int z = 0; z < a.part_nz; ++z) acc += pr[z * a.part_zstride + c];
    return dequant(acc, a.part_sw[c], sx);
  };
  float* v0 = sv[wave][0];
  const float* gain = vi < a.H ? a.qn : a.kn;
  const NormRopeOps ops = norm_rope_ops(gain, a, pos, lane);   // requested with the head vector
  if (vi < a.H) {
    for (int j = lane; j < hd; j += 64) v0[j] = col(vi * hd + j);
    __builtin_amdgcn_wave_barrier();
    head_norm_rope(v0, gain != nullptr, ops, a, lane);
    for (int j = lane; j < hd; j += 64) qkv[vi * hd + j] = v0[j];
    return;
  }
  const int g = vi - a.H;
  float* v1 = sv[wave][1];
  for (int j = lane; j < hd; j += 64) {
    v0[j] = col(q_dim + g * hd + j);
    v1[j] = col(q_dim + kv_dim + g * hd + j);
  }
  __builtin_amdgcn_wave_barrier();
  head_norm_rope(v0, gain != nullptr, ops, a, lane);
  int8_t* kc = a.kc + row * a.kv_row_stride + (long long)pos * kv_dim + g * hd;
  int8_t* vc = a.vc + row * a.kv_row_stride + (long long)pos * kv_dim + g * hd;
  for (int j = lane; j < hd / 4; j += 64) {
    int k4[4], v4[4];
    for (int b = 0; b < 4; ++b) {
      const int ch = g * hd + 4 * j + b;
      k4[b] = to_i8(v0[4 * j + b] * (a.ch_isk ? a.ch_isk[ch] : a.inv_sk));
      v4[b] = to_i8(v1[4 * j + b] * (a.ch_isv ? a.ch_isv[ch] : a.inv_sv));
    }
    *(int*)(kc + 4 * j) = pack_i8x4(k4[0], k4[1], k4[2], k4[3]);
    *(int*)(vc + 4 * j) = pack_i8x4(v4[0], v4[1], v4[2], v4[3]);
  }
}

// k_attn_prep at head dims 64 and 128 (NV = HD / 64 elements a lane: element lane + 64 k), without
// branches on the elements: the head vector, the norm gains and the RoPE tables are requested
// together; lanes [0, D) run the RMSNorm chain over an LDS copy; the RoPE partner of element j (j ^ 1,
// the lane next door) comes by one DPP exchange; q goes back as fp32, k and v to int8 cache rows (a
// byte a lane, consecutive lanes consecutive bytes). The numerics are head_norm_rope's.
template <int HD>
__global__ __launch_bounds__(64 * kPrepWaves) void k_attn_prep_h(AttnArgs a) {
  constexpr int NV = HD / 64;
  __shared__ float sv[kPrepWaves][HD];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = blockIdx.y, vi = blockIdx.x * kPrepWaves + wave;
  if (vi >= a.H + a.Hk) return;                  // (wave-uniform; the kernel has no block barrier)
  const int pos = a.pos[row];
  if (pos < 0 || pos >= a.S) {                   // a position outside the cache: nothing is written
    if (lane == 0) flag_bad_pos(a.status);
    return;
  }
  const int q_dim = a.H * HD, kv_dim = a.Hk * HD;
  float* qkv = a.qkv + row * a.qkv_stride;
  const bool isq = vi < a.H;
  const int g = vi - a.H;
  const int c0 = isq ? vi * HD : q_dim + g * HD;    // the vector (k for a KV head's wave)
  const int ycol = isq ? c0 : q_dim + kv_dim + g * HD;   // its V vector (a q wave: its own, unused)
  const float* gain = isq ? a.qn : a.kn;
  const float* gsrc = gain != nullptr ? gain : qkv;      // (no gain: any readable vector, unused)
  const float* cs = a.cos_t + (long long)pos * (HD / 2);
  const float* sn = a.sin_t + (long long)pos * (HD / 2);
  // every load issued before the first wait: unconditional, the split-K sums on a path of their own
  // (a load under a branch makes the compiler's wait counts path-dependent, and it then waits for
  // each before the next is issued)
  float x[NV], y[NV], gv[NV], c[NV], s[NV];
  if (a.part_nz <= 1) {
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      x[k] = qkv[c0 + lane + 64 * k];
      y[k] = qkv[ycol + lane + 64 * k];
    }
  } else {
    const int32_t* pr = a.part + row * a.qkv_stride;
    const float sx = a.part_sx[row];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int j = lane + 64 * k;
      int ax = 0, ay = 0;
      for (int z = 0; z < a.part_nz; ++z) {
        ax += pr[z * a.part_zstride + c0 + j];
        ay += pr[z * a.part_zstride + ycol + j];
      }
      x[k] = dequant(ax, a.part_sw[c0 + j], sx);
      y[k] = dequant(ay, a.part_sw[ycol + j], sx);
    }
  }
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int j = lane + 64 * k;
    gv[k] = gsrc[j];
    c[k] = cs[j >> 1];
    s[k] = sn[j >> 1];
  }
  // int8 q (a.q8): RECIP's 64 table pairs, lane i holding pair i, read by lane exchange
  const float2 rt = sfu_recip_pair(lane, c_sfu);
  if (gain != nullptr) {
    float* v = sv[wave];
#pragma unroll
    for (int k = 0; k < NV; ++k) v[lane + 64 * k] = x[k];
    __builtin_amdgcn_s_waitcnt(0xc07f);          // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
    float acc = 0.0f;
    if (lane < a.D) {
      const int n = HD / a.D;                    // the chain's length (HD a multiple of D)
      acc = v[lane] * v[lane];
#pragma unroll
      for (int m = 1; m < HD / 8; ++m)
        if (m < n) {
          const float e = v[lane + m * a.D];
          acc = acc + e * e;
        }
    }
    const float r = sfu_rsqrt(lane_tree_sum(acc, a.D, lane) * a.inv_hd + a.eps);
#pragma unroll
    for (int k = 0; k < NV; ++k) x[k] = (x[k] * r) * gv[k];
  }
  // RoPE: even element 2i -> (x c) + ((-x[2i+1]) s), odd 2i+1 -> (x c) + (x[2i] s)
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const float p = __int_as_float(dpp_mov_i<kDppXor1>(__float_as_int(x[k])));
    x[k] = (lane & 1) ? (x[k] * c[k]) + (p * s[k]) : (x[k] * c[k]) + ((-p) * s[k]);
  }
  if (isq && a.q8 != nullptr) {
    // quant_act of the q vector for k_attn_pw: s = F(max |q| F(1/127)), q8 = to_i8(F(q RECIP(s)))
    uint32_t am = abs_bits(x[0]);
#pragma unroll
    for (int k = 1; k < NV; ++k) am = max(am, abs_bits(x[k]));
    const float sq = fv(wave_max_u32(am)) * kInv127;
    const float inv = sfu_recip_by(sq, [&](int i) { return make_float2(__shfl(rt.x, i), __shfl(rt.y, i)); });
    int8_t* q8 = a.q8 + row * a.q8_stride + vi * HD;
#pragma unroll
    for (int k = 0; k < NV; ++k) q8[lane + 64 * k] = (int8_t)to_i8(x[k] * inv);
    if (lane == 0) a.q8s[row * a.H + vi] = sq;
    return;
  }
  if (isq) {
#pragma unroll
    for (int k = 0; k < NV; ++k) qkv[c0 + lane + 64 * k] = x[k];
    return;
  }
  int8_t* kc = a.kc + row * a.kv_row_stride + (long long)pos * kv_dim + g * HD;
  int8_t* vc = a.vc + row * a.kv_row_stride + (long long)pos * kv_dim + g * HD;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int j = lane + 64 * k, ch = g * HD + j;
    kc[j] = (int8_t)to_i8(x[k] * (a.ch_isk ? a.ch_isk[ch] : a.inv_sk));
    vc[j] = (int8_t)to_i8(y[k] * (a.ch_isv ? a.ch_isv[ch] : a.inv_sv));
  }
}

// k_attn_prep_h with half a wave per head vector (two vectors a wave): the same steps per vector, with
// the two vectors' chains, pairwise trees and RSQRTs in the same instructions (lanes [0, D) and
// [32, 32 + D)). At head dim 128 lane hl of a half holds the 4 consecutive elements 4 hl .. 4 hl + 3:
// the row's columns and gains come as one vector load each, an element's RoPE partner (j ^ 1) is in
// the same lane, and q, the int8 q and the int8 cache rows go out as one store a lane (C3's prep
// kernel, writing the int8 q, 15.5 us against 15.9 writing fp32 q from the strided layout). At head
// dim 64 lane hl holds elements hl and hl + 32 (the partner one DPP exchange away, byte stores): two
// consecutive elements a lane, with 16-bit cache stores, took 5.6 us against 5.3 at C4. A wave's
// halves may hold a q and a k vector (odd H): each half stores what its vector writes. R: rows a
// wave, every row's loads issued before the first row's steps.
template <int HD, int R = 1>
__global__ __launch_bounds__(64 * kPrepWaves) void k_attn_prep_h2(AttnArgs a, int rows) {
  constexpr int NV = HD / 32;
  constexpr bool CONTIG = HD == 128;
  static_assert(NV == 2 || NV == 4, "head dims 64 and 128");
  __shared__ __align__(16) float sv[kPrepWaves][2][HD];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, half = lane >> 5, hl = lane & 31;
  const int w2 = 2 * (blockIdx.x * kPrepWaves + wave);
  const int nvec = a.H + a.Hk;
  if (w2 >= nvec) return;                        // (wave-uniform; the kernel has no block barrier)
  const bool live = w2 + half < nvec;            // the second half of the last wave when nvec is odd
  const int vi = min(w2 + half, nvec - 1);
  const int q_dim = a.H * HD, kv_dim = a.Hk * HD;
  const bool isq = vi < a.H;
  const int g = isq ? 0 : vi - a.H;
  const int c0 = isq ? vi * HD : q_dim + g * HD;  // the vector (k for a KV head's half)
  const float* gain = isq ? a.qn : a.kn;
  auto el = [&](int k) { return CONTIG ? NV * hl + k : hl + 32 * k; };   // the lane's element k
  // the wave's R rows blockIdx.y R + rr (rows past the call or at a position outside the cache: skipped,
  // the latter flagged; both wave-uniform)
  int row[R], pos[R];
  bool ok[R];
#pragma unroll
  for (int rr = 0; rr < R; ++rr) {
    row[rr] = blockIdx.y * R + rr;
    pos[rr] = a.pos[min(row[rr], rows - 1)];
    ok[rr] = row[rr] < rows && pos[rr] >= 0 && pos[rr] < a.S;
    if (row[rr] < rows && !ok[rr] && lane == 0) flag_bad_pos(a.status);
  }
  // every row's loads first, all of them unconditional (a load under a branch makes the compiler's
  // wait counts path-dependent, and it then waits for each before the next is issued): rows that are
  // skipped read row 0 at position 0, q halves read their own vector again for y, a missing gain
  // reads the row-0 vector; those values are not used
  float x[R][NV], y[R][NV], c[R][NV], s[R][NV], gv[NV];
  const int ycol = isq ? c0 : q_dim + kv_dim + g * HD;   // the V vector of a KV head's half
  int prow[R], ppos[R];
#pragma unroll
  for (int rr = 0; rr < R; ++rr) {
    prow[rr] = ok[rr] ? row[rr] : 0;
    ppos[rr] = ok[rr] ? pos[rr] : 0;
  }
  auto vec = [&](const float* p, float (&o)[NV]) {       // the lane's elements of the vector at p
    if constexpr (CONTIG) {
      const v4f_t v = *(const v4f_t*)(p + el(0));
      o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
    } else {
#pragma unroll
      for (int k = 0; k < NV; ++k) o[k] = p[el(k)];
    }
  };
  if (a.part_nz <= 1) {
#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
      const float* qkv = a.qkv + prow[rr] * a.qkv_stride;
      vec(qkv + c0, x[rr]);
      vec(qkv + ycol, y[rr]);
    }
  } else {                                       // Wqkv's split-K partials summed (the store epilogue)
#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
      const int32_t* pr = a.part + prow[rr] * a.qkv_stride;
      const float sx = a.part_sx[prow[rr]];
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        int ax = 0, ay = 0;
        for (int z = 0; z < a.part_nz; ++z) {
          ax += pr[z * a.part_zstride + c0 + el(k)];
          ay += pr[z * a.part_zstride + ycol + el(k)];
        }
        x[rr][k] = dequant(ax, a.part_sw[c0 + el(k)], sx);
        y[rr][k] = dequant(ay, a.part_sw[ycol + el(k)], sx);
      }
    }
  }
#pragma unroll
  for (int rr = 0; rr < R; ++rr) {
    const float* cs = a.cos_t + (long long)ppos[rr] * (HD / 2);
    const float* sn = a.sin_t + (long long)ppos[rr] * (HD / 2);
#pragma unroll
    for (int k = 0; k < NV; ++k) {               // element j's RoPE entry j / 2 (CONTIG: k, k + 1 share it)
      if (CONTIG && (k & 1)) {
        c[rr][k] = c[rr][k - 1];
        s[rr][k] = s[rr][k - 1];
      } else {
        c[rr][k] = cs[el(k) >> 1];
        s[rr][k] = sn[el(k) >> 1];
      }
    }
  }
  vec(gain != nullptr ? gain : a.qkv, gv);
  // int8 q (a.q8): RECIP's 64 table pairs, lane i holding pair i, read by lane exchange
  const float2 rt = sfu_recip_pair(lane, c_sfu);
  auto put8 = [&](int8_t* p, const int (&b)[NV]) {   // the lane's bytes of a vector
    if constexpr (CONTIG) {
      *(int*)(p + el(0)) = pack_i8x4(b[0], b[1], b[2], b[3]);
    } else {
#pragma unroll
      for (int k = 0; k < NV; ++k) p[el(k)] = (int8_t)b[k];
    }
  };
#pragma unroll
  for (int rr = 0; rr < R; ++rr) {
    if (!ok[rr]) continue;
    float* xr = x[rr];
    if (a.qn != nullptr || a.kn != nullptr) {    // QK-norm of the halves whose vector has a gain
      float* v = sv[wave][half];                 // (a wave's LDS operations run in order: the previous
      if constexpr (CONTIG) {                    //  row's chain reads come before these stores)
        *(v4f_t*)(v + el(0)) = v4f_t{xr[0], xr[1], xr[2], xr[3]};
      } else {
#pragma unroll
        for (int k = 0; k < NV; ++k) v[el(k)] = xr[k];
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);        // lgkmcnt(0)
      __builtin_amdgcn_wave_barrier();
      float acc = 0.0f;
      if (hl < a.D) {
        const int n = HD / a.D;                  // the chain's length (HD a multiple of D)
        acc = v[hl] * v[hl];
#pragma unroll
        for (int m = 1; m < HD / 8; ++m)
          if (m < n) {
            const float e = v[hl + m * a.D];
            acc = acc + e * e;
          }
      }
      acc = lane_tree_rows(acc, a.D, lane);
      const float s0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), 0));
      const float s1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), 32));
      const float r = sfu_rsqrt((half ? s1 : s0) * a.inv_hd + a.eps);
      if (gain != nullptr)
#pragma unroll
        for (int k = 0; k < NV; ++k) xr[k] = (xr[k] * r) * gv[k];
    }
    // RoPE: even element 2i -> (x c) + ((-x[2i+1]) s), odd 2i+1 -> (x c) + (x[2i] s)
    if constexpr (CONTIG) {
#pragma unroll
      for (int k = 0; k < NV; k += 2) {
        const float xe = xr[k], xo = xr[k + 1];
        xr[k] = (xe * c[rr][k]) + ((-xo) * s[rr][k]);
        xr[k + 1] = (xo * c[rr][k + 1]) + (xe * s[rr][k + 1]);
      }
    } else {
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const float p = __int_as_float(dpp_mov_i<kDppXor1>(__float_as_int(xr[k])));
        xr[k] = (lane & 1) ? (xr[k] * c[rr][k]) + (p * s[rr][k]) : (xr[k] * c[rr][k]) + ((-p) * s[rr][k]);
      }
    }
    // quant_act of a q vector for k_attn_pw (as k_attn_prep_h): each half's maximum over its 32
    // lanes; formed with every lane active (the table's lane exchange reads all 64)
    float sq = 0.0f, inv = 0.0f;
    if (a.q8 != nullptr) {
      uint32_t am = abs_bits(xr[0]);
#pragma unroll
      for (int k = 1; k < NV; ++k) am = max(am, abs_bits(xr[k]));
      sq = fv(half_max_u32(am, half)) * kInv127;
      inv = sfu_recip_by(sq, [&](int i) { return make_float2(__shfl(rt.x, i), __shfl(rt.y, i)); });
    }
    if (!live) continue;
    const int rw = row[rr];
    if (isq) {
      if (a.q8 != nullptr) {
        int b[NV];
#pragma unroll
        for (int k = 0; k < NV; ++k) b[k] = to_i8(xr[k] * inv);
        put8(a.q8 + rw * a.q8_stride + vi * HD, b);
        if (hl == 0) a.q8s[rw * a.H + vi] = sq;
      } else if constexpr (CONTIG) {
        *(v4f_t*)(a.qkv + rw * a.qkv_stride + c0 + el(0)) = v4f_t{xr[0], xr[1], xr[2], xr[3]};
      } else {
#pragma unroll
        for (int k = 0; k < NV; ++k) a.qkv[rw * a.qkv_stride + c0 + el(k)] = xr[k];
      }
    } else {
      int bk[NV], bv[NV];
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const int ch = g * HD + el(k);
        bk[k] = to_i8(xr[k] * (a.ch_isk ? a.ch_isk[ch] : a.inv_sk));
        bv[k] = to_i8(y[rr][k] * (a.ch_isv ? a.ch_isv[ch] : a.inv_sv));
      }
      put8(a.kc + rw * a.kv_row_stride + (long long)pos[rr] * kv_dim + g * HD, bk);
      put8(a.vc + rw * a.kv_row_stride + (long long)pos[rr] * kv_dim + g * HD, bv);
    }
  }
}

// ------------------------------------------------------------------ prefill attention
// ATTN_ONLY for many rows at once (rows whose q is rotated and whose KV rows are in the cache), one
// workgroup of 8 or 16 waves per (query head, 16 consecutive rows). Scores and P.V run on the int8
// matrix cores (v_mfma_i32_32x32x32_i8, query rows 16..31 of each tile zero): every lane feeds 16
// consecutive k-bytes of its A row and of its B row, the same k for both, so each int32 is the exact
// dot product. The softmax is per row and follows the decode numerics exactly:
//  - the row maximum (order-free) and e = EXP(s - max) (+0 padding to a multiple of D), 32 or 64
//    threads per row, every element independent;
//  - thread (row i, lane l < D) then adds the row's e[t], t = l, l + D, ... in order: the lane
//    chain of the D-lane ordered sum; DPP pairs the D lanes, and RECIP gives r.
// P.V packs to_i8(e r 127) of 16 t per lane against V transposed in LDS (wave-private tiles, 32 or
// 64 columns at a time).
constexpr int kPreRows = 16;
constexpr size_t kPreMaxLds = 136 * 1024;     // dynamic LDS the kernels are set up for (of 160 KB per CU)
// Threads of k_attn_pre: 1024 (16 waves; a wave per row in the softmax) at head dims over 64, where
// the registers (<= 128 a lane) and long caches' score rows leave one workgroup per CU: twice the
// waves per SIMD to hide the EXP's table reads and the phases' barriers. 512 (8 waves, half a wave
// per row) at head dims <= 64, where two or more workgroups share a CU.
__host__ __device__ constexpr int pre_threads(int HDP) { return HDP > 64 ? 1024 : 512; }

// Row stride (floats) of the score / exp rows: at least S + 16, and 17 mod 64. The P.V pass reads one
// key of all 16 rows per instruction (and, in lanes 32-63, the key 16 on): 32 distinct LDS banks.
// (A stride of 0 or 32 mod 64 put the 16 rows of a key in 2 banks.)
__host__ __device__ inline int pre_est(int S) { return ((S + 16 + 63) & ~63) + 17; }

template <int HDP, bool OPT = false>   // head dim padded to a multiple of 32 (MFMA k-steps); OPT: HF options
__global__ __launch_bounds__(pre_threads(HDP)) void k_attn_pre(AttnArgs a, int M) {
  constexpr int NT = pre_threads(HDP), NW = NT / 64;
  constexpr int TPR = NT / kPreRows;           // softmax threads per row: 32 or 64, all in one wave
  constexpr int KS = HDP / 32;                 // k-steps of the score MFMA; column tiles of P.V
  constexpr int NV = HDP > 64 ? 2 : 1;
  constexpr int VTC = NW > 8 ? 32 : (HDP < 64 ? HDP : 64);   // V columns transposed per pass (16 KB of VT)
  // cache tiles in flight per wave: the score pass 4 (all 64 tiles of a 2048-key block at 16 waves);
  // P.V at 16 waves 8 (a wave takes one 32-column quarter of V: 16 bytes a lane per tile; 16 spill),
  // else 4
  constexpr int PTS = 4, PTV = NW > 8 ? 8 : 4;
  constexpr int NPASS = HDP / VTC, QP = VTC / 32;   // V transpose passes; 16-byte chunks a lane per pass
  extern __shared__ __align__(16) float E[];   // [16][est] scores, then exps; then the P.V sums
  __shared__ __align__(16) float tab[kSfuWords];
  __shared__ __align__(16) int8_t Q8[kPreRows][HDP];
  __shared__ __align__(16) int8_t VT[NW][VTC][32];
  __shared__ float s_sq[kPreRows];
  __shared__ int s_T[kPreRows];
  __shared__ int s_qs[kPreRows];
  __shared__ float s_mx[NW][kPreRows];          // each wave's maximum of each row's scores
  // row blocks in reverse: a causal prompt's later rows attend to more positions, and the blocks
  // dispatched first should be the longest (the short ones then fill in behind them)
  const int h = blockIdx.x, r0 = (gridDim.y - 1 - blockIdx.y) * kPreRows, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int HD = a.hd, G = a.H / a.Hk, g = h / G, S = a.S, D = a.D;
  const int cap = a.t_cap > 0 && a.t_cap < S ? a.t_cap : S;   // positions a row may attend to
  const int kv_dim = a.Hk * HD, est = pre_est(cap);
  if (tid < kSfuWords / 4) ((v4f_t*)tab)[tid] = ((const v4f_t*)a.tab)[tid];
  __syncthreads();

  // ---- q of the block's rows to int8 (a wave per row or per 2 rows); rows without a valid position: T = 0
  for (int i = wave; i < kPreRows; i += NW) {
    const int r = min(r0 + i, M - 1);
    const int pos = a.pos[r];
    const bool ok = r0 + i < M && pos >= 0 && pos < S;
    const float* q = a.qkv + (long long)r * a.qkv_stride + (long long)h * HD;
    float x[NV];
    uint32_t am = 0;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int j = lane + 64 * k;
      x[k] = q[min(j, HD - 1)];
      if (OPT && a.ch_sk) x[k] = x[k] * a.ch_sk[(long long)g * HD + min(j, HD - 1)];   // K per channel
      if (j < HD) am = max(am, abs_bits(x[k]));
    }
    const float sq = fv(wave_max_u32(am)) * kInv127;
    const float inv = sfu_recip(sq, tab);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int j = lane + 64 * k;
      if (j < HDP) Q8[i][j] = (int8_t)(ok && j < HD ? to_i8(x[k] * inv) : 0);
    }
    if (lane == 0) {
      s_sq[i] = sq;
      s_T[i] = ok ? min(pos + 1, cap) : 0;       // (cap bounds every position by construction)
    }
  }
  __syncthreads();
  int Tmax = 0;
#pragma unroll
  for (int i = 0; i < kPreRows; ++i) Tmax = max(Tmax, s_T[i]);
  const int ntile = (Tmax + 31) / 32;
  const __amdgpu_buffer_rsrc_t krs = buffer_rsrc(a.kc, (uint32_t)S * kv_dim);
  const __amdgpu_buffer_rsrc_t vrs = buffer_rsrc(a.vc, (uint32_t)S * kv_dim);
  const int lr = lane & 31, lk = (lane >> 5) * 16;

  // ---- scores of the wave's tiles (t = 32 tile + n), PTS tiles' K rows in flight at a time. A tile
  // past the block's last gets an offset outside the buffer: zeros, with no memory access. Each lane
  // also keeps the maximum of the scores it writes of each of its 8 rows (keys t < T of the row;
  // smax: order-free, NaN winning).
  constexpr uint32_t kNoRow = 0x80000000u;      // beyond every cache (S kv_dim < 2^31)
  v4i_t qa[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
    qa[ks] = lr < kPreRows ? *(const v4i_t*)&Q8[lr][32 * ks + lk] : v4i_t{0, 0, 0, 0};
  float rmx[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) rmx[r] = -__builtin_inff();
  for (int c0 = wave; c0 < ntile; c0 += NW * PTS) {
    v4i_t kb[PTS][KS];
#pragma unroll
    for (int u = 0; u < PTS; ++u) {
      const int ti = c0 + NW * u;
      const uint32_t off = ti < ntile ? (uint32_t)(32 * ti + lr) * kv_dim + g * HD + lk : kNoRow;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kb[u][ks] = buffer_load16(krs, off + 32 * ks);
    }
#pragma unroll
    for (int u = 0; u < PTS; ++u) {
      const int ti = c0 + NW * u;
      if (ti >= ntile) break;
      v16i_t acc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = 0;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(qa[ks], kb[u][ks], acc, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 8; ++r) {                   // output rows m < 16
        const int m = (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        const float sv = ((float)acc[r] * s_sq[m]) * a.a_k;
        E[m * est + 32 * ti + lr] = sv;
        rmx[r] = smax(rmx[r], 32 * ti + lr < s_T[m] ? sv : -__builtin_inff());
      }
    }
  }
  // the wave's maximum of each row: over the 32 lanes of a half (which share their 8 rows)
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    float v = rmx[r];
    v = smax(v, dpp_f<kDppXor1>(v));
    v = smax(v, dpp_f<kDppXor2>(v));
    v = smax(v, dpp_f<kDppHalfMirror>(v));
    v = smax(v, dpp_f<kDppMirror>(v));
    v = smax(v, __shfl_xor(v, 16));
    if (lr == 0) s_mx[wave][(r >> 2) * 8 + (lane >> 5) * 4 + (r & 3)] = v;
  }
  __syncthreads();

  // ---- per row (TPR threads of one wave each): the row maximum from the waves' maxima, e = EXP(s -
  // max) (s <= max: the softmax form of EXP) with +0 padding to a multiple of D; the D-lane ordered
  // sum and RECIP; then the row's int8 probabilities
  {
    const int i = tid / TPR, sub = tid % TPR;
    const int T = s_T[i];
    float* row = E + i * est;
    float mx = s_mx[0][i];
#pragma unroll
    for (int w = 1; w < NW; ++w) mx = smax(mx, s_mx[w][i]);
    const int groups = T > 0 ? (T + D - 1) / D : 0, Tpad = groups * D;
    for (int t = sub; t < Tpad; t += TPR * 4) {
      float e[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) e[j] = t + TPR * j < T ? row[t + TPR * j] : 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) e[j] = t + TPR * j < T ? sfu_exp_np(e[j] - mx, tab) : 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (t + TPR * j < Tpad) row[t + TPR * j] = e[j];
    }
    // the row's exps were written by this wave's lanes: wait for them, then the lane chains
    __builtin_amdgcn_s_waitcnt(0xc07f);            // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
    float acc = 0.0f;
    if (sub < D) {
      int gi = 0;
      for (; gi + 8 <= groups; gi += 8) {
        float e[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) e[j] = row[sub + (gi + j) * D];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc = gi + j == 0 ? e[j] : acc + e[j];
      }
      for (; gi < groups; ++gi) {
        const float e = row[sub + gi * D];
        acc = gi == 0 ? e : acc + e;
      }
    }
    // pairwise tree over the D lanes of the row (lane l, l % 2s == 0, takes lane l + s); the row's
    // lanes sub 0..15 are one 16-lane DPP row
    float o = dpp_f<0x101>(acc);
    if (D > 1 && (sub & 1) == 0) acc = acc + o;
    o = dpp_f<0x102>(acc);
    if (D > 2 && (sub & 3) == 0) acc = acc + o;
    o = dpp_f<0x104>(acc);
    if (D > 4 && (sub & 7) == 0) acc = acc + o;
    o = dpp_f<0x108>(acc);
    if (D > 8 && (sub & 15) == 0) acc = acc + o;
    // r (qsum: 1, so p = to_i8(F(F(e * 1) * 127))) from the row's first lane to all of its lanes
    const uint32_t rb = fb((OPT && a.qsum) ? 1.0f : sfu_recip(acc, tab));
    const float ri = fv((uint32_t)(TPR == 64 || lane < 32 ? __builtin_amdgcn_readlane((int)rb, 0)
                                                          : __builtin_amdgcn_readlane((int)rb, 32)));

    // int8 probabilities p = to_i8(F(F(e r) 127)), once per (row, key), written over the row's own
    // exps: bytes from byte ((4 i est + 15) & ~15) of E (inside row i's floats), zero from T to the
    // tiles' end. Keys go in blocks of 512: the row's lanes read their exps of the block, then write
    // the bytes, which land on exps of this block or of earlier ones: the row is this wave's alone,
    // and a wave's LDS accesses complete in order, so no workgroup barrier is needed.
    constexpr int PE = 512 / TPR;
    int8_t* prow = (int8_t*)E + (((long long)i * est * 4 + 15) & ~15LL);
    int qsr = 0;                                      // qsum: the row's probabilities (exact)
    for (int c0 = 0; c0 < 32 * ntile; c0 += 512) {
      float e[PE];
#pragma unroll
      for (int j = 0; j < PE; ++j) {
        const int t = c0 + sub + TPR * j;
        e[j] = t < T ? row[t] : 0.0f;
      }
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int j = 0; j < PE; ++j) {
        const int t = c0 + sub + TPR * j;
        const int p8 = t < T ? to_i8((e[j] * ri) * 127.0f) : 0;
        if (OPT) qsr += p8;
        if (t < 32 * ntile) prow[t] = (int8_t)p8;
      }
    }
    if (OPT && a.qsum) {                              // the row's TPR threads: half a wave or a wave
      qsr = TPR == 64 ? wave_sum_i32(qsr) : wave_half_sum_i32(qsr);
      if (sub == 0) s_qs[i] = qsr;
    }
  }
  __syncthreads();

  // ---- P.V: per tile, int8 p of 16 t per lane (A) against V transposed (B), exact int32
  const int pm = lr;                                  // A row of this lane
  const int8_t* pmrow = (const int8_t*)E + (((long long)min(pm, kPreRows - 1) * est * 4 + 15) & ~15LL);
  int8_t* vt = &VT[wave][0][0];
  // V tile transposed, 32 x 16 bytes (lane: row lr, 16 columns from jb) into VT[j][tt] for the 32 rows
  // tt. The four lanes of a quad hold four consecutive rows; two exchanges (lane ^ 1, lane ^ 2) with
  // byte selects leave lane 4k + c holding column c of each 4-column group for the quad's rows, one
  // word of VT.
  auto v_transpose = [&](const v4i_t v, int jb) {
    const int w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t x = (uint32_t)w4[d];
      const uint32_t y = (uint32_t)dpp_i<kDppXor1>((int)x);
      const uint32_t s1 = __builtin_amdgcn_perm(y, x, (lane & 1) ? 0x03070105u : 0x06020400u);
      const uint32_t y2 = (uint32_t)dpp_i<kDppXor2>((int)s1);
      const uint32_t col = __builtin_amdgcn_perm(y2, s1, (lane & 2) ? 0x03020706u : 0x05040100u);
      *(uint32_t*)&vt[(jb + 4 * d + (lane & 3)) * 32 + 4 * (lr >> 2)] = col;
    }
  };
  int* part = (int*)E;
  if constexpr (NW > 8) {
    // a wave per (32-column quarter q of V, tile group tg): the quarter's 32 x 32 bytes of each of the
    // group's tiles, up to PTV tiles in flight
    constexpr int NG = NW / KS;                       // tile groups (KS = 4 at these head dims)
    const int q = wave % KS, tg = wave / KS;
    v16i_t pv;
#pragma unroll
    for (int r = 0; r < 16; ++r) pv[r] = 0;
    for (int c0 = tg; tg < NG && c0 < ntile; c0 += NG * PTV) {
      v4i_t vb[PTV];
#pragma unroll
      for (int u = 0; u < PTV; ++u) {
        const int ti = c0 + NG * u;
        vb[u] = buffer_load16(vrs, ti < ntile ? (uint32_t)(32 * ti + lr) * kv_dim + g * HD + 32 * q + lk : kNoRow);
      }
#pragma unroll
      for (int u = 0; u < PTV; ++u) {
        const int ti = c0 + NG * u;
        if (ti >= ntile) break;
        // A: p of row pm, t = 32 ti + lk + 0..15 (rows 16..31 of the tile zero)
        const v4i_t pa = pm < kPreRows ? *(const v4i_t*)(pmrow + 32 * ti + lk) : v4i_t{0, 0, 0, 0};
        __builtin_amdgcn_wave_barrier();
        v_transpose(vb[u], lk);
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
        const v4i_t fb = *(const v4i_t*)&vt[lr * 32 + lk];
        pv = __builtin_amdgcn_mfma_i32_32x32x32_i8(pa, fb, pv, 0, 0, 0);
      }
    }
    // E is free: the waves' P.V partials are added into sums [16][HDP] by LDS integer atomics (int32
    // adds: exact in any order; |sum| <= 127 * 127 * T < 2^31)
    __syncthreads();
    for (int k = tid; k < kPreRows * HDP; k += NT) part[k] = 0;
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int m = (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
      if (tg < NG) atomicAdd(&part[m * HDP + 32 * q + lr], pv[r]);
    }
  } else {
    v16i_t pv[KS];
#pragma unroll
    for (int jt = 0; jt < KS; ++jt)
#pragma unroll
      for (int r = 0; r < 16; ++r) pv[jt][r] = 0;
    for (int c0 = wave; c0 < ntile; c0 += NW * PTV) {
      // V rows: lane takes row (lane & 31); in pass p the columns p VTC + (lane / 32) VTC / 2 + 16 q
      v4i_t vb[PTV][NPASS][QP];
#pragma unroll
      for (int u = 0; u < PTV; ++u) {
        const int ti = c0 + NW * u;
        const uint32_t off = ti < ntile ? (uint32_t)(32 * ti + lr) * kv_dim + g * HD + (lane >> 5) * (VTC / 2) : kNoRow;
#pragma unroll
        for (int p = 0; p < NPASS; ++p)
#pragma unroll
          for (int q = 0; q < QP; ++q) vb[u][p][q] = buffer_load16(vrs, off + p * VTC + 16 * q);
      }
#pragma unroll
      for (int u = 0; u < PTV; ++u) {
        const int ti = c0 + NW * u;
        if (ti >= ntile) break;
        const v4i_t pa = pm < kPreRows ? *(const v4i_t*)(pmrow + 32 * ti + lk) : v4i_t{0, 0, 0, 0};
#pragma unroll
        for (int p = 0; p < NPASS; ++p) {
          __builtin_amdgcn_wave_barrier();
#pragma unroll
          for (int q = 0; q < QP; ++q) v_transpose(vb[u][p][q], (lane >> 5) * (VTC / 2) + 16 * q);
          __builtin_amdgcn_s_waitcnt(0xc07f);
          __builtin_amdgcn_wave_barrier();
#pragma unroll
          for (int jt = p * VTC / 32; jt < (p + 1) * VTC / 32; ++jt) {
            const v4i_t fb = *(const v4i_t*)&vt[(32 * jt - p * VTC + lr) * 32 + lk];
            pv[jt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(pa, fb, pv[jt], 0, 0, 0);
          }
        }
      }
    }
    // E is free: the waves' P.V partials are added into sums [16][HDP] by LDS integer atomics (int32
    // adds: exact in any order; |sum| <= 127 * 127 * T < 2^31)
    __syncthreads();
    for (int k = tid; k < kPreRows * HDP; k += NT) part[k] = 0;
    __syncthreads();
#pragma unroll
    for (int jt = 0; jt < KS; ++jt)
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int m = (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        atomicAdd(&part[m * HDP + 32 * jt + lr], pv[jt][r]);
      }
  }
  __syncthreads();
  for (int k = tid; k < kPreRows * HD; k += NT) {
    const int m = k / HD, j = k % HD;
    if (s_T[m] == 0) continue;
    const int sum = part[m * HDP + j];
    if constexpr (OPT) {
      float o = (float)sum;
      if (a.qsum) o = o * qsum_scale(s_qs[m], tab);
      a.att[(long long)(r0 + m) * a.att_stride + (long long)h * HD + j] =
          o * (a.ch_av ? a.ch_av[(long long)g * HD + j] : a.a_v);
    } else {
      a.att[(long long)(r0 + m) * a.att_stride + (long long)h * HD + j] = (float)sum * a.a_v;
    }
  }
}

// dynamic LDS bytes of k_attn_pre: 16 rows of scores / exps (also the P.V sums afterwards)
inline size_t attn_pre_lds_bytes(int S, int HDP) {
  const size_t e = (size_t)kPreRows * pre_est(S) * 4, p = (size_t)kPreRows * HDP * 4;
  return e > p ? e : p;
}

// ------------------------------------------------------------------ prefill attention, 32-row blocks
// k_attn_pre's numerics without the HF options at head dims 128 (up to 2048 positions) and 64 (up to
// 512), one 512-thread workgroup per (query head, 32 rows): every K and V byte read serves 32 rows,
// and the MFMAs' 32 query columns / rows are all rows of the block. Wave w owns the key tiles (32
// keys) w, w + 8, ... (TW of them at the largest T) from the scores to P.V, and keeps them in
// registers:
//  - K tiles go global -> LDS by global_load_lds (whole rows, 16 rows of 64 bytes or 8 of 128 per
//    instruction; chunk kc of row r at 16-byte position CPR r + (kc ^ swz(r)), the GEMM operand
//    swizzle) into a ring of the wave's own; scores as S^T = K Q^T (v_mfma_i32_32x32x32_i8, A = the
//    tile's 32 keys, B = the block's int8 q): lane (n, half) holds row n's scores of keys
//    8 (r / 4) + 4 half + r % 4, r < 16;
//  - the row maximum (order-free) from each lane's, the two halves' and the waves' (LDS);
//  - e = EXP(s - max) in place (sfu_exp_sm) and the D-lane ordered sums: the waves' tiles of 256
//    keys at a time go to LDS and each chain lane (row, l < D) adds keys l, l + D, ... of the chunk in
//    order; chunks in key order, so every chain adds its keys in the reference's order (keys past T
//    are +0, which leave a sum of non-negative terms unchanged); then the pairwise tree over the D
//    lanes and RECIP;
//  - p = to_i8(F(F(e r) 127)) packed in the lane's own key order: the P.V MFMA's A operand (its k
//    order within a tile is that permutation of the keys; the V operand is gathered to match);
//  - P.V: the tile's V rows loaded whole (16-byte chunks, HD / 32 loads a lane), stored in the K
//    ring's layout to an LDS tile of the wave's own and read back transposed by the LDS transpose
//    read (ds_read_b64_tr_b8), two reads a B operand gathering column n's bytes of the A operand's
//    keys; HD / 32 MFMAs a tile;
//  - the waves' int32 sums added by LDS integer atomics (exact in any order) and scaled.
// HD 128 keeps 8 tiles a wave (128 score registers, one workgroup per CU, a four-tile K ring, two
// exp-chunk buffers); HD 64 keeps 2 (512 positions), so that two workgroups share a CU.
constexpr int kApRows = 32, kApThreads = 512, kApWaves = kApThreads / 64;
constexpr int kApStage = 256 + 16;                       // float stride of a row of a 256-key chunk
template <int HD> struct ApCfg;
template <> struct ApCfg<128> { static constexpr int TW = 8, RING = 4, NSB = 2, MINB = 1; };
template <> struct ApCfg<64> { static constexpr int TW = 2, RING = 2, NSB = 1, MINB = 2; };
template <int HD> constexpr int ap_keys() { return 32 * kApWaves * ApCfg<HD>::TW; }   // positions a row may attend to
// dynamic LDS: the waves' K rings, then (reused) the exp-chunk buffers, then (reused) the waves'
// transposed V tiles
template <int HD> constexpr size_t ap_lds() {
  constexpr size_t ring = (size_t)kApWaves * ApCfg<HD>::RING * 32 * HD;
  constexpr size_t stage = (size_t)ApCfg<HD>::NSB * kApRows * kApStage * 4;
  constexpr size_t vt = (size_t)kApWaves * HD * 32;
  return ring > stage ? (ring > vt ? ring : vt) : (stage > vt ? stage : vt);
}

// ds_read_b64_tr_b8 (gfx950 LDS transpose read): in each 16-lane group, lane 8 h + j receives as
// byte b (b < 8) the byte at the address supplied by the group's lane 2 b + h, plus j
T2R_DEV v2i_t lds_read_tr8(int8_t* p) {
  typedef __attribute__((address_space(3))) v2i_t lds_v2i_t;
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i_t*)p);
}

// Q8I: q comes quantized (a.q8 / a.q8s, the prep kernel's quant_act of each head vector): the
// block's rows are loaded straight into the score MFMA's B operands, and the SFU tables, the P.V sums'
// zeroing and the row bounds go to LDS after the scores, before the barrier the row maxima need
// anyway (no barrier before the scores).
template <int HD, bool Q8I>
__global__ __launch_bounds__(kApThreads, ApCfg<HD>::MINB) void k_attn_pw(AttnArgs a, int M) {
  constexpr int KS = HD / 32, NW = kApWaves, TW = ApCfg<HD>::TW, RING = ApCfg<HD>::RING, NSB = ApCfg<HD>::NSB;
  constexpr int CPR = HD / 16;                    // 16-byte chunks of a K row
  constexpr int NDMA = HD / 32;                   // DMA instructions (1 KB) a K tile
  constexpr int TB = 32 * HD;                     // bytes of a K tile
  constexpr int NQ = HD / 64;                     // q elements a lane and row
  constexpr int NV = HD / 32;                     // 16-byte V loads a lane and tile
  constexpr int NCT = HD / 32;                    // P.V column tiles
  constexpr int OST = HD + 8;                     // int32 stride of a row of the P.V sums
  extern __shared__ __align__(16) float big[];
  __shared__ __align__(16) float tab[kSfuWords];
  __shared__ __align__(16) float2 et[kSfuExpPairs];
  __shared__ __align__(16) int8_t Q8[kApRows][HD];
  __shared__ __align__(16) int O[kApRows * OST];
  __shared__ __align__(16) float s_mx[kApRows][NW];
  __shared__ float s_sq[kApRows], s_r[kApRows];
  __shared__ int s_T[kApRows];
  // row blocks longest first (a causal prompt's later rows attend to more positions)
  const int h = blockIdx.x, r0 = (gridDim.y - 1 - blockIdx.y) * kApRows, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6, n = lane & 31, half = lane >> 5;
  const int G = a.H / a.Hk, g = h / G, S = a.S, D = a.D;
  const int cap = a.t_cap > 0 && a.t_cap < S ? a.t_cap : S;
  const int kv_dim = a.Hk * HD;

  // ---- the loads that depend on nothing first, all unconditional and issued before the first wait
  // (a load under a branch makes the compiler's wait counts path-dependent, and it then waits for
  // each before the next is issued): lane n's row's position, which the K tiles' requests wait for;
  // q of the wave's rows (rows wave, wave + 8, ...), or (Q8I) lane n's row's int8 q, straight into
  // the score MFMA's B operands, and its scale; the SFU tables. Then the row's position bounds T
  // (rows past M or outside the cache: 0).
  const int pn = a.pos[min(r0 + n, M - 1)];
  float qx[kApRows / NW][NQ];
  v4i_t qb[KS];
  float sqn = 0.0f;
  if constexpr (Q8I) {
    const int rq = min(r0 + n, M - 1);
    const int8_t* q8 = a.q8 + (long long)rq * a.q8_stride + (long long)h * HD + 16 * half;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qb[ks] = *(const v4i_t*)(q8 + 32 * ks);
    sqn = a.q8s[(long long)rq * a.H + h];
  } else {
#pragma unroll
    for (int k = 0; k < kApRows / NW; ++k) {
      const int r = min(r0 + wave + NW * k, M - 1);
      const float* q = a.qkv + (long long)r * a.qkv_stride + (long long)h * HD;
#pragma unroll
      for (int e = 0; e < NQ; ++e) qx[k][e] = q[lane + 64 * e];
    }
  }
  const v4f_t tv = ((const v4f_t*)a.tab)[tid & (kSfuWords / 4 - 1)];      // (stored by tid < kSfuWords / 4)
  const float2 ev = sfu_exp_pair(min(tid, kSfuExpPairs - 1), a.tab);      // (stored by tid < kSfuExpPairs)
  const int Tn = r0 + n < M && pn >= 0 && pn < S ? min(pn + 1, cap) : 0;
  if constexpr (Q8I) sqn = Tn > 0 ? sqn : 0.0f;   // an invalid row (its q8 may be stale): scores 0
  const int ntile = ((int)wave_max_u32((uint32_t)Tn) + 31) / 32;   // lanes n cover the 32 rows
  const int nown = ntile > wave ? (ntile - wave + NW - 1) / NW : 0;  // tiles this wave owns

  // ---- the first RING - 1 owned K tiles requested (DMA into the wave's ring) before q's
  // quantisation. Rows past the cache are clamped to its last (their keys are past every T).
  auto swz = [](int r) { return CPR == 8 ? ((r ^ (r >> 3)) & 7) : ((r >> 2) & 3); };
  int8_t* ring = (int8_t*)big + wave * (RING * TB);
  const int8_t* kcol[NDMA];                          // this lane's 16-byte chunk of instruction i
#pragma unroll
  for (int i = 0; i < NDMA; ++i) {
    const int pos = 64 * i + lane, r = pos / CPR;
    kcol[i] = a.kc + (long long)g * HD + 16 * ((pos % CPR) ^ swz(r));
  }
  auto k_issue = [&](int j) {                        // owned tile j into ring slot j % RING
    const int ti = wave + NW * j;
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      const int row = min(32 * ti + (64 * i + lane) / CPR, S - 1);
      __builtin_amdgcn_global_load_lds((const void*)(kcol[i] + (long long)row * kv_dim),
                                       (void*)(ring + TB * (j % RING) + 1024 * i), 16, 0, 0);
    }
  };
#pragma unroll
  for (int j = 0; j < RING - 1; ++j)
    if (j < nown) k_issue(j);
  // the SFU tables, the P.V sums' zeroing and the row bounds (Q8I: after the scores)
  auto lds_setup = [&]() {
    for (int k = tid; k < kApRows * OST; k += kApThreads) O[k] = 0;
    if (wave == 0 && half == 0) s_T[n] = Tn;
    if (tid < kSfuWords / 4) ((v4f_t*)tab)[tid] = tv;
    if (tid < kSfuExpPairs) et[tid] = ev;
  };

  // ---- q of the block's rows to int8, a wave per row; invalid rows 0
  if constexpr (!Q8I) {
    lds_setup();
    __syncthreads();
    // the four rows' |q| maxima, then s_q = F(max (1/127)) and RECIP once for all four (lane k: row
    // wave + 8 k); an invalid row's multiplier 0 gives q8 = to_i8(0 or NaN) = 0
    uint32_t am[kApRows / NW];
#pragma unroll
    for (int k = 0; k < kApRows / NW; ++k) {
      uint32_t m = abs_bits(qx[k][0]);
#pragma unroll
      for (int e = 1; e < NQ; ++e) m = max(m, abs_bits(qx[k][e]));
      am[k] = wave_max_u32(m);
    }
    static_assert(kApRows / NW == 4, "four rows a wave");
    const uint32_t mine = lane == 0 ? am[0] : lane == 1 ? am[1] : lane == 2 ? am[2] : am[3];
    const float sq_l = fv(mine) * kInv127;
    const float inv_l = sfu_recip(sq_l, tab);
#pragma unroll
    for (int k = 0; k < kApRows / NW; ++k) {
      const int i = wave + NW * k;
      const bool ok = __shfl(Tn, i) > 0;            // lane i holds row i
      const float inv = ok ? fv((uint32_t)__builtin_amdgcn_readlane((int)fb(inv_l), k)) : 0.0f;
#pragma unroll
      for (int e = 0; e < NQ; ++e) Q8[i][lane + 64 * e] = (int8_t)to_i8(qx[k][e] * inv);
      if (lane == k) s_sq[i] = sq_l;
    }
    __syncthreads();
    sqn = s_sq[n];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qb[ks] = *(const v4i_t*)&Q8[n][32 * ks + 16 * half];
  }

  // ---- scores of the owned tiles: tile j + RING - 1 requested into the slot tile j - 1 left (its
  // fragments were read before its MFMAs), then wait for tile j's DMA (the newer ones may be in
  // flight), its A fragments from the ring and KS MFMAs. Tiles wholly below every valid row's T need
  // no mask.
  const int Tmin = (int)~wave_max_u32(~(Tn > 0 ? (uint32_t)Tn : 0xFFFFFFFFu));
  float sc[TW][16];
  float rmx = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < TW; ++j) {
    if (j >= nown) break;
    if (j + RING - 1 < nown) k_issue(j + RING - 1);
    const int newer = min(nown - 1, j + RING - 1) - j;      // tiles requested after tile j
    if (newer >= 3) __builtin_amdgcn_s_waitcnt(waitcnt_vm(3 * NDMA));
    else if (newer == 2) __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * NDMA));
    else if (newer == 1) __builtin_amdgcn_s_waitcnt(waitcnt_vm(NDMA));
    else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    asm volatile("" ::: "memory");
    const int8_t* kt = ring + TB * (j % RING);
    v4i_t ka[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) ka[ks] = *(const v4i_t*)(kt + 16 * (CPR * n + ((2 * ks + half) ^ swz(n))));
    v16i_t acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(ka[ks], qb[ks], acc, 0, 0, 0);
    const int ti = wave + NW * j;
    if (32 * ti + 32 <= Tmin) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        sc[j][r] = ((float)acc[r] * sqn) * a.a_k;
        rmx = smax(rmx, sc[j][r]);
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int t = 32 * ti + 8 * (r >> 2) + 4 * half + (r & 3);
        const float sv = ((float)acc[r] * sqn) * a.a_k;
        sc[j][r] = t < Tn ? sv : -__builtin_inff();
        rmx = smax(rmx, sc[j][r]);
      }
    }
  }
  rmx = smax(rmx, __shfl_xor(rmx, 32));
  if (half == 0) s_mx[n][wave] = rmx;
  if constexpr (Q8I) lds_setup();
  __syncthreads();
  float mx;
  {
    const v4f_t m0 = *(const v4f_t*)&s_mx[n][0], m1 = *(const v4f_t*)&s_mx[n][4];
    mx = smax(smax(smax(m0.x, m0.y), smax(m0.z, m0.w)), smax(smax(m1.x, m1.y), smax(m1.z, m1.w)));
  }
  // every valid row's maximum finite: its e sum is >= 1 (EXP(0) = 1 at the maximum), so
  // y = F(F(e r) 127) lies in [0, 127] and to_i8(y) is y's RNE integer
  const bool fast = __all(Tn == 0 || __builtin_isfinite(mx));

  // the first owned tiles' V rows requested now, in flight through the softmax (P.V below): load i
  // of a tile gives the lane chunk (64 i + lane) % CPR of row (64 i + lane) / CPR (rows past the
  // cache read 0 through the buffer's range; their p is 0)
  const __amdgpu_buffer_rsrc_t vrs = buffer_rsrc(a.vc, (uint32_t)S * kv_dim);
  auto v_load = [&](v4i_t (&dst)[NV], int j) {
    const int ti = wave + NW * j;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int pos = 64 * i + lane;
      dst[i] = buffer_load16(vrs, (uint32_t)(32 * ti + pos / CPR) * kv_dim + g * HD + 16 * (pos % CPR));
    }
  };
  v4i_t vb[NV], vn[NV], vn2[NV];
  if (nown > 0) v_load(vb, 0);
  if (nown > 1) v_load(vn, 1);

  // ---- e = EXP(s - max) in place, keys past T included (their s is -inf), and the D-lane ordered
  // sums, a 256-key chunk at a time: chunk k is tile 8 k + w of wave w (its slot k), whose exps the
  // wave forms and stores; then chain lane (row cr, l < D) adds keys l, l + D, ... of the chunk.
  // With a finite maximum e is k_attn_pre's (sfu_exp_sm = EXP on x <= 0, EXP(-inf) = 0). A row
  // whose maximum is not finite (NaN, +inf, or -inf over its keys) ends with every p = 0 in the
  // reference (its e sum is NaN, p = to_i8(NaN)); here s - max is NaN or -inf for all its keys,
  // sfu_exp_sm gives 0, the sum is 0 and p = to_i8(F(0 RECIP(0))) = 0 as well (the full to_i8 below).
  const int cpr = 64 / D, cr = wave * cpr + lane / D, cl = lane % D;
  const bool chain = cr < kApRows;
  const int nchunk = (ntile + NW - 1) / NW;
  // Key k of row n sits at float n kApStage + 4 ((k / 4) ^ ((n / 4) % 4)) + k % 4: the 16-byte stores
  // of 16 rows land in distinct bank groups, and a chain lane's 4-byte reads stay in one row's 16
  // banks. The XOR touches the low two bits of the 16-byte slot, so each lane's addresses are a lane
  // constant plus a fixed offset: the writer's slot 8 w + 2 rr + half -> wb[rr % 2] + 16 (rr / 2)
  // floats; a chain lane's keys l + 16 u (D 16) -> cb0 + 16 u, l + 8 u (D 8) -> cb[u % 2] + 16 (u / 2).
  const int sx = (n >> 2) & 3, cx = (cr >> 2) & 3;
  const int wb0 = n * kApStage + 4 * ((8 * wave + half) ^ sx), wb1 = n * kApStage + 4 * ((8 * wave + 2 + half) ^ sx);
  const int cb0 = cr * kApStage + 4 * ((cl >> 2) ^ cx) + (cl & 3);
  const int cb1 = cr * kApStage + 4 * ((2 + (cl >> 2)) ^ cx) + (cl & 3);      // D 8: odd u
  float acc = 0.0f;
#pragma unroll
  for (int k = 0; k < TW; ++k) {
    if (k >= nchunk) break;
    float* sb = big + (k % NSB) * (kApRows * kApStage);
    if (k < nown) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sc[k][r] = sfu_exp_sm(sc[k][r] - mx, et);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr)
        *(v4f_t*)(sb + ((rr & 1) ? wb1 : wb0) + 16 * (rr >> 1)) =
            v4f_t{sc[k][4 * rr], sc[k][4 * rr + 1], sc[k][4 * rr + 2], sc[k][4 * rr + 3]};
    } else {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) *(v4f_t*)(sb + ((rr & 1) ? wb1 : wb0) + 16 * (rr >> 1)) = v4f_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
    __syncthreads();
    if (chain) {
      if (D == 16) {
        const float* c0 = sb + cb0;
#pragma unroll
        for (int h8 = 0; h8 < 2; ++h8) {
          float e[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) e[u] = c0[16 * (8 * h8 + u)];
#pragma unroll
          for (int u = 0; u < 8; ++u) acc = acc + e[u];
        }
      } else {
        const float* c0 = sb + cb0;
        const float* c1 = sb + cb1;
#pragma unroll
        for (int h8 = 0; h8 < 4; ++h8) {
          float e[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) e[u] = (u & 1) ? c1[16 * ((8 * h8 + u) >> 1)] : c0[16 * ((8 * h8 + u) >> 1)];
#pragma unroll
          for (int u = 0; u < 8; ++u) acc = acc + e[u];
        }
      }
    }
    if (NSB == 1 && k + 1 < nchunk) __syncthreads();   // one buffer: its reads before the next stores
  }
  // pairwise tree over the row's D lanes (within a 16-lane DPP row), RECIP on the row's first lane
  {
    float o = dpp_f<0x101>(acc);                  // row_shl:1
    if (D > 1 && (cl & 1) == 0) acc = acc + o;
    o = dpp_f<0x102>(acc);
    if (D > 2 && (cl & 3) == 0) acc = acc + o;
    o = dpp_f<0x104>(acc);
    if (D > 4 && (cl & 7) == 0) acc = acc + o;
    o = dpp_f<0x108>(acc);
    if (D > 8 && (cl & 15) == 0) acc = acc + o;
    if (chain && cl == 0) s_r[cr] = sfu_recip(acc, tab);
  }
  __syncthreads();

  // ---- p = to_i8(F(F(e r) 127)) of the owned tiles, 16 bytes a lane and tile (the A operand)
  v4i_t pa[TW];
  {
    const float rn = s_r[n];
    auto pack = [&](int j, auto to_byte) {
      uint32_t w4[4];
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        uint32_t b[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) b[c] = to_byte((sc[j][4 * rr + c] * rn) * 127.0f);
        const uint32_t lo = __builtin_amdgcn_perm(b[1], b[0], 0x0C0C0400u);   // bytes b0[0], b1[0]
        const uint32_t hi = __builtin_amdgcn_perm(b[3], b[2], 0x0C0C0400u);
        w4[rr] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
      }
      pa[j] = v4i_t{(int)w4[0], (int)w4[1], (int)w4[2], (int)w4[3]};
    };
    if (fast) {
      // y in [0, 127]: v_cvt_pk_u8_f32 converts with round-to-nearest-even (checked on the device
      // over every half-way point of [0, 128)) and inserts the byte, four to a word
#pragma unroll
      for (int j = 0; j < TW; ++j)
        if (j < nown) {
          uint32_t w4[4];
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            uint32_t w = 0;
#pragma unroll
            for (int c = 0; c < 4; ++c) w = __builtin_amdgcn_cvt_pk_u8_f32((sc[j][4 * rr + c] * rn) * 127.0f, c, w);
            w4[rr] = w;
          }
          pa[j] = v4i_t{(int)w4[0], (int)w4[1], (int)w4[2], (int)w4[3]};
        }
    } else {
#pragma unroll
      for (int j = 0; j < TW; ++j)
        if (j < nown) pack(j, [](float y) { return (uint32_t)to_i8(y); });
    }
  }

  // ---- P.V of the owned tiles: a tile's V rows stored as loaded, row r's chunk kc at 16-byte slot
  // CPR r + (kc ^ swz(r)) of the wave's LDS tile (the K ring's layout), and read back transposed
  // (lds_read_tr8). The B operand of lane (column n, half) is column 32 c + n over keys
  // 8 (q / 4) + 4 half + q % 4, q < 16 (the A operand's key order): its read t (bytes q = 8 t ..)
  // takes, from group lane k, row 16 t + 8 (k / 8) + 4 half + (k / 2) % 4 at column
  // 32 c + 16 (group % 2) + 8 (k % 2). The stores of a 16-lane pass and each group's reads meet
  // distinct 16-byte bank groups.
  int8_t* vt = (int8_t*)big + wave * TB;
  uint32_t tra[NCT][2];                            // the lane's read addresses in the tile
  {
    const int gq = lane >> 4, b = (lane & 15) >> 1;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int row = 16 * t + 8 * (b >> 2) + 4 * (gq >> 1) + (b & 3);
#pragma unroll
      for (int c = 0; c < NCT; ++c)
        tra[c][t] = (uint32_t)(row * HD + 16 * ((2 * c + (gq & 1)) ^ swz(row)) + 8 * (lane & 1));
    }
  }
  v16i_t pv[NCT];
#pragma unroll
  for (int c = 0; c < NCT; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) pv[c][r] = 0;
#pragma unroll
  for (int j = 0; j < TW; ++j) {
    if (j >= nown) break;
    if (j + 2 < nown) v_load(vn2, j + 2);
    __builtin_amdgcn_wave_barrier();                // the previous tile's operand reads come first
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int pos = 64 * i + lane, r = pos / CPR;
      *(v4i_t*)(vt + 16 * (CPR * r + ((pos % CPR) ^ swz(r)))) = vb[i];
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);              // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int c = 0; c < NCT; ++c) {
      const v2i_t lo = lds_read_tr8(vt + tra[c][0]), hi = lds_read_tr8(vt + tra[c][1]);
      pv[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(pa[j], v4i_t{lo.x, lo.y, hi.x, hi.y}, pv[c], 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      vb[i] = vn[i];
      vn[i] = vn2[i];
    }
  }

  // ---- the waves' sums (exact int32 atomics), then att = F(f32(sum) a_v) of the valid rows
  if (nown > 0) {
#pragma unroll
    for (int c = 0; c < NCT; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = 8 * (r >> 2) + 4 * half + (r & 3);
        atomicAdd(&O[m * OST + 32 * c + n], pv[c][r]);
      }
  }
  __syncthreads();
  {
    constexpr int CPT = HD / 16;                   // output columns a thread
    const int m = tid >> 4, c0 = CPT * (tid & 15);
    if (s_T[m] > 0) {
      float* out = a.att + (long long)(r0 + m) * a.att_stride + (long long)h * HD + c0;
#pragma unroll
      for (int u = 0; u < CPT / 4; ++u) {
        const v4i_t sv = *(const v4i_t*)&O[m * OST + c0 + 4 * u];
        *(v4f_t*)(out + 4 * u) = v4f_t{(float)sv.x * a.a_v, (float)sv.y * a.a_v, (float)sv.z * a.a_v, (float)sv.w * a.a_v};
      }
    }
  }
}

// dynamic LDS bytes of k_attn: the scores (lane-major, D * osum_stride(S, D) floats) and the int8
// probabilities of S cache rows
inline size_t attn_lds_bytes(int S, int D) { return (size_t)D * osum_stride(S, D) * 4 + (size_t)S; }
// dynamic LDS bytes of k_attn_dec: the scores (lane-major), one spare slot per lane, then the int8
// probabilities of every row slot of the passes (S rounded up to a pass, <= S + 4096)
inline size_t attn_dec_lds_bytes(int S, int D) { return ((size_t)D * osum_stride(S, D) + 64) * 4 + (size_t)S + 4096; }

// ------------------------------------------------------------------ grouped decode attention
// Decode attention of the G <= 4 query heads that share a KV head, split over G / GW workgroups per
// (row, KV head g), each taking GW of the group's query heads (2 for four-head groups, else 1): the
// numerics are k_attn_dec's step for step, the work is split differently.
//  - Vector jobs, one per wave: the KV head (k: QK-norm, RoPE, int8; v: int8; the cache row) and
//    the workgroup's GW query heads (QK-norm, RoPE, quant_act). Every workgroup of the KV head forms
//    its new row; split 0 is the only one that writes it to the cache.
//  - Scores: the K rows are read once per workgroup, straight into the MFMA B layout (lane = key
//    row, 16 k-bytes), and v_mfma_i32_32x32x32_i8 takes the GW int8 q vectors as its A rows (rows
//    past GW zero): exact int32 dot products of its heads, 32 keys per instruction pair.
//  - Per key, the GW heads' EXPs side by side (independent table-lookup chains); per head the
//    D-lane ordered sum (one wave each) and RECIP; then the int8 probabilities of every (head, key)
//    into LDS rows, so P.V reads one word per four consecutive keys and head.
//  - P.V: a thread takes four consecutive V rows of one 16-byte chunk, transposes them once
//    (4 x 4 bytes, v_perm) for all G heads' v_dot4s; partial sums meet by DPP within 16-lane rows,
//    then in LDS, one slot per (wave, row of 16 lanes): no atomics.
constexpr int kGqaThreads = 512, kGqaWaves = kGqaThreads / 64, kGqaMaxG = 4;   // G + 1 <= 8 vector jobs
constexpr int kGqaRK = 4;                        // key tiles (32 rows) per wave per pass

// dynamic LDS: per head the lane-major scores (D P floats + 64 spare), then per head S int8 p; the
// kernels are set up for up to kGqaMaxLds (two heads of an 8192-position cache)
constexpr size_t kGqaMaxLds = 96 * 1024;
inline size_t attn_gqa_lds_bytes(int S, int D, int G) {
  return (size_t)G * ((size_t)D * osum_stride(S, D) + 64) * 4 + (size_t)G * ((S + 15) & ~15);
}

// GW: query heads per workgroup (G a multiple of GW): a KV head's group is split over G / GW
// workgroups (blockIdx.x = KV head * splits + split); each computes the KV head's new row for
// itself, and split 0 writes it to the cache.
template <int NCH, bool OPT, int GW>   // hd = 16 NCH (64 or 128); OPT: HF options
__global__ __launch_bounds__(kGqaThreads) void k_attn_gqa(AttnArgs a) {
  constexpr int HD = 16 * NCH, KS = HD / 32;                // MFMA k-steps per key tile
  constexpr int NCHP = NCH;                                 // (4 or 8: a power of two)
  constexpr int TS = kGqaThreads / NCHP;                    // V row slices (4 rows each)
  constexpr int RQ = 2;                                     // 4-row groups per thread per pass
  constexpr int NV = HD > 64 ? 2 : 1;                       // head-vector floats per lane
  static_assert(HD == 64 || HD == 128, "k_attn_gqa: hd 64 or 128");
  extern __shared__ __align__(16) float dyn[];
  __shared__ __align__(16) float tab[kSfuWords];
  static_assert(GW >= 1 && GW <= kGqaMaxG, "k_attn_gqa: 1..4 query heads per workgroup");
  __shared__ __align__(16) int8_t s_q8[GW][HD];
  __shared__ __align__(16) int8_t s_k8[HD], s_v8[HD];
  __shared__ __align__(16) float s_vec[kGqaWaves][HD];
  __shared__ float s_sq[GW], s_r[GW];
  __shared__ float red[kGqaWaves][GW];
  __shared__ int s_qs[kGqaWaves][GW];
  __shared__ int part[kGqaWaves * 4][GW * HD];

  const int row = blockIdx.y, tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lr = lane & 31, kh = lane >> 5;
  const int G = a.H / a.Hk, S = a.S, D = a.D, P = osum_stride(S, D), SH = D * P + 64;
  const int NSPL = G / GW;                       // workgroups per KV head
  const int g = (int)blockIdx.x / NSPL, spl = (int)blockIdx.x - g * NSPL;
  const int GH = GW;                             // query heads of this workgroup
  const int h0 = g * G + spl * GW;               // its first query head
  const int SP = (S + 15) & ~15;                 // int8 p row stride
  int8_t* pq = (int8_t*)(dyn + GH * SH);
  a.kc += row * a.kv_row_stride;                 // this row's sequence cache
  a.vc += row * a.kv_row_stride;
  const long long q_dim = (long long)a.H * HD;
  const int kv_dim = a.Hk * HD;
  // ---- issue: the position (a vector load, so that its wait leaves the later loads in flight), the
  // SFU tables and this wave's vector job inputs, none of which depend on it; then the RoPE rows and
  // the first pass of K tiles and V chunks. No branch before the position's wait (it would let the
  // compiler sink the loads below it): a position outside the cache runs as position 0 and writes
  // nothing (no cache row, no output; the status bit at the end).
  const int pos_v = (int)__builtin_amdgcn_raw_buffer_load_b32(buffer_rsrc_u(a.pos + row, 4), 0, 0, 0);
  const float* qkv = a.qkv + row * a.qkv_stride;
  v4f_t tb[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) tb[k] = ((const v4f_t*)a.tab)[(lane + 64 * k) & (kSfuWords / 4 - 1)];
  const int job = wave;                          // 0: the KV head, 1 .. GH: query head job - 1 (GH < waves)
  const bool has_job = job <= GH;
  const int hq = h0 + (job - 1);                 // global query head of job >= 1
  const float* va = job == 0 ? qkv + q_dim + (long long)g * HD : qkv + (long long)(has_job ? hq : 0) * HD;
  const float* vb = job == 0 ? qkv + q_dim + kv_dim + (long long)g * HD : va;
  const float* gn = job == 0 ? a.kn : a.qn;
  const bool norm = gn != nullptr;
  if (!norm) gn = va;                            // any readable address: the values are unused
  float xa[NV], xb[NV], xg[NV], cs[NV], sn[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int j = min(lane + 64 * k, HD - 1);
    xa[k] = va[j];
    xb[k] = vb[j];
    xg[k] = gn[j];
  }
  // OPT: per-channel scales of the KV head (job 0: 1 / s_k, 1 / s_v; query jobs: the q multiplier
  // s_k), loaded unconditionally from a readable address when absent
  float xc1[NV], xc2[NV];
  if constexpr (OPT) {
    const float* c1 = job == 0 ? a.ch_isk : a.ch_sk;
    c1 = c1 ? c1 + (long long)g * HD : va;
    const float* c2 = job == 0 && a.ch_isv ? a.ch_isv + (long long)g * HD : va;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int j = min(lane + 64 * k, HD - 1);
      xc1[k] = c1[j];
      xc2[k] = c2[j];
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  const int pos_in = __builtin_amdgcn_readfirstlane(pos_v);
  const bool pos_ok = pos_in >= 0 && pos_in < S;
  const int pos = pos_ok ? pos_in : 0;
  const int T = pos + 1;
  // cache rows [0, pos) of this KV head's columns: rows past pos - 1 read as zero
  const __amdgpu_buffer_rsrc_t krs = buffer_rsrc_u(a.kc + (long long)g * HD, (uint32_t)pos * kv_dim);
  const __amdgpu_buffer_rsrc_t vrs = buffer_rsrc_u(a.vc + (long long)g * HD, (uint32_t)pos * kv_dim);
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const long long ip = (long long)pos * (HD / 2) + (min(lane + 64 * k, HD - 1) >> 1);
    cs[k] = a.cos_t[ip];
    sn[k] = a.sin_t[ip];
  }
  __builtin_amdgcn_sched_barrier(0);
  v4i_t kw[kGqaRK][KS];
  auto load_k = [&](int pass) {
#pragma unroll
    for (int i = 0; i < kGqaRK; ++i) {
      const int t = 32 * (pass * kGqaWaves * kGqaRK + wave + kGqaWaves * i) + lr;
#pragma unroll
      for (int s = 0; s < KS; ++s) kw[i][s] = buffer_load16(krs, (uint32_t)t * kv_dim + 32 * s + 16 * kh);
    }
  };
  const int c = tid & (NCHP - 1), ts = tid / NCHP;
  v4i_t vw[RQ][4];                               // rows 4 (ts + TS j) + u
  auto load_v = [&](int base) {
#pragma unroll
    for (int j = 0; j < RQ; ++j)
#pragma unroll
      for (int u = 0; u < 4; ++u) vw[j][u] = buffer_load16(vrs, (uint32_t)(base + 4 * (ts + TS * j) + u) * kv_dim + 16 * c);
  };
  load_k(0);
  load_v(0);
  __builtin_amdgcn_sched_barrier(0);

  // ---- tables to LDS (each wave writes all of them, so it needs only its own stores); the jobs
#pragma unroll
  for (int k = 0; k < 2; ++k) ((v4f_t*)tab)[lane + 64 * k] = tb[k];
  __builtin_amdgcn_s_waitcnt(0xc07f);            // lgkmcnt(0): this wave's table stores are done
  __builtin_amdgcn_wave_barrier();
  if (has_job) {
    if (norm) {
      float* vec = s_vec[wave];
#pragma unroll
      for (int k = 0; k < NV; ++k)
        if (lane + 64 * k < HD) vec[lane + 64 * k] = xa[k];
      __builtin_amdgcn_s_waitcnt(0xc07f);
      __builtin_amdgcn_wave_barrier();
      float ss = 0.0f;
      if (lane < D) ss = ordered_sum<true>(vec, HD, D, lane);
      const float r = sfu_rsqrt(__shfl(ss, 0) * a.inv_hd + a.eps, tab);
#pragma unroll
      for (int k = 0; k < NV; ++k) xa[k] = (xa[k] * r) * xg[k];
    }
    float xr[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const float partner = dpp_f<kDppXor1>(xa[k]);
      xr[k] = (lane & 1) ? (xa[k] * cs[k]) + (partner * sn[k]) : (xa[k] * cs[k]) + ((-partner) * sn[k]);
    }
    if (job == 0) {
      const long long crow = (long long)pos * kv_dim + (long long)g * HD;
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const int j = lane + 64 * k;
        float isk = a.inv_sk, isv = a.inv_sv;
        if constexpr (OPT) {
          if (a.ch_isk) isk = xc1[k];
          if (a.ch_isv) isv = xc2[k];
        }
        const int8_t kb = (int8_t)to_i8(xr[k] * isk), vb8 = (int8_t)to_i8(xb[k] * isv);
        if (j < HD) {
          s_k8[j] = kb;
          s_v8[j] = vb8;
          if (spl == 0 && pos_ok) {
            a.kc[crow + j] = kb;
            a.vc[crow + j] = vb8;
          }
        }
      }
    } else {
      if constexpr (OPT) {
        if (a.ch_sk) {                           // K per channel: its scales folded into q
#pragma unroll
          for (int k = 0; k < NV; ++k) xr[k] = xr[k] * xc1[k];
        }
      }
      uint32_t am = 0;
#pragma unroll
      for (int k = 0; k < NV; ++k)
        if (lane + 64 * k < HD) am = max(am, abs_bits(xr[k]));       // lanes past HD hold no element
      const float sq = fv(wave_max_u32(am)) * kInv127;
      const float inv = sfu_recip(sq, tab);
#pragma unroll
      for (int k = 0; k < NV; ++k)
        if (lane + 64 * k < HD) s_q8[job - 1][lane + 64 * k] = (int8_t)to_i8(xr[k] * inv);
      if (lane == 0) s_sq[job - 1] = sq;
    }
  }
  __syncthreads();

  // ---- scores of the workgroup's GH heads: C[head][key] = q8[head] . k8[key] on MFMA, 32 keys per tile.
  // Lane (lr, kh) holds key lr of the tile and heads 4 kh + r (r < 4) in acc[r].
  v4i_t qa[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const v4i_t z = {0, 0, 0, 0};
    qa[s] = lr < GH ? *(const v4i_t*)(&s_q8[lr < GH ? lr : 0][32 * s + 16 * kh]) : z;
  }
  float sqh[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) sqh[r] = s_sq[r < GH ? r : 0];
  const int ntile = (T + 31) >> 5;
  const int npk = (ntile + kGqaWaves * kGqaRK - 1) / (kGqaWaves * kGqaRK);
  float mloc[4] = {-__builtin_inff(), -__builtin_inff(), -__builtin_inff(), -__builtin_inff()};
  for (int pass = 0; pass < npk; ++pass) {
    if (pass > 0) load_k(pass);
#pragma unroll
    for (int i = 0; i < kGqaRK; ++i) {
      const int t0 = 32 * (pass * kGqaWaves * kGqaRK + wave + kGqaWaves * i);
      if (t0 >= T) break;                        // (wave-uniform)
      const int t = t0 + lr;
      v16i_t acc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = 0;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const v4i_t kn = t == pos ? *(const v4i_t*)(&s_k8[32 * s + 16 * kh]) : kw[i][s];
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(qa[s], kn, acc, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int h = 4 * kh + r;
        const bool ok = h < GH && t < T;
        const float sv = ((float)acc[r] * sqh[r]) * a.a_k;
        dyn[ok ? h * SH + osum_index(t, D, P) : (r < GH ? r : 0) * SH + D * P + lane] = sv;   // (spare slot)
        mloc[r] = nanmax(mloc[r], ok ? sv : -__builtin_inff());
      }
    }
  }
  // per head: the maximum over the wave's 32 lanes of half kh = 0 (G <= 4), then over the waves
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float v = mloc[r];
    v = nanmax(v, dpp_f<kDppXor1>(v));
    v = nanmax(v, dpp_f<kDppXor2>(v));
    v = nanmax(v, dpp_f<kDppHalfMirror>(v));
    v = nanmax(v, dpp_f<kDppMirror>(v));
    const float m0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float m1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    if (lane == 0 && r < GH) red[wave][r] = nanmax(m0, m1);
  }
  __syncthreads();

  // ---- e = EXP(s - m) (+0 padding to a multiple of D), key t by thread t % 512, all heads at once
  const int Tpad = ((T + D - 1) / D) * D;
  float mh[GW];
#pragma unroll
  for (int r = 0; r < GW; ++r) {
    const int h = r < GH ? r : 0;
    float m = red[0][h];
#pragma unroll
    for (int w = 1; w < kGqaWaves; ++w) m = nanmax(m, red[w][h]);
    mh[r] = m;
  }
  for (int t = tid; t < Tpad; t += kGqaThreads) {
    const int k = osum_index(t, D, P);
    float sv[GW], ev[GW];
#pragma unroll
    for (int h = 0; h < GW; ++h) sv[h] = dyn[(h < GH ? h : 0) * SH + k];
#pragma unroll
    for (int h = 0; h < GW; ++h) ev[h] = sfu_exp_np(sv[h] - mh[h], tab);
#pragma unroll
    for (int h = 0; h < GW; ++h)
      if (h < GH) dyn[h * SH + k] = t < T ? ev[h] : 0.0f;
  }
  __syncthreads();
  if (wave < GH) {
    float ssum = 0.0f;
    if (lane < D) ssum = ordered_sum_t<false>(dyn + wave * SH, T, D, P, lane);
    if (lane == 0) s_r[wave] = (OPT && a.qsum) ? 1.0f : sfu_recip(ssum, tab);   // qsum: to_i8(F(F(e * 1) * 127))
  }
  __syncthreads();

  // ---- the int8 probabilities p = to_i8(F(F(e r) 127)) of every (head, key) in [0, T4), zero past T
  float rh[GW];
#pragma unroll
  for (int r = 0; r < GW; ++r) rh[r] = s_r[r < GH ? r : 0];
  const int T4 = (T + 3) & ~3;
  int qs[GW];                                    // qsum: the probabilities of the thread's keys, per head
#pragma unroll
  for (int h = 0; h < GW; ++h) qs[h] = 0;
  for (int t = tid; t < T4; t += kGqaThreads) {
    const int k = osum_index(min(t, T - 1), D, P);
    float ev[GW];
#pragma unroll
    for (int h = 0; h < GW; ++h) ev[h] = dyn[(h < GH ? h : 0) * SH + k];
#pragma unroll
    for (int h = 0; h < GW; ++h)
      if (h < GH) {
        const int p = t < T ? to_i8((ev[h] * rh[h]) * 127.0f) : 0;
        pq[h * SP + t] = (int8_t)p;
        if (OPT) qs[h] += p;
      }
  }
  if (OPT && a.qsum) {
#pragma unroll
    for (int h = 0; h < GW; ++h) {
      const int v = wave_sum_i32(qs[h]);
      if (lane == 0) s_qs[wave][h] = v;
    }
  }
  __syncthreads();

  // ---- P.V: thread (chunk c, row slice ts) takes rows 4 (ts + TS j) + u; the four rows' V chunks
  // transposed once, then per head one word of four p against each column word
  int vpos[4];
#pragma unroll
  for (int w = 0; w < 4; ++w) vpos[w] = ((const int*)s_v8)[4 * c + w];
  int acc[GW][16];
#pragma unroll
  for (int h = 0; h < GW; ++h)
#pragma unroll
    for (int b = 0; b < 16; ++b) acc[h][b] = 0;
  const int npv = (T + 4 * TS * RQ - 1) / (4 * TS * RQ);
  for (int pass = 0; pass < npv; ++pass) {
    const int base = pass * 4 * TS * RQ;
    if (pass > 0) load_v(base);
#pragma unroll
    for (int j = 0; j < RQ; ++j) {
      const int t0 = base + 4 * (ts + TS * j);
      if (t0 < T) {
        int rw[4][4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int w = 0; w < 4; ++w) rw[u][w] = t0 + u == pos ? vpos[w] : vw[j][u][w];
        int col[4][4];
#pragma unroll
        for (int w = 0; w < 4; ++w) transpose4x4(rw[0][w], rw[1][w], rw[2][w], rw[3][w], col[w]);
        int pp[GW];
#pragma unroll
        for (int h = 0; h < GW; ++h) pp[h] = *(const int*)(pq + (h < GH ? h : 0) * SP + t0);
#pragma unroll
        for (int h = 0; h < GW; ++h)
#pragma unroll
          for (int w = 0; w < 4; ++w)
#pragma unroll
            for (int k = 0; k < 4; ++k) acc[h][4 * w + k] = __builtin_amdgcn_sdot4(col[w][k], pp[h], acc[h][4 * w + k], false);
      }
    }
  }
  // lanes of a 16-lane row with the same chunk rotate-and-add over the row-slice bits; then one
  // partial row per (wave, row of 16 lanes) in LDS, summed by (head, column)
#pragma unroll
  for (int h = 0; h < GW; ++h)
#pragma unroll
    for (int b = 0; b < 16; ++b) {
      int v = acc[h][b];
      if (NCHP <= 2) v += dpp_i<0x122>(v);                    // row_ror:2
      if (NCHP <= 4) v += dpp_i<0x124>(v);                    // row_ror:4
      if (NCHP <= 8) v += dpp_i<0x128>(v);                    // row_ror:8
      acc[h][b] = v;
    }
  if ((lane & 15) < NCHP) {
#pragma unroll
    for (int h = 0; h < GW; ++h)
      if (h < GH)
#pragma unroll
        for (int b = 0; b < 16; ++b) part[wave * 4 + (lane >> 4)][h * HD + 16 * c + b] = acc[h][b];
  }
  __syncthreads();
  if (!pos_ok) {
    if (tid == 0) flag_bad_pos(a.status);
    return;
  }
  float* out = a.att + row * a.att_stride;
  for (int idx = tid; idx < GH * HD; idx += kGqaThreads) {
    int ssum = 0;
#pragma unroll
    for (int w = 0; w < kGqaWaves * 4; ++w) ssum += part[w][idx];
    const int h = idx / HD, j = idx - h * HD;
    if constexpr (OPT) {
      float o = (float)ssum;
      if (a.qsum) {
        int tot = 0;
#pragma unroll
        for (int w = 0; w < kGqaWaves; ++w) tot += s_qs[w][h];
        o = o * qsum_scale(tot, tab);
      }
      out[(long long)(h0 + h) * HD + j] = o * (a.ch_av ? a.ch_av[(long long)g * HD + j] : a.a_v);
    } else {
      out[(long long)(h0 + h) * HD + j] = (float)ssum * a.a_v;
    }
  }
}

}  // namespace t2r
