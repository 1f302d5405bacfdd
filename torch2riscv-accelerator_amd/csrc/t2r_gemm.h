// W8A8 GEMM over prefill rows on CDNA4 int8 MFMA: acc[M, N] = xq[M, K] . W[N, K]^T in exact int32
// (v_mfma_i32_32x32x32_i8), then per element y = F(F(f32(acc) * s_w[n]) * s_x[m]) with the same
// epilogues as the decode GEMV (store, residual add, SwiGLU gate) (expandLinearRows,
// compiler/plugins/sa/transforms/SahlExpandKernels.cpp:205; the rows are independent, so one pass
// over all prompt rows gives the logits and KV of row-by-row decoding bit for bit).
//
// Tiling: a wave computes a 64 x 64 block of C as 2 x 2 MFMA tiles of 32 x 32; a workgroup is
// WM x WN waves (BM = 64 WM rows, BN = 64 WN columns). K advances by 64: the next K-slab of A and B
// is loaded from global memory into registers while the MFMAs consume the current slab from LDS
// (two LDS buffers, rows padded to 80 bytes). Every lane feeds an MFMA 16 consecutive k-values of
// its A row and of its B column, the same k for both operands, so the product is the exact sum
// whatever order the instruction pairs them in. SwiGLU: the B tile's columns alternate 32 rows
// of W1 and the same 32 rows of W3, so a lane holds h1 and h3 of the same (m, n).
#pragma once
#include "t2r_gemv.h"
#include <type_traits>

namespace t2r {

__host__ __device__ inline int cdiv_i(long long a, long long b) { return (int)((a + b - 1) / b); }

// ------------------------------------------------------------------ GEMV launcher (decode, op level)
// The GEMV over `rows` activation rows (grid y) with register-slice width NCB (by K), RU rows per
// wave and NT threads per block. Every block repeats the prologue over the whole input, so fewer,
// larger tiles repeat it less: RU is the largest that still leaves >= 768 waves (3 per CU), and a
// long input (NCB >= 4) takes 512-thread blocks. (Measured on the Llama-3.2-1B decode shapes:
// W1/W3 8192 x 2048 best at RU 4 / 256 threads, Wqkv 3072 x 2048 at RU 4, Wo 2048 x 2048 at RU 2,
// W2 2048 x 8192 at 512 threads.)
template <int NCB>
constexpr int gemv_rumax() { return NCB <= 2 ? 4 : (NCB == 4 ? 2 : 1); }

struct GemvShape {
  int ru, nt, blocks;
};

template <int NCB>
inline GemvShape gemv_shape(int N) {
  GemvShape g;
  g.ru = 1;
  while (g.ru < gemv_rumax<NCB>() && (long long)N / (2 * g.ru) >= 768) g.ru *= 2;
  const int waves = cdiv_i(N, g.ru);
  g.nt = NCB >= 4 ? 512 : 256;
  g.blocks = cdiv_i(waves, g.nt / 64);
  // at most 3072 waves (three per SIMD); a longer N walks more tiles per wave. Measured on the
  // Llama-3.2-1B classifier (128256 rows): 42.6 us at 3072 waves against 46.6 at 8192, 45.2 at 4096
  // and 43.7 at 2048.
  const int cap = 3072 * 64 / g.nt;
  if (g.blocks > cap) g.blocks = cap;
  return g;
}

template <int PRO, int EPI, int NCB, int NT, bool IDX>
void gemv_launch_nt(const GemvArgs& a, int rows, int ru, int blocks, hipStream_t st) {
  constexpr int RUMAX = gemv_rumax<NCB>();
  dim3 grid(blocks, rows), block(NT);
  if (ru == 1) launch((k_gemv<PRO, EPI, NCB, 1, NT, IDX>), grid, block, 0, st, a);
  else if (ru == 2) launch((k_gemv<PRO, EPI, NCB, (RUMAX >= 2 ? 2 : 1), NT, IDX>), grid, block, 0, st, a);
  else launch((k_gemv<PRO, EPI, NCB, RUMAX, NT, IDX>), grid, block, 0, st, a);
}

// MoE id indirection (a.ids) exists for the expert gate / up GEMV only (int8 input, SwiGLU).
template <int PRO, int EPI, int NCB>
int gemv_launch_shape(const GemvArgs& a, int rows, GemvShape g, hipStream_t st) {
  if (g.ru < 1 || g.ru > gemv_rumax<NCB>() || (g.ru & (g.ru - 1)) || g.blocks < 1) return -2;
  if (g.nt != 256 && g.nt != 512) return -2;
  if (a.ids != nullptr) {
    if constexpr (PRO == PRO_XQ && EPI == EPI_SWIGLU) {
      if (a.rows_per_id <= 0 || a.N % a.rows_per_id) return -2;
      if (g.nt == 512) gemv_launch_nt<PRO, EPI, NCB, 512, true>(a, rows, g.ru, g.blocks, st);
      else gemv_launch_nt<PRO, EPI, NCB, 256, true>(a, rows, g.ru, g.blocks, st);
    } else {
      return -2;
    }
  } else if (g.nt == 512) {
    gemv_launch_nt<PRO, EPI, NCB, 512, false>(a, rows, g.ru, g.blocks, st);
  } else {
    gemv_launch_nt<PRO, EPI, NCB, 256, false>(a, rows, g.ru, g.blocks, st);
  }
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

// Operand checks: the staged loads read the activations (and the SFU tables) 16 bytes at a time.
template <int PRO, int EPI>
inline bool gemv_operands_ok(const GemvArgs& a) {
  if ((PRO != PRO_XQ || EPI == EPI_SWIGLU) && (a.tab == nullptr || ((uintptr_t)a.tab & 15))) return false;
  if (PRO == PRO_XQ) return ((uintptr_t)a.xq & 15) == 0 && a.xq_stride % 16 == 0;
  if (PRO == PRO_SPLITQ) return a.xs != nullptr && ((uintptr_t)a.xs & 15) == 0 && a.xs_stride % 4 == 0 && a.K % 4 == 0;
  if (((uintptr_t)a.x & 15) || a.x_stride % 4) return false;
  return PRO != PRO_NORM_QUANT || ((uintptr_t)a.g & 15) == 0;
}

// The prologue-wave form of the SwiGLU GEMV (k_gemv_pw: eight streaming waves and one prologue wave
// per block). It pays where the weight stream fills every CU, i.e. at one block per CU or more
// (Llama-3.2-1B's W1/W3, 8192 rows: 9.49 -> 9.05 us per launch, decode 1,792 -> 1,852 tok/s);
// smaller grids keep the all-wave prologue, since one wave's share of the elementwise work is then
// the longer path (Qwen3-0.6B's 3072 rows: decode 1,217 -> 1,187 tok/s in that form).
constexpr int kPwWaves = 8;
constexpr int kPwMinBlocks = 256;
constexpr int kPwMaxBlocks = 512;

template <int EPI, int NCB>
bool gemv_pw_try(const GemvArgs& a, int rows, hipStream_t st, int& rc) {
  const GemvShape g = gemv_shape<NCB>(a.N);
  const int blocks = cdiv_i(cdiv_i(a.N, g.ru), kPwWaves);   // one tile per streaming wave
  if (a.ids != nullptr || blocks < kPwMinBlocks || blocks > kPwMaxBlocks) return false;
  dim3 grid(blocks, rows), block(64 * (kPwWaves + 1));
  constexpr int RUMAX = gemv_rumax<NCB>();
  if (g.ru == 1) launch((k_gemv_pw<EPI, NCB, 1, kPwWaves>), grid, block, 0, st, a);
  else if (g.ru == 2) launch((k_gemv_pw<EPI, NCB, (RUMAX >= 2 ? 2 : 1), kPwWaves>), grid, block, 0, st, a);
  else launch((k_gemv_pw<EPI, NCB, RUMAX, kPwWaves>), grid, block, 0, st, a);
  rc = hipGetLastError() == hipSuccess ? 0 : -4;
  return true;
}

template <int PRO, int EPI>
int gemv_launch(const GemvArgs& a, int rows, hipStream_t st) {
  if (a.K <= 0 || a.K % 16 || a.K > kMaxK || a.N <= 0 || rows <= 0) return -2;
  if (!gemv_operands_ok<PRO, EPI>(a)) return -2;
  const int nc = cdiv_i(a.K, 1024);
  if constexpr (PRO == PRO_NORM_QUANT && EPI == EPI_SWIGLU) {
    int rc = 0;
    if (nc <= 1 && gemv_pw_try<EPI, 1>(a, rows, st, rc)) return rc;
    if (nc == 2 && gemv_pw_try<EPI, 2>(a, rows, st, rc)) return rc;
  }
  if (nc <= 1) return gemv_launch_shape<PRO, EPI, 1>(a, rows, gemv_shape<1>(a.N), st);
  if (nc <= 2) return gemv_launch_shape<PRO, EPI, 2>(a, rows, gemv_shape<2>(a.N), st);
  if (nc <= 4) return gemv_launch_shape<PRO, EPI, 4>(a, rows, gemv_shape<4>(a.N), st);
  return gemv_launch_shape<PRO, EPI, 8>(a, rows, gemv_shape<8>(a.N), st);
}

// ------------------------------------------------------------------ MFMA GEMM

constexpr int kBK = 64;                 // K per slab
constexpr int kLdsRow = kBK + 16;       // padded LDS row (bytes)

struct GemmArgs {
  const int8_t* xq;          // [M, K] activations
  const float* s_x;          // [M]
  const int8_t* w;           // [N, K] (SwiGLU: W1)
  const float* s_w;          // [N]
  const int8_t* w3;          // SwiGLU: W3 [N, K]
  const float* s_w3;
  int M, N, K;               // N: output columns (SwiGLU: F)
  float* y;                  // [M, N] (stride y_stride)
  const float* res;          // EPI_RESID residual [M, N] (stride y_stride; may alias y)
  long long y_stride;
  int32_t* acc_out;          // optional [M, N] (SwiGLU: [M, 2N], W1 then W3 columns)
  int32_t* part;             // split-K partial sums [splits, M, N] (nullptr: no split)
  long long part_cap;        // int32 elements `part` holds (0: as many as the GEMM split needs)
  const float* tab;          // SFU tables (device copy of c_sfu; required for EPI_SWIGLU)
  unsigned long long* argmax_key;  // optional (k_bgemv, EPI_STORE): per row m the atomic max of
                                   // argmax_key(y, n), the greedy token of the row (keys zeroed before)
  int act;                   // EPI_SWIGLU gate: 0 SiLU, 1 GELU-tanh (gate_mul)
};

// source row of tile column c (0 .. BN) for the block's column origin n0 (SwiGLU interleave)
template <int EPI>
T2R_DEV const int8_t* b_row(const GemmArgs& a, int n0, int c, int& n, bool& ok) {
  if (EPI == EPI_SWIGLU) {
    const int half = c >> 5 & 1;                 // 32-column groups alternate W1 / W3
    n = (n0 >> 1) + ((c >> 6) << 5) + (c & 31);  // the block covers BN / 2 output columns
    ok = n < a.N;
    return (half ? a.w3 : a.w) + (long long)(ok ? n : 0) * a.K;
  }
  n = n0 + c;
  ok = n < a.N;
  return a.w + (long long)(ok ? n : 0) * a.K;
}

template <int EPI, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN) void k_gemm(GemmArgs a) {
  constexpr int BM = 64 * WM, BN = 64 * WN, NT = 64 * WM * WN;
  constexpr int CH_A = BM * kBK / 16, CH_B = BN * kBK / 16;      // 16-byte chunks per slab
  constexpr int PA = (CH_A + NT - 1) / NT, PB = (CH_B + NT - 1) / NT;
  __shared__ __align__(16) int8_t As[2][BM * kLdsRow];
  __shared__ __align__(16) int8_t Bs[2][BN * kLdsRow];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  // m tiles fastest: the workgroups that share a weight slab run together (L2 / MALL reuse)
  const int mt = blockIdx.x % cdiv_i(a.M, BM), nt = blockIdx.x / cdiv_i(a.M, BM);
  const int m0 = mt * BM, n0 = nt * BN;
  const int K = a.K;

  int4 ra[PA], rb[PB];
  auto load_slab = [&](int k0) {
#pragma unroll
    for (int p = 0; p < PA; ++p) {
      const int c = tid + p * NT, r = c / (kBK / 16), kc = (c % (kBK / 16)) * 16;
      const int m = m0 + r, k = k0 + kc;
      ra[p] = (c < CH_A && m < a.M && k < K) ? *(const int4*)(a.xq + (long long)m * K + k) : make_int4(0, 0, 0, 0);
    }
#pragma unroll
    for (int p = 0; p < PB; ++p) {
      const int c = tid + p * NT, r = c / (kBK / 16), kc = (c % (kBK / 16)) * 16;
      int n;
      bool ok;
      const int8_t* src = b_row<EPI>(a, n0, r, n, ok);
      const int k = k0 + kc;
      rb[p] = (c < CH_B && ok && k < K) ? load_nt16(src + k) : make_int4(0, 0, 0, 0);
    }
  };
  auto store_slab = [&](int buf) {
#pragma unroll
    for (int p = 0; p < PA; ++p) {
      const int c = tid + p * NT;
      if (c < CH_A) *(int4*)(&As[buf][(c / (kBK / 16)) * kLdsRow + (c % (kBK / 16)) * 16]) = ra[p];
    }
#pragma unroll
    for (int p = 0; p < PB; ++p) {
      const int c = tid + p * NT;
      if (c < CH_B) *(int4*)(&Bs[buf][(c / (kBK / 16)) * kLdsRow + (c % (kBK / 16)) * 16]) = rb[p];
    }
  };

  v16i_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  const int nk = cdiv_i(K, kBK);
  load_slab(0);
  store_slab(0);
  __syncthreads();
  const int lr = lane & 31, lk = (lane >> 5) * 16;
  for (int s = 0; s < nk; ++s) {
    const int buf = s & 1;
    if (s + 1 < nk) load_slab((s + 1) * kBK);
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 32) {
      v4i_t fa[2], fb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) fa[i] = *(const v4i_t*)(&As[buf][(wm * 64 + i * 32 + lr) * kLdsRow + kk + lk]);
#pragma unroll
      for (int j = 0; j < 2; ++j) fb[j] = *(const v4i_t*)(&Bs[buf][(wn * 64 + j * 32 + lr) * kLdsRow + kk + lk]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    if (s + 1 < nk) {
      store_slab(buf ^ 1);
    }
    __syncthreads();
  }

  // epilogue: lane holds C[m][n] for n = lane % 32 of each 32 x 32 tile, m = 8 (r / 4) + 4 (lane / 32) + r % 4
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = m0 + wm * 64 + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
      if (m >= a.M) continue;
      const float sx = a.s_x[m];
      if (EPI == EPI_SWIGLU) {
        // tile columns [wn * 64, wn * 64 + 32) are W1 rows, the next 32 the same W3 rows
        const int n = (n0 >> 1) + wn * 32 + lr;
        if (n >= a.N) continue;
        const int ac1 = acc[i][0][r], ac3 = acc[i][1][r];
        const float h1 = dequant(ac1, a.s_w[n], sx), h3 = dequant(ac3, a.s_w3[n], sx);
        a.y[(long long)m * a.y_stride + n] = gate_mul(h1, h3, a.act);
        if (a.acc_out) {
          a.acc_out[(long long)m * 2 * a.N + n] = ac1;
          a.acc_out[(long long)m * 2 * a.N + a.N + n] = ac3;
        }
      } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int n = n0 + wn * 64 + j * 32 + lr;
          if (n >= a.N) continue;
          float v = dequant(acc[i][j][r], a.s_w[n], sx);
          if (EPI == EPI_RESID) v = a.res[(long long)m * a.y_stride + n] + v;
          a.y[(long long)m * a.y_stride + n] = v;
          if (a.acc_out) a.acc_out[(long long)m * a.N + n] = acc[i][j][r];
        }
      }
    }
  }
}

constexpr int kGT = 128;                // tile edge of the direct-to-LDS GEMM below


// Workgroup b runs on XCD b % 8 (round-robin dispatch). Give each XCD a contiguous range of the
// n work items, so that the consecutive ones (the M tiles of one weight slab) share that XCD's L2.
T2R_DEV int xcd_order(int b, int n) {
  const int x = b & 7, q = b >> 3, base = n >> 3, extra = n & 7;
  return x * base + min(x, extra) + q;
}

// ---- GEMM with direct-to-LDS loads (K % BKD == 0): 128 x 128 tiles, four waves (2 x 2, 64 x 64
// each), a ring of NST LDS stages filled by global_load_lds_dwordx4 (16 bytes per lane straight into
// LDS, no register staging) NST - 1 slabs ahead of the MFMAs. A slab stage holds A (128 rows x BKD
// bytes) then B; its 16-byte chunk (row r, k-chunk kc) sits at position (BKD/16) r + (kc ^ swz(r)),
// so each 16-lane pass of a 128-bit fragment read hits all 64 banks once.
// Wave w issues the slab's DMA instructions NI w .. NI w + NI - 1 (1 KB each, NI = BKD/16: the first
// half fill A, the second B); lane l of instruction i fills position 64 (i mod 2NI) + l of its operand.
// Every wave issues its share of every slab, slabs 0 .. nk - 1 only: before the MFMAs of slab s the
// wave waits until at most min(NST - 2, nk - 1 - s) newer slabs of its own are in flight (its own
// in-order vmcnt), then the barrier makes every wave's share of slab s visible.
// BKD: K bytes per slab (64 or 128: a 128-byte row segment is one cache line per request);
// NST: LDS stages (NST - 1 slabs in flight). Stage bytes 2 * 128 * BKD.
template <int BKD, int NST, int BM = kGT>
constexpr size_t gemm_d_lds() { return (size_t)NST * (BM + kGT) * BKD; }
// the two configurations launched: 128-byte slabs (one full cache line per row and request) double
// buffered when K % 128 == 0, else 64-byte slabs four deep; both 64 KB of LDS, two workgroups per CU
constexpr size_t kGemmDLds = gemm_d_lds<128, 2>();
static_assert(gemm_d_lds<64, 4>() == kGemmDLds, "both GEMM configurations use the same LDS");
// and the deep ring for grids of at most one workgroup per CU (needs the large-LDS launch attribute)
constexpr size_t kGemmDDeepLds = gemm_d_lds<128, 4>();
// and the 256-row tiles' ring (3 x 48 KB)
constexpr size_t kGemmDTallLds = gemm_d_lds<128, 3, 2 * kGT>();

// The LDS epilogue of k_gemm_d (store / residual). C (int32) of the 64-row band b is staged as
// ct[64][kEpiCS]; then row mr, columns 4 c .. 4 c + 3 are finished by one thread.
constexpr int kEpiCS = kGT + 4;                   // staged row stride (ints): 16-byte aligned rows
template <int EPI, bool SPLIT, int BM>
T2R_DEV void gemm_d_epilogue_vec(const GemmArgs& a, const v16i_t (&acc)[2][2], int8_t* lds, int m0, int n0, int z,
                                 int wm, int wn, int lane, int tid) {
  static_assert(EPI != EPI_SWIGLU, "the gate epilogue runs in registers");
  constexpr int NT = 2 * BM, NB = BM / 64;
  constexpr int OC = kGT, CS = kEpiCS;                            // output columns of the tile, stride
  int* c1 = (int*)lds;                                            // [64][CS]
  const int lr = lane & 31, kh = lane >> 5;
  const int nbase = n0;                                           // first output column of the tile
  // item k of band b is row 64 b + (tid + NT k) / (OC / 4), columns 4 (tid % (OC / 4)) + 0..3 (the
  // same four in every item). Their scales and residual rows are requested here, all at once and
  // from clamped (always readable) addresses, before the staging: loads inside the item loop would
  // each be waited for before the next is issued.
  constexpr int IT = 64 * (OC / 4) / NT;
  static_assert(IT * NT == 64 * (OC / 4) && NT % (OC / 4) == 0, "whole items, fixed columns per thread");
  const int nct = 4 * (tid % (OC / 4));
  v4f_t swp = v4f_t{0.0f, 0.0f, 0.0f, 0.0f};
  float sxp[NB][IT];
  v4f_t rvp[EPI == EPI_RESID ? NB : 1][EPI == EPI_RESID ? IT : 1];
  if constexpr (!SPLIT) {
    swp = *(const v4f_t*)&a.s_w[min(nbase + nct, a.N - 4)];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int k = 0; k < IT; ++k) {
        const int m = min(m0 + 64 * b + (tid + NT * k) / (OC / 4), a.M - 1);
        sxp[b][k] = a.s_x[m];
        if constexpr (EPI == EPI_RESID)
          rvp[b][k] = *(const v4f_t*)&a.res[(long long)m * a.y_stride + min(nbase + nct, a.N - 4)];
      }
  }
  __syncthreads();                                                // every wave is done with the ring
  for (int b = 0; b < NB; ++b) {
    if (wm == b) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int mr = 32 * i + 8 * (r >> 2) + 4 * kh + (r & 3);
#pragma unroll
          for (int j = 0; j < 2; ++j) c1[mr * CS + wn * 64 + j * 32 + lr] = acc[i][j][r];
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < IT; ++k) {
      const int mr = (tid + NT * k) / (OC / 4), nc = nct;
      const int m = m0 + 64 * b + mr, n = nbase + nc;
      if (m < a.M && n < a.N) {                                   // (N % 4 == 0: all four columns)
        const v4i_t v = *(const v4i_t*)&c1[mr * CS + nc];
        if constexpr (SPLIT) {
          *(v4i_t*)&a.part[((long long)z * a.M + m) * a.N + n] = v;
        } else {
          v4f_t y;
#pragma unroll
          for (int q = 0; q < 4; ++q) y[q] = dequant(v[q], swp[q], sxp[b][k]);
          if constexpr (EPI == EPI_RESID) {
#pragma unroll
            for (int q = 0; q < 4; ++q) y[q] = rvp[b][k][q] + y[q];
          }
          *(v4f_t*)&a.y[(long long)m * a.y_stride + n] = y;
        }
      }
    }
    __syncthreads();
  }
}

// BM: tile rows (128: four waves, 2 x 2; 256: eight waves, 4 x 2), always 128 columns.
template <int EPI, bool SPLIT, int BKD, int NST, int BM = kGT>
__global__ __launch_bounds__(2 * BM, (BKD == 64 && NST == 3) ? 3 : 1) void k_gemm_d(GemmArgs a, int ntile, int nz) {
  constexpr int CPR = BKD / 16;                   // 16-byte chunks per row per slab
  constexpr int NWAVE = 2 * BM / 64;
  constexpr int NA = BM * CPR / 64;               // DMA instructions (1 KB each) of A per slab; B: 2 CPR
  constexpr int NI = (NA + 2 * CPR) / NWAVE;      // DMA instructions per wave per slab
  static_assert(NI * NWAVE == NA + 2 * CPR, "whole DMA instructions per wave");
  constexpr int OPA = BM * BKD, OPB = kGT * BKD;  // bytes of A / B per slab
  constexpr int STB = OPA + OPB;
  extern __shared__ __align__(16) int8_t lds[];   // NST stages
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  // work item w = (split z, tile): tiles of one split consecutive, M tiles fastest (weight slabs shared)
  const int w = xcd_order((int)blockIdx.x, ntile * nz);
  const int z = w / ntile, tile = w % ntile;
  const int mtiles = cdiv_i(a.M, BM);
  const int mt = tile % mtiles, nt = tile / mtiles;
  const int m0 = mt * BM, n0 = nt * kGT;
  const int K = a.K, nslab = K / BKD;
  const int per = cdiv_i(nslab, nz);
  const int s0 = z * per, nk = max(0, min(nslab, s0 + per) - s0);
  // chunk (row r, k-chunk kc) of an operand slab sits at position CPR r + (kc ^ swz(r)). gfx950
  // serves a 128-bit LDS read in four passes of 16 lanes over 64 banks (256 bytes), lanes
  // {0-3, 8-11, 20-23, 28-31} + {0, 4, 32, 36} (measured with the bank-conflict counter); the rows
  // one pass reads (lane % 32, one kc) then land in 16 distinct 16-byte bank groups
  auto swz = [](int r) { return CPR == 8 ? ((r ^ (r >> 3)) & 7) : ((r >> 2) & 3); };
  // this lane's DMA sources (instructions NI wave + j: the first NA of all instructions fill A)
  const int8_t* src[NI];
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int i = NI * wave + j, ii = i < NA ? i : i - NA, pos = 64 * ii + lane;
    const int r = pos / CPR, kc = (pos % CPR) ^ swz(r);
    if (i < NA) {
      src[j] = a.xq + (long long)min(m0 + r, a.M - 1) * K + 16 * kc;
    } else {
      int n;
      bool ok;
      src[j] = b_row<EPI>(a, n0, r, n, ok) + 16 * kc;
    }
  }
  // Each workgroup walks its K range from a different slab (the int32 sums are exact in any order):
  // the workgroups that share an A or B tile then do not request the same lines at the same time.
  const int rot = nk > 0 ? (mt + 3 * nt) % nk : 0;
  // instruction j of this wave's share of slab s (s < nk) into stage s % NST
  auto issue1 = [&](int s, int j) {
    const long long k0 = (long long)(s0 + (s + rot) % nk) * BKD;
    const int i = NI * wave + j;
    int8_t* dst = lds + (s % NST) * STB + (i >= NA ? OPA + 1024 * (i - NA) : 1024 * i);
    __builtin_amdgcn_global_load_lds((const void*)(src[j] + k0), (void*)dst, 16, 0, 0);
  };
  constexpr int KKS = BKD / 32;                   // MFMA k-steps per slab
  v16i_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
  const int lr = lane & 31, kh = lane >> 5;
  auto frag = [&](const int8_t* base, int row, int kc) {
    return *(const v4i_t*)(base + (row * CPR + (kc ^ swz(row))) * 16);
  };
  const int mr0 = m0 + wm * 64 + kh * 4;
  auto mrow = [&](int i, int r) { return mr0 + 32 * i + 8 * (r >> 2) + (r & 3); };
  // (SwiGLU on 256-row tiles: one workgroup a CU, registers to spare) the epilogue's row and column
  // scales and the gate's table pairs requested before the K loop, so that the epilogue does not wait
  // for them after it
  constexpr bool EARLY = EPI == EPI_SWIGLU && BM == 2 * kGT;
  float sx_e[EARLY ? 2 : 1][EARLY ? 16 : 1];
  float sw1_e = 0.0f, sw3_e = 0.0f;
  float2 ep_e = make_float2(0.0f, 0.0f), rp_e = make_float2(0.0f, 0.0f);
  if constexpr (EARLY) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) sx_e[i][r] = a.s_x[min(mrow(i, r), a.M - 1)];
    const int nc = min((n0 >> 1) + wn * 32 + lr, a.N - 1);
    sw1_e = a.s_w[nc];
    sw3_e = a.s_w3[nc];
    ep_e = sfu_exp_pair(min(tid, kSfuExpPairs - 1), a.tab);
    rp_e = sfu_recip_pair(tid & 63, a.tab);
  }
#pragma unroll
  for (int p = 0; p < NST - 1; ++p)
    if (p < nk) {
#pragma unroll
      for (int j = 0; j < NI; ++j) issue1(p, j);
    }
  // slab s: MORE = slab s + NST - 1 exists (it goes into the stage slab s - 1 used)
  auto step = [&](int s, auto more) {
    constexpr bool MORE = decltype(more)::value;
    // this wave's share of slab s landed; then a bare s_barrier: every wave's share of slab s is in
    // LDS, and every wave's reads of stage (s + NST - 1) % NST (slab s - 1) are done. (__syncthreads
    // would also wait for the newer DMAs.)
    if constexpr (MORE) {
      __builtin_amdgcn_s_waitcnt(waitcnt_vm((NST - 2) * NI));
    } else {
      const int newer = nk - 1 - s;                 // < NST - 1
      if (newer >= 2) __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * NI));
      else if (newer == 1) __builtin_amdgcn_s_waitcnt(waitcnt_vm(NI));
      else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if constexpr (MORE) {
#pragma unroll
      for (int j = 0; j < NI; ++j) issue1(s + NST - 1, j);
    }
    const int8_t* As = lds + (s % NST) * STB;
    const int8_t* Bs = As + OPA;
#pragma unroll
    for (int kk = 0; kk < KKS; ++kk) {
      v4i_t fa[2], fb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) fa[i] = frag(As, wm * 64 + i * 32 + lr, 2 * kk + kh);
#pragma unroll
      for (int j = 0; j < 2; ++j) fb[j] = frag(Bs, wn * 64 + j * 32 + lr, 2 * kk + kh);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
  };
  int s = 0;
  for (; s + NST - 1 < nk; ++s) step(s, std::true_type{});
  for (; s < nk; ++s) step(s, std::false_type{});
  __builtin_amdgcn_s_waitcnt(0x0F70);             // vmcnt(0): no DMA into LDS outlives the workgroup

  // Store / residual epilogue through LDS (16-byte aligned operands, no int32 copy requested): the
  // tile's int32 sums go to LDS a 64-row band at a time (written by the band's two waves, read back by
  // every thread), and each thread then finishes four consecutive columns of a row with one 16-byte
  // load per operand (scales, residual) and one 16-byte store, instead of the MFMA layout's 4-byte
  // accesses. The SwiGLU gate runs on the accumulators in registers (below): it is VALU-bound, its
  // W1 and W3 sums of an output sit in one lane, and a wave's 4-byte stores cover two 128-byte rows.
  {
    const bool vec = a.acc_out == nullptr && a.N % 4 == 0 && a.y_stride % 4 == 0 &&
                     ((uintptr_t)a.s_w & 15) == 0 &&
                     (SPLIT ? ((uintptr_t)a.part & 15) == 0 : ((uintptr_t)a.y & 15) == 0) &&
                     (EPI != EPI_RESID || SPLIT || ((uintptr_t)a.res & 15) == 0);
    if constexpr (EPI != EPI_SWIGLU) {
      if (vec) {
        gemm_d_epilogue_vec<EPI, SPLIT, BM>(a, acc, lds, m0, n0, z, wm, wn, lane, tid);
        return;
      }
    }
  }

  // Epilogue. Lane holds C[m][n] for n = lane % 32 of each 32 x 32 tile, m = 8 (r / 4) + 4 (lane / 32)
  // + r % 4. Every load it needs (scales, residual, SFU table) is issued before its first store:
  // y may alias the residual, so a load after a store would wait out the store's round trip.
  // (Each element is read and written by its own lane only, so reading all first is the same.)
  if constexpr (SPLIT) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int m = mrow(i, r), n = n0 + wn * 64 + j * 32 + lr;
          if (m < a.M && n < a.N) a.part[((long long)z * a.M + m) * a.N + n] = acc[i][j][r];
        }
    return;
  }
  float sx[2][16];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) sx[i][r] = EARLY ? sx_e[EARLY ? i : 0][EARLY ? r : 0] : a.s_x[min(mrow(i, r), a.M - 1)];
  if constexpr (EPI == EPI_SWIGLU) {
    const int n = (n0 >> 1) + wn * 32 + lr, nc = min(n, a.N - 1);
    const float sw1 = EARLY ? sw1_e : a.s_w[nc], sw3 = EARLY ? sw3_e : a.s_w3[nc];
    float2* ep = (float2*)lds;                    // the gates' pair tables
    float2* rp = ep + kSfuExpPairs;
    __syncthreads();                              // every wave is done with the stage ring
    if (tid < kSfuExpPairs) ep[tid] = EARLY ? ep_e : sfu_exp_pair(tid, a.tab);
    if (tid < 64) rp[tid] = EARLY ? rp_e : sfu_recip_pair(tid, a.tab);
    __syncthreads();
    // A whole tile without an int32 copy: no bounds checks, one gate branch for the tile, and each
    // store at the tile's (uniform) origin plus a 32-bit byte offset: one add per output.
    if (a.acc_out == nullptr && m0 + BM <= a.M && (n0 >> 1) + kGT / 2 <= a.N) {
      char* yb = (char*)(a.y + (long long)m0 * a.y_stride + (n0 >> 1));
      const uint32_t ys4 = 4u * (uint32_t)a.y_stride;
      const uint32_t lo4 = (uint32_t)(wm * 64 + kh * 4) * ys4 + 4u * (uint32_t)(wn * 32 + lr);
      auto run = [&](auto gelu) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float h1 = dequant(acc[i][0][r], sw1, sx[i][r]), h3 = dequant(acc[i][1][r], sw3, sx[i][r]);
            const float g = decltype(gelu)::value ? gelu_mul_p(h1, h3, ep, rp) : silu_mul_p(h1, h3, ep, rp);
            *(float*)(yb + (lo4 + (uint32_t)(32 * i + 8 * (r >> 2) + (r & 3)) * ys4)) = g;
          }
      };
      if (a.act) run(std::true_type{});
      else run(std::false_type{});
      return;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = mrow(i, r);
        if (m >= a.M || n >= a.N) continue;
        const int ac1 = acc[i][0][r], ac3 = acc[i][1][r];
        a.y[(long long)m * a.y_stride + n] = gate_mul_p(dequant(ac1, sw1, sx[i][r]), dequant(ac3, sw3, sx[i][r]), a.act, ep, rp);
        if (a.acc_out) {
          a.acc_out[(long long)m * 2 * a.N + n] = ac1;
          a.acc_out[(long long)m * 2 * a.N + a.N + n] = ac3;
        }
      }
  } else {
    float sw[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) sw[j] = a.s_w[min(n0 + wn * 64 + j * 32 + lr, a.N - 1)];
    float rv[2][16][2];
    if constexpr (EPI == EPI_RESID) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            rv[i][r][j] = a.res[(long long)min(mrow(i, r), a.M - 1) * a.y_stride + min(n0 + wn * 64 + j * 32 + lr, a.N - 1)];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int m = mrow(i, r), n = n0 + wn * 64 + j * 32 + lr;
          float v = dequant(acc[i][j][r], sw[j], sx[i][r]);
          if (EPI == EPI_RESID) v = rv[i][r][j] + v;
          if (m < a.M && n < a.N) {
            a.y[(long long)m * a.y_stride + n] = v;
            if (a.acc_out) a.acc_out[(long long)m * a.N + n] = acc[i][j][r];
          }
        }
  }
}

// ---- narrow store / residual linears (Wqkv, Wo, W2 at a few hundred rows): small tiles, K split over
// the four waves of the workgroup instead of over workgroups. Tile TM x TN (TM = 64, TN = 64 or 96); wave
// w takes the K range [w K/4, (w + 1) K/4) in 128-byte slabs through a ring of its own (kGwStages
// stages of (TM + TN) x 128 bytes, the k_gemm_d layout and swizzle), so the K loop has no workgroup
// barrier: each wave waits on its own in-order vmcnt only, with kGwStages - 1 of its slabs in flight
// behind the one it multiplies (a stage is refilled as soon as its fragments are in registers). The
// four int32 partial tiles meet in LDS (exact in any order) and the epilogue finishes four columns per
// thread with 16-byte accesses. No int32 partials leave the workgroup, so no finishing pass follows.
// Requires K % 512 == 0, N % 4 == 0 and 16-byte aligned s_w / y / res (the launcher checks).
constexpr int kGwStages = 2;
template <int TM, int TN>
constexpr size_t gemm_w_lds() { return (size_t)4 * kGwStages * (TM + TN) * 128; }
template <int EPI, int TM, int TN>
__global__ __launch_bounds__(256) void k_gemm_w(GemmArgs a, int ntile) {
  static_assert(EPI != EPI_SWIGLU, "store / residual only");
  constexpr int CPR = 8, FM = TM / 32, FN = TN / 32;
  constexpr int NA = TM * CPR / 64, NI = (TM + TN) * CPR / 64;     // DMA instructions per slab (A, all)
  constexpr int STB = (TM + TN) * 128, WRB = kGwStages * STB;      // stage / wave ring bytes
  constexpr int PS = TN + 4;                                       // partial tile row stride (ints)
  static_assert(NI * (kGwStages - 1) <= 63, "vmcnt range");
  static_assert(4 * TM * PS * 4 <= 4 * WRB, "partial tiles fit in the rings");
  extern __shared__ __align__(16) int8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int mtiles = cdiv_i(a.M, TM);
  const int w = xcd_order((int)blockIdx.x, ntile);                // M tiles fastest: weight tiles shared in L2
  const int mt = w % mtiles, nt = w / mtiles, m0 = mt * TM, n0 = nt * TN;
  const int K = a.K, nk = K / 512, s0 = wave * nk;                 // this wave's slabs s0 .. s0 + nk - 1
  int8_t* ring = lds + wave * WRB;
  auto swz = [](int r) { return (r ^ (r >> 3)) & 7; };
  // lane's source row and chunk for DMA instruction i (A rows 0 .. TM - 1, then B rows)
  const int8_t* src[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int ii = i < NA ? i : i - NA, pos = 64 * ii + lane, r = pos / CPR, kc = (pos % CPR) ^ swz(r);
    if (i < NA) {
      src[i] = a.xq + (long long)min(m0 + r, a.M - 1) * K + 16 * kc;
    } else {
      int n;
      bool ok;
      src[i] = b_row<EPI>(a, n0, r, n, ok) + 16 * kc;
    }
  }
  auto issue = [&](int s) {
    const long long k0 = (long long)(s0 + s) * 128;
    int8_t* st = ring + (s % kGwStages) * STB;
#pragma unroll
    for (int i = 0; i < NI; ++i) __builtin_amdgcn_global_load_lds((const void*)(src[i] + k0), (void*)(st + 1024 * i), 16, 0, 0);
  };
  v16i_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
  const int lr = lane & 31, kh = lane >> 5;
  auto frag = [&](const int8_t* base, int row, int kc) { return *(const v4i_t*)(base + (row * CPR + (kc ^ swz(row))) * 16); };
  // the epilogue's scales and residual rows (item k: e = tid + 256 k), requested first, all at once
  // and from clamped (always readable) addresses: inside the item loop each load would be waited
  // for before the next is issued. (Older than every slab, they only add to the first slab's wait.)
  constexpr int IT = TM * (TN / 4) / 256;
  static_assert(IT * 256 == TM * (TN / 4), "whole items per thread");
  float sxp[IT];
  v4f_t swp[IT], rvp[EPI == EPI_RESID ? IT : 1];
#pragma unroll
  for (int k = 0; k < IT; ++k) {
    const int e = tid + 256 * k;
    const int m = min(m0 + e / (TN / 4), a.M - 1), n = min(n0 + 4 * (e % (TN / 4)), a.N - 4);
    sxp[k] = a.s_x[m];
    swp[k] = *(const v4f_t*)&a.s_w[n];
    if constexpr (EPI == EPI_RESID) rvp[k] = *(const v4f_t*)&a.res[(long long)m * a.y_stride + n];
  }
#pragma unroll
  for (int p = 0; p < kGwStages; ++p)
    if (p < nk) issue(p);
  for (int s = 0; s < nk; ++s) {
    // slab s landed: kGwStages - 1 newer ones in flight, fewer at the end of the range
    if (s + kGwStages - 1 < nk) __builtin_amdgcn_s_waitcnt(waitcnt_vm((kGwStages - 1) * NI));
    else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    asm volatile("" ::: "memory");
    const int8_t* As = ring + (s % kGwStages) * STB;
    const int8_t* Bs = As + TM * 128;
    v4i_t fa[4][FM], fb[4][FN];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
      for (int i = 0; i < FM; ++i) fa[kk][i] = frag(As, i * 32 + lr, 2 * kk + kh);
#pragma unroll
      for (int j = 0; j < FN; ++j) fb[kk][j] = frag(Bs, j * 32 + lr, 2 * kk + kh);
    }
    // the stage's fragments are in registers: refill it with slab s + kGwStages
    __builtin_amdgcn_s_waitcnt(0xC07F);           // lgkmcnt(0)
    asm volatile("" ::: "memory");
    if (s + kGwStages < nk) issue(s + kGwStages);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[kk][i], fb[kk][j], acc[i][j], 0, 0, 0);
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);             // vmcnt(0): no DMA into LDS outlives the K loop
  __syncthreads();                                // every wave is done with every ring
  int* pt = (int*)lds + wave * TM * PS;           // this wave's partial tile [TM][PS]
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) pt[(32 * i + 8 * (r >> 2) + 4 * kh + (r & 3)) * PS + 32 * j + lr] = acc[i][j][r];
  __syncthreads();
  const int* p0 = (const int*)lds;
#pragma unroll
  for (int k = 0; k < IT; ++k) {
    const int e = tid + 256 * k;
    const int mr = e / (TN / 4), nc = 4 * (e % (TN / 4));
    const int m = m0 + mr, n = n0 + nc;
    if (m >= a.M || n >= a.N) continue;                           // (N % 4 == 0: all four columns)
    v4i_t v = *(const v4i_t*)(p0 + mr * PS + nc);
#pragma unroll
    for (int q = 1; q < 4; ++q) v += *(const v4i_t*)(p0 + q * TM * PS + mr * PS + nc);
    v4f_t y;
#pragma unroll
    for (int q = 0; q < 4; ++q) y[q] = dequant(v[q], swp[k][q], sxp[k]);
    if constexpr (EPI == EPI_RESID) {
#pragma unroll
      for (int q = 0; q < 4; ++q) y[q] = rvp[k][q] + y[q];
    }
    *(v4f_t*)&a.y[(long long)m * a.y_stride + n] = y;
  }
}

// split-K finish: acc = sum of the nz partials (exact), then the STORE / RESID epilogue
template <int EPI>
__global__ __launch_bounds__(256) void k_gemm_fin(GemmArgs a, int nz) {
  const long long total = (long long)a.M * a.N;
  for (long long e = blockIdx.x * 256LL + threadIdx.x; e < total; e += (long long)gridDim.x * 256) {
    const int m = (int)(e / a.N), n = (int)(e % a.N);
    int acc = 0;
    for (int z = 0; z < nz; ++z) acc += a.part[(long long)z * total + e];
    float v = dequant(acc, a.s_w[n], a.s_x[m]);
    if (EPI == EPI_RESID) v = a.res[(long long)m * a.y_stride + n] + v;
    a.y[(long long)m * a.y_stride + n] = v;
    if (a.acc_out) a.acc_out[e] = acc;
  }
}

// split count for the pipelined GEMM. Only a caller that finishes the partials in a pass it runs
// anyway (`defer`) gets a split: a separate finishing pass costs more than the split saves. Up to
// one workgroup per CU (the deep-ring configuration then runs), >= 8 slabs each, the partials within
// the `part_rows` rows x 4 splits of the caller's buffer.
inline int gemm_splits(int M, int ncols, int K, int part_rows, int epi, bool defer) {
  if (epi == EPI_SWIGLU || part_rows <= 0 || !defer) return 1;
  const long long tiles = (long long)cdiv_i(M, kGT) * cdiv_i(ncols, kGT);
  int z = 1;
  while (z < 4 && tiles * z * 2 <= 256 && K / kBK >= 16 * z && (long long)M * z * 2 <= 4LL * part_rows) z *= 2;
  return z;
}

// The wave-split-K kernel where its tiles fill the chip in one round (at most 256 workgroups of 64 x 64,
// else of 64 x 96) and its operand rules hold; -1: not taken (the caller uses k_gemm_d). Two rounds
// (C3's 2032-row Wo and W2: 512 tiles) measured slower than k_gemm_d's split-K: 20.1 / 24.9 against
// 14.8 / 17.5 us.
template <int EPI>
int gemm_w_launch(const GemmArgs& a, hipStream_t st) {
  if (a.K % 512 || a.N % 4 || a.y_stride % 4 || a.acc_out != nullptr || ((uintptr_t)a.s_w & 15) ||
      ((uintptr_t)a.y & 15) || (EPI == EPI_RESID && ((uintptr_t)a.res & 15)))
    return -1;
  const long long mt = cdiv_i(a.M, 64), t64 = mt * cdiv_i(a.N, 64), t96 = mt * cdiv_i(a.N, 96);
  if (t64 <= 256) {
    launch((k_gemm_w<EPI, 64, 64>), dim3((unsigned)t64), dim3(256), gemm_w_lds<64, 64>(), st, a, (int)t64);
  } else if (t96 <= 256) {
    launch((k_gemm_w<EPI, 64, 96>), dim3((unsigned)t96), dim3(256), gemm_w_lds<64, 96>(), st, a, (int)t96);
  } else {
    return -1;
  }
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

// defer_z (STORE / RESID): when the launch splits K, the int32 partials [z, M, N] are left in a.part
// for the caller's own finishing pass and *defer_z = z; otherwise *defer_z = 1 (output written)
template <int EPI, int BKD, int NST, int BM = kGT>
int gemm_d_launch(const GemmArgs& a, hipStream_t st, int z, int* defer_z) {
  if (defer_z) *defer_z = z;
  const long long nb = (long long)cdiv_i(a.M, BM) * cdiv_i(EPI == EPI_SWIGLU ? 2 * a.N : a.N, kGT);
  if (nb * z > 0x7FFFFFFF) return -2;
  const dim3 grid((unsigned)(nb * z));
  const size_t lb = gemm_d_lds<BKD, NST, BM>();
  if (z == 1) {
    launch((k_gemm_d<EPI, false, BKD, NST, BM>), grid, dim3(2 * BM), lb, st, a, (int)nb, z);
  } else if constexpr (EPI != EPI_SWIGLU) {
    launch((k_gemm_d<EPI, true, BKD, NST, BM>), grid, dim3(2 * BM), lb, st, a, (int)nb, z);
    const long long total = (long long)a.M * a.N;
    if (!defer_z) launch((k_gemm_fin<EPI>), dim3((unsigned)min(4096LL, (total + 255) / 256)), dim3(256), 0, st, a, z);
  }
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

// ---- batched decode linears (M <= 64 activation rows): y[m][n] on int8 MFMA with every weight
// byte read once, in whole 128-byte lines. A workgroup takes a tile of 32 weight rows (SwiGLU: 16
// rows of W1 and the same 16 of W3) and kBgWin-byte k-windows of it, one window per wave at a time:
// the wave copies its 32 x 256-byte window into its own 8 KB of LDS with global_load_lds (four rows
// of 256 contiguous bytes per instruction), loads the matching activation bytes into registers in
// the MFMA layout (L2-resident rows), then runs 8 k-steps of v_mfma_i32_32x32x32_i8 (A: activation
// row lane % 32, B: weight row lane % 32, the same 16 k-bytes in both: exact int32 sums). No
// workgroup barrier until the waves' tiles are added in LDS. With nz > 1 the windows are split over
// nz workgroups per tile, which write int32 partials [nz, M, N] for k_gemm_fin. Activation rows past
// M read row M - 1 and are never stored. MG row groups of 32 (M <= 32 MG): each weight fragment read
// from LDS feeds MG MFMAs, one per group's activation rows (a prompt of 33..64 rows streams the
// weights once instead of filling one mostly empty 128-row tile of the prefill GEMM).
constexpr int kBgMaxRows = 32;
constexpr int kBgMaxGroups = 2;                   // M <= kBgMaxRows * kBgMaxGroups
constexpr int kBgWin = 256;                       // k-bytes of a wave window
constexpr int kBgWaveLds = 32 * kBgWin;           // one wave's window of 32 weight rows
// LDS per wave: the window, or the wave's int32 tile [32 MG][33] when that is larger
__host__ __device__ constexpr int bg_wave_lds(int MG) { return 32 * MG * 33 * 4 > kBgWaveLds ? 32 * MG * 33 * 4 : kBgWaveLds; }


template <int EPI, int KW, bool SPLIT, int MG = 1>
__global__ __launch_bounds__(64 * KW) void k_bgemv(GemmArgs a, int nz) {
  constexpr int WS = bg_wave_lds(MG);
  extern __shared__ __align__(16) int8_t lds[];    // KW x WS
  __shared__ __align__(16) float tab_lds[EPI == EPI_SWIGLU ? kSfuWords : 4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 31, kh = lane >> 5;
  constexpr int NT = EPI == EPI_SWIGLU ? 16 : 32;            // output columns per tile
  const int tile = blockIdx.x / nz, z = blockIdx.x % nz;
  const int n0 = tile * NT, K = a.K;
  const int nwin = cdiv_i(K, kBgWin), wpz = cdiv_i(nwin, nz);
  const int w_end = min(nwin, (z + 1) * wpz);
  int8_t* wl = lds + wave * WS;
  if (EPI == EPI_SWIGLU && tid < kSfuWords / 4) ((v4f_t*)tab_lds)[tid] = ((const v4f_t*)a.tab)[tid];
  // chunk q of window row r sits at 256 r + 16 (q ^ (r & 15)): the 16 rows a 16-lane LDS pass reads
  // (rows {0-3, 8-11, 20-23, 28-31} or the other 16 of a half-wave, one chunk) hit 16 bank groups
  const int8_t* rowp[8];
  int qo[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 4 * i + (lane >> 4);
    qo[i] = 16 * ((lane & 15) ^ (r & 15));
    if (EPI == EPI_SWIGLU) rowp[i] = (r < 16 ? a.w : a.w3) + (long long)min(n0 + (r & 15), a.N - 1) * K;
    else rowp[i] = a.w + (long long)min(n0 + r, a.N - 1) * K;
  }
  const int8_t* xrow[MG];
#pragma unroll
  for (int g = 0; g < MG; ++g) xrow[g] = a.xq + (long long)min(32 * g + lr, a.M - 1) * K + 16 * kh;
  // the epilogue's scales and residuals, loaded now (their latency hides under the weight stream):
  // output i of this thread is o = tid + i 64 KW, (m, j) = (o / NT, o % NT)
  constexpr int OPT = (32 * MG * NT + 64 * KW - 1) / (64 * KW);
  float e_sx[OPT], e_sw[OPT], e_sw3[OPT], e_res[OPT];
  if constexpr (!SPLIT) {
#pragma unroll
    for (int i = 0; i < OPT; ++i) {
      const int o = tid + i * 64 * KW, m = min(o / NT, a.M - 1), n = min(n0 + o % NT, a.N - 1);
      e_sx[i] = a.s_x[m];
      e_sw[i] = a.s_w[n];
      if (EPI == EPI_SWIGLU) e_sw3[i] = a.s_w3[n];
      if (EPI == EPI_RESID) e_res[i] = a.res[(long long)m * a.y_stride + n];
    }
  }
  v16i_t acc[MG];
#pragma unroll
  for (int g = 0; g < MG; ++g)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[g][r] = 0;
  for (int w = z * wpz + wave; w < w_end; w += KW) {
    const int k0 = w * kBgWin, nst = min(kBgWin, K - k0) >> 5;   // k-steps of this window (uniform)
    asm volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < 8; ++i)                                 // (chunks past K: clamped, unused)
      __builtin_amdgcn_global_load_lds((const void*)(rowp[i] + min(k0 + qo[i], K - 16)), (void*)(wl + 1024 * i), 16, 0, 0);
    v4i_t xv[MG][8];
#pragma unroll
    for (int g = 0; g < MG; ++g)
#pragma unroll
      for (int st = 0; st < 8; ++st) xv[g][st] = *(const v4i_t*)(xrow[g] + min(k0 + 32 * st, K - 32));
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    asm volatile("" ::: "memory");
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      if (st < nst) {
        const v4i_t wv = *(const v4i_t*)(wl + 256 * lr + 16 * ((2 * st + kh) ^ (lr & 15)));
#pragma unroll
        for (int g = 0; g < MG; ++g) acc[g] = __builtin_amdgcn_mfma_i32_32x32x32_i8(xv[g][st], wv, acc[g], 0, 0, 0);
      }
    }
  }
  // the wave's 32 MG x 32 tile into its own LDS (its DMA has landed and its reads are done)
  asm volatile("" ::: "memory");
  int* red = (int*)wl;
#pragma unroll
  for (int g = 0; g < MG; ++g)
#pragma unroll
    for (int r = 0; r < 16; ++r) red[(32 * g + (r >> 2) * 8 + kh * 4 + (r & 3)) * 33 + lr] = acc[g][r];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < OPT; ++i) {
    const int o = tid + i * 64 * KW, m = o / NT, j = o % NT, n = n0 + j;
    if (EPI == EPI_STORE && !SPLIT && a.argmax_key) {
      // the row's greedy key over this tile's 32 columns: the 32 threads of row m are one half-wave
      unsigned long long key = 0;
      if (m < a.M && n < a.N) {
        int s = 0;
#pragma unroll
        for (int v = 0; v < KW; ++v) s += ((const int*)(lds + v * WS))[m * 33 + j];
        key = argmax_key(dequant(s, e_sw[i], e_sx[i]), n);
      }
#pragma unroll
      for (int off = 1; off < 32; off <<= 1) {
        const unsigned long long other = __shfl_xor(key, off);
        key = other > key ? other : key;
      }
      // all tiles hit the same M keys: skip the atomic when the key already holds a larger one
      if (j == 0 && m < a.M && key != 0 && key > __atomic_load_n(a.argmax_key + m, __ATOMIC_RELAXED))
        atomicMax(a.argmax_key + m, key);
    }
    if (m >= a.M || n >= a.N) continue;
    int s1 = 0, s3 = 0;
#pragma unroll
    for (int v = 0; v < KW; ++v) {
      const int* rv = (const int*)(lds + v * WS);
      s1 += rv[m * 33 + j];
      if (EPI == EPI_SWIGLU) s3 += rv[m * 33 + 16 + j];
    }
    if constexpr (SPLIT) {
      a.part[((long long)z * a.M + m) * a.N + n] = s1;
    } else if constexpr (EPI == EPI_SWIGLU) {
      a.y[(long long)m * a.y_stride + n] = gate_mul(dequant(s1, e_sw[i], e_sx[i]), dequant(s3, e_sw3[i], e_sx[i]), a.act,
                                                 tab_lds);
      if (a.acc_out) {
        a.acc_out[(long long)m * 2 * a.N + n] = s1;
        a.acc_out[(long long)m * 2 * a.N + a.N + n] = s3;
      }
    } else {
      float v = dequant(s1, e_sw[i], e_sx[i]);
      if (EPI == EPI_RESID) v = e_res[i] + v;
      a.y[(long long)m * a.y_stride + n] = v;
      if (a.acc_out) a.acc_out[(long long)m * a.N + n] = s1;
    }
  }
}

// the batched-decode linear when it applies (1 <= M <= 64, K % 32 == 0, 16-byte aligned rows), else -1.
// Waves per workgroup: one per window up to 8; the windows split over up to 4 workgroups per tile when
// the caller finishes the partials (defer_z) and its buffer (a.part, a.part_cap int32) holds them.
template <int EPI, int MG>
void bgemv_go(const GemmArgs& a, hipStream_t st, int kw, int nz, dim3 grid, bool split) {
  const size_t lb = (size_t)kw * bg_wave_lds(MG);
  auto go = [&](auto kern) { launch(kern, grid, dim3(64 * kw), lb, st, a, nz); };
  if (split) {
    if constexpr (EPI != EPI_SWIGLU) {
      if (kw == 8) go(k_bgemv<EPI, 8, true, MG>);
      else if (kw == 4) go(k_bgemv<EPI, 4, true, MG>);
      else if (kw == 2) go(k_bgemv<EPI, 2, true, MG>);
      else go(k_bgemv<EPI, 1, true, MG>);
    }
  } else {
    if (kw == 8) go(k_bgemv<EPI, 8, false, MG>);
    else if (kw == 4) go(k_bgemv<EPI, 4, false, MG>);
    else if (kw == 2) go(k_bgemv<EPI, 2, false, MG>);
    else go(k_bgemv<EPI, 1, false, MG>);
  }
}

template <int EPI>
int bgemv_launch(const GemmArgs& a, hipStream_t st, int* defer_z) {
  if (a.M < 1 || a.M > kBgMaxRows * kBgMaxGroups || a.K % 32 || ((uintptr_t)a.w & 15) || ((uintptr_t)a.xq & 15))
    return -1;
  if (EPI == EPI_SWIGLU && (!a.tab || !a.w3 || ((uintptr_t)a.tab & 15) || ((uintptr_t)a.w3 & 15))) return -1;
  const int nwin = cdiv_i(a.K, kBgWin);
  const int kw = nwin >= 8 ? 8 : nwin >= 4 ? 4 : nwin >= 2 ? 2 : 1;
  int nz = 1;                                     // (split only into a finish the caller runs anyway)
  if (EPI != EPI_SWIGLU && a.part && defer_z)
    while (nz < 4 && nwin > kw * nz && (long long)(2 * nz) * a.M * a.N <= a.part_cap) nz *= 2;
  const long long blocks = (long long)cdiv_i(a.N, EPI == EPI_SWIGLU ? 16 : 32) * nz;
  if (blocks > 0x7FFFFFFF) return -2;
  if (defer_z) *defer_z = nz;
  const dim3 grid((unsigned)blocks);
  if (a.M > kBgMaxRows) bgemv_go<EPI, 2>(a, st, kw, nz, grid, nz > 1);
  else bgemv_go<EPI, 1>(a, st, kw, nz, grid, nz > 1);
  if constexpr (EPI != EPI_SWIGLU) {
    const long long total = (long long)a.M * a.N;
    if (nz > 1 && !defer_z)
      launch((k_gemm_fin<EPI>), dim3((unsigned)min(4096LL, (total + 255) / 256)), dim3(256), 0, st, a, nz);
  }
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

// The M-row GEMM: the batched-decode kernel for M <= 32, else the direct-to-LDS kernel when K % 64 == 0 (split-K into the caller's
// `part_rows`-row partial buffer for narrow layers), else the register-staged k_gemm with the
// largest tile that still gives >= 256 workgroups (one per CU).
template <int EPI>
int gemm_launch(const GemmArgs& a, hipStream_t st, int part_rows = 0, int* defer_z = nullptr) {
  if (a.M <= 0 || a.N <= 0 || a.K <= 0 || a.K % 16) return -2;
  if (EPI == EPI_SWIGLU && (a.tab == nullptr || ((uintptr_t)a.tab & 15))) return -1;
  if (a.M <= kBgMaxRows * kBgMaxGroups) {                 // few rows: stream the weights once
    const int r = bgemv_launch<EPI>(a, st, EPI == EPI_SWIGLU ? nullptr : defer_z);
    if (r != -1) return r;
  }
  const int ncols = EPI == EPI_SWIGLU ? 2 * a.N : a.N;   // B rows the tiles cover
  // the direct-to-LDS kernel (split-K for the narrow STORE / RESID layers)
  if (EPI == EPI_SWIGLU) defer_z = nullptr;
  if (defer_z) *defer_z = 1;
  if constexpr (EPI != EPI_SWIGLU) {                     // narrow linears: K split over waves
    const int r = gemm_w_launch<EPI>(a, st);
    if (r != -1) return r;
  }
  if (a.K % 64 == 0) {
    const int z = gemm_splits(a.M, ncols, a.K, a.part != nullptr ? part_rows : 0, EPI, defer_z != nullptr);
    // a grid of at most one workgroup per CU takes the deep ring (4 x 32 KB: three 128-byte slabs in
    // flight, measured faster on the narrow layers: Wqkv / Wo / W2 at 512 rows 18.6 / 16.3 / 54.8 us
    // -> 14.0 / 12.8 / 42.0); larger grids two workgroups per CU with the double buffer
    const long long nwg = (long long)cdiv_i(a.M, kGT) * cdiv_i(ncols, kGT) * z;
    if (a.K % 128) return gemm_d_launch<EPI, 64, 4>(a, st, z, defer_z);
    if constexpr (EPI == EPI_SWIGLU) {
      // 256-row tiles (eight waves) with a 3 x 48 KB ring: two slabs in flight, one workgroup per CU
      if (a.M >= 2 * kGT && a.M <= 1024) return gemm_d_launch<EPI, 128, 3, 2 * kGT>(a, st, z, defer_z);
      // three 128 x 128 workgroups a CU (3 x 16 KB stages of 64-byte slabs each, 160 VGPRs) where two a
      // CU would leave a partial second round (C3's 768 tiles: 36.9 -> 31.3 us)
      if (a.M > 1024) {
        const long long t = (long long)cdiv_i(a.M, kGT) * cdiv_i(2 * a.N, kGT);
        if (t > 512 && t <= 768) return gemm_d_launch<EPI, 64, 3>(a, st, z, defer_z);
      }
    }
    return nwg <= 256 ? gemm_d_launch<EPI, 128, 4>(a, st, z, defer_z) : gemm_d_launch<EPI, 128, 2>(a, st, z, defer_z);
  }
  auto blocks = [&](int bm, int bn) { return (long long)cdiv_i(a.M, bm) * cdiv_i(ncols, bn); };
  int wm = 1, wn = 1;
  if (blocks(128, 128) >= 256) { wm = 2; wn = 2; }
  else if (blocks(64, 128) >= 256) { wm = 1; wn = 2; }
  const long long nb = blocks(64 * wm, 64 * wn);
  if (nb > 0x7FFFFFFF) return -2;
  dim3 grid((unsigned)nb), block(64 * wm * wn);
  if (wm == 2) launch((k_gemm<EPI, 2, 2>), grid, block, 0, st, a);
  else if (wn == 2) launch((k_gemm<EPI, 1, 2>), grid, block, 0, st, a);
  else launch((k_gemm<EPI, 1, 1>), grid, block, 0, st, a);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

// The op-level GEMM entry: MFMA over the rows.
template <int EPI>
int gemm_dispatch(const GemvArgs& g, int M, hipStream_t st) {
  GemmArgs a{};
  a.xq = g.xq; a.s_x = g.s_x; a.w = g.w; a.s_w = g.s_w; a.w3 = g.w3; a.s_w3 = g.s_w3;
  a.M = M; a.N = g.N; a.K = g.K; a.y = g.y; a.res = g.res; a.y_stride = g.y_stride; a.acc_out = g.acc_out;
  a.tab = g.tab;
  return gemm_launch<EPI>(a, st);
}

}  // namespace t2r
