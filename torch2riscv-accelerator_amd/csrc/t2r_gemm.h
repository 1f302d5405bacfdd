// W8A8 GEMM over prefill rows: C[M, N] = xq[M, K] . W[N, K]^T (int32), dequantised per row and
// column like the GEMV (expandLinearRows, compiler/plugins/sa/transforms/SahlExpandKernels.cpp:205).
#pragma once
#include "t2r_gemv.h"

namespace t2r {

inline int cdiv_i(long long a, long long b) { return (int)((a + b - 1) / b); }

// The GEMV over `rows` activation rows (grid y): register-slice width and rows per wave by K.
template <int PRO, int EPI>
int gemv_launch(const GemvArgs& a, int rows, hipStream_t st) {
  if (a.K <= 0 || a.K % 16 || a.K > kMaxK || a.N <= 0 || rows <= 0) return -2;
  const int nc = cdiv_i(a.K, 1024);
  int ru, ncb;
  if (nc <= 1) { ncb = 1; ru = 8; }
  else if (nc <= 2) { ncb = 2; ru = 4; }
  else if (nc <= 4) { ncb = 4; ru = 2; }
  else { ncb = 8; ru = 1; }
  const int waves = cdiv_i(a.N, ru);
  int blocks = cdiv_i(waves, kGemvThreads / 64);
  if (blocks > 2048) blocks = 2048;
  dim3 grid(blocks, rows), block(kGemvThreads);
  switch (ncb) {
    case 1: hipLaunchKernelGGL((k_gemv<PRO, EPI, 1, 8>), grid, block, 0, st, a); break;
    case 2: hipLaunchKernelGGL((k_gemv<PRO, EPI, 2, 4>), grid, block, 0, st, a); break;
    case 4: hipLaunchKernelGGL((k_gemv<PRO, EPI, 4, 2>), grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL((k_gemv<PRO, EPI, 8, 1>), grid, block, 0, st, a); break;
  }
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

// Rows through the GEMV kernel, one activation row per grid row.
template <int EPI>
int gemm_dispatch(const GemvArgs& a, int M, hipStream_t st) {
  return gemv_launch<PRO_XQ, EPI>(a, M, st);
}

}  // namespace t2r
