// W8A8 GEMM over prefill rows: C[M, N] = xq[M, K] . W[N, K]^T (int32), dequantised per row and
// column like the GEMV (expandLinearRows, compiler/plugins/sa/transforms/SahlExpandKernels.cpp:205).
#pragma once
#include "t2r_gemv.h"

namespace t2r {

inline int cdiv_i(long long a, long long b) { return (int)((a + b - 1) / b); }

// The GEMV over `rows` activation rows (grid y): register-slice width NCB by K, rows per wave RU
// by N (enough waves to fill the 256 CUs, up to 8 per CU).
template <int PRO, int EPI, int NCB>
int gemv_launch_ncb(const GemvArgs& a, int rows, hipStream_t st) {
  constexpr int RUMAX = NCB <= 2 ? 4 : (NCB == 4 ? 2 : 1);
  int ru = 1;
  while (ru < RUMAX && (long long)a.N / (2 * ru) >= 2048) ru *= 2;
  const int waves = cdiv_i(a.N, ru);
  int blocks = cdiv_i(waves, kGemvThreads / 64);
  if (blocks > 2048) blocks = 2048;
  dim3 grid(blocks, rows), block(kGemvThreads);
  if (ru == 1) hipLaunchKernelGGL((k_gemv<PRO, EPI, NCB, 1>), grid, block, 0, st, a);
  else if (ru == 2) hipLaunchKernelGGL((k_gemv<PRO, EPI, NCB, (RUMAX >= 2 ? 2 : 1)>), grid, block, 0, st, a);
  else hipLaunchKernelGGL((k_gemv<PRO, EPI, NCB, RUMAX>), grid, block, 0, st, a);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

template <int PRO, int EPI>
int gemv_launch(const GemvArgs& a, int rows, hipStream_t st) {
  if (a.K <= 0 || a.K % 16 || a.K > kMaxK || a.N <= 0 || rows <= 0) return -2;
  const int nc = cdiv_i(a.K, 1024);
  if (nc <= 1) return gemv_launch_ncb<PRO, EPI, 1>(a, rows, st);
  if (nc <= 2) return gemv_launch_ncb<PRO, EPI, 2>(a, rows, st);
  if (nc <= 4) return gemv_launch_ncb<PRO, EPI, 4>(a, rows, st);
  return gemv_launch_ncb<PRO, EPI, 8>(a, rows, st);
}

// Rows through the GEMV kernel, one activation row per grid row.
template <int EPI>
int gemm_dispatch(const GemvArgs& a, int M, hipStream_t st) {
  return gemv_launch<PRO_XQ, EPI>(a, M, st);
}

}  // namespace t2r
