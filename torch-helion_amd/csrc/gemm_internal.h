// Internal structures shared by the gemm kernels (gemm.hip, gemm_fp8.hip).
#pragma once

#include "common.h"

namespace th {

struct EpiOutK {
  int op, a, b, e;
  void* ptr;
  int64_t ld;
  int dtype, vec;  // vec: 4-element vector access possible
  int vec8;        // 8-element (16-byte bf16 / 2 x 16-byte fp32) access possible
  int cb, ce;      // accumulator columns [cb, ce) land at output columns 0 .. ce - cb
};

struct GemmK {
  const void* A;
  int64_t lda;
  const void* B;
  int64_t ldb;
  int64_t M, N, K;
  int tiles_m, tiles_n;
  int bn, n_acc;
  int sumsq;
  unsigned rscale_mask;
  float inv_k, eps;
  const void* extra[TH_MAX_EXTRA];
  int64_t ld_extra[TH_MAX_EXTRA];
  int extra_dtype[TH_MAX_EXTRA];
  int extra_vec[TH_MAX_EXTRA];
  int extra_vec8[TH_MAX_EXTRA];
  const float* rcos;
  const float* rsin;
  int hd, period;
  int n_out;
  int asplit;  // persistent kernel: each wave's column half is one whole accumulator (n_acc == 2)
  EpiOutK out[TH_MAX_OUT];
  float* sumsq_out;
};

// fp8-weight path (gemm_fp8.hip)
struct Fp8K {
  GemmK k;           // output ops, row scale, extras, RoPE tables
  const void* A;     // bf16 [M, K]
  int64_t lda;
  const void* B;     // packed e4m3 rhs, K contiguous
  int64_t ldb;       // bytes per packed row
  int64_t M, N, K, Npk, bn;
  const float* scale;  // [n_acc][N]
  int splits;
  int64_t ksplit;
  float* part;       // [splits][M][Npk]
  float* sumsq_part; // [splits][M]
  int fused;         // one split finishing its tiles in the main kernel (no reduce pass)
};

int64_t fp8_workspace_bytes(int64_t M, int64_t Npk, int64_t K, int bn, int n_acc);
int launch_gemm_fp8(const GemmK& k, int64_t Npk, const float* scale, float* ws, int64_t ws_bytes, hipStream_t s);

}  // namespace th
