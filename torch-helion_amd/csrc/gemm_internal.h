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
  const float* gain;  // optional [K]: products use lhs[m, k] * gain[k] (fp8 path); sumsq stays unscaled
  // optional [M][n_rs_parts] (row stride ld_rs_parts): each row's sum of squares as
  // partial sums made by the lhs's producer, summed in order instead of sum_k lhs^2
  const float* rs_parts;
  int64_t ld_rs_parts;
  int n_rs_parts;
  // optional (fp8 path): output gain_index stored as bf16(bf16(v) * gain_out[n]),
  // each row's sums of bf16(v)^2 per 256 columns to ss_parts_out
  const float* gain_out;
  float* ss_parts_out;
  int64_t ld_ss_parts_out;
  int gain_index;
};

// Row `row`'s sum of squares: `own` (the kernel's sum over its lhs fragments), or
// the sum of the producer's partial sums when the caller gave them, added one
// after another in order; rows past M read row M - 1, whose scale is never
// used. The parts are fetched 32 at a time, every load issued before the
// first addition (indices clamped, additions past the end selected away: no
// branch for the compiler to put a wait into), so a row costs one memory
// round trip per 32 parts instead of one per 4.
__device__ __forceinline__ float row_sumsq(const GemmK& p, int64_t row, float own) {
  if (p.rs_parts == nullptr) return own;
  const float4* q = (const float4*)(p.rs_parts + (row < p.M ? row : p.M - 1) * p.ld_rs_parts);
  const int n4 = p.n_rs_parts >> 2;
  float v = 0.f;
  for (int i0 = 0; i0 < n4; i0 += 8) {
    float4 f[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = q[i0 + j < n4 ? i0 + j : n4 - 1];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float t = v + f[j].x;
      t += f[j].y;
      t += f[j].z;
      t += f[j].w;
      v = i0 + j < n4 ? t : v;
    }
  }
  return v;
}

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
  int ss_pre;        // row sums of squares already in sumsq_part (split 0; the others zero)
};

// 4 consecutive elements (one 8-byte bf16 / 16-byte fp32 access when vec,
// element by element for a ragged end or unaligned rows).
__device__ __forceinline__ float4 load4(const void* p, int64_t off, int dtype, bool vec, int valid) {
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (vec && valid >= 4) {
    if (dtype == TH_BF16) {
      const uint2 w = *(const uint2*)((const uint16_t*)p + off);
      v.x = __uint_as_float(w.x << 16);
      v.y = __uint_as_float(w.x & 0xffff0000u);
      v.z = __uint_as_float(w.y << 16);
      v.w = __uint_as_float(w.y & 0xffff0000u);
    } else {
      v = *(const float4*)((const float*)p + off);
    }
    return v;
  }
  float t[4] = {0.f, 0.f, 0.f, 0.f};
  for (int q = 0; q < 4 && q < valid; ++q) t[q] = load_elem(p, off + q, dtype);
  return make_float4(t[0], t[1], t[2], t[3]);
}

__device__ __forceinline__ void store4(void* p, int64_t off, int dtype, bool vec, int valid, float4 v) {
  if (vec && valid >= 4) {
    if (dtype == TH_BF16) {
      uint2 w;
      w.x = pk_bf16x2(v.x, v.y);
      w.y = pk_bf16x2(v.z, v.w);
      *(uint2*)((uint16_t*)p + off) = w;
    } else {
      *(float4*)((float*)p + off) = v;
    }
    return;
  }
  const float t[4] = {v.x, v.y, v.z, v.w};
  for (int q = 0; q < 4 && q < valid; ++q) store_elem(p, off + q, dtype, t[q]);
}

int64_t fp8_workspace_bytes(int64_t M, int64_t Npk, int64_t K, int bn, int n_acc);
int launch_gemm_fp8(const GemmK& k, int64_t Npk, const float* scale, float* ws, int64_t ws_bytes, hipStream_t s);

}  // namespace th
