// gemm kind with fp8 (OCP e4m3) weights and bf16 activations for few rows
// (M <= 128, the decode step): acc_i[m, n] = s_i[n] * sum_k x[m, k] q_i[k, n],
// q_i the e4m3 weights packed by th_gemm_pack_rhs, s_i the per-output-channel
// fp32 scales. No counterpart kernel in the reference (its IR has no fp8 type);
// the math is the gemm kind of codegen/interpret.py:22-35 on dequantised weights.
//
// Such GEMMs stream every weight byte from HBM once and do little arithmetic
// per byte, so the work is split along K as well as N until the whole GPU is
// pulling bandwidth:
//   gemm_fp8_splitk_kernel  one workgroup per (32 packed columns, K range), the
//                           four waves splitting the range; per 32-K chunk a
//                           wave loads one contiguous KiB of weights (the
//                           fragment-major packing of th_gemm_pack_rhs), a lane
//                           32 contiguous activation bytes (the K order inside a
//                           chunk is permuted identically for both operands),
//                           converts the weights with v_cvt_scalef32_pk_bf16_fp8
//                           (exact: every e4m3 value is a bf16 value) and runs
//                           v_mfma_f32_32x32x16_bf16; fp32 partial sums per
//                           split go to the workspace (and, from the first
//                           column block, partial row sums of squares);
//   gemm_fp8_reduce_kernel  sums the splits in a fixed order (deterministic),
//                           applies s_i[n], the RMS row scale and the fused
//                           output op, and stores.
#include "common.h"
#include "gemm_internal.h"

namespace th {

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

__device__ __forceinline__ bf16x8_t fp8x8_to_bf16x8(uint32_t lo, uint32_t hi) {
  union {
    bf16x2_t h[4];
    bf16x8_t v;
  } u;
  u.h[0] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false);
  u.h[1] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true);
  u.h[2] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false);
  u.h[3] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true);
  return u.v;
}

// grid (Npk / (32 NG), splits); Npk = packed rows of the rhs (a multiple of 32).
// All four waves of a workgroup own the same 32*NG packed columns and split the
// workgroup's K range four ways. A wave works in groups of U 32-K chunks: every
// global load of a group (NG KiB of weights per chunk, contiguous thanks to the
// fragment-major packing, and the activation fragments) is issued before the
// group's first MFMA, so the group costs one memory latency, not U of them.
// The waves' sums meet in LDS and one partial per split is written.
template <int TM, int NG, int U>  // 32-row tiles of M (M <= 32*TM); column groups; chunks per group
__global__ void __launch_bounds__(256) gemm_fp8_splitk_kernel(Fp8K p) {
  __shared__ float red[3][TM * NG][16][64];
  __shared__ float ssr[3][TM][32];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, c32 = lane & 31;
  const int split = blockIdx.y;
  const int64_t ks0 = (int64_t)split * p.ksplit;
  const int64_t ks1 = min(p.K, ks0 + p.ksplit);
  const int64_t kw = p.ksplit / 4;  // a multiple of 32
  const int64_t kb = min(ks1, ks0 + wave * kw), ke = min(ks1, kb + kw);
  const int64_t nch = p.ldb / 32;   // 32-K chunks per packed row
  // fragment-major rhs: chunk c of 32-row group g is the KiB at (g * nch + c) * 1024
  const uint8_t* bgrp = (const uint8_t*)p.B + (int64_t)blockIdx.x * NG * nch * 1024 + 16 * lane;
  const uint16_t* A = (const uint16_t*)p.A;
  const bool do_ss = p.sumsq_part != nullptr && blockIdx.x == 0;

  f32x16_t acc[TM][NG];
  float ss[TM];
#pragma unroll
  for (int t = 0; t < TM; ++t) {
    ss[t] = 0.f;
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[t][g][r] = 0.f;
  }
  for (int64_t kc = kb; kc < ke; kc += 32 * U) {
    uint4 wb[U][NG];
    bf16x8_t af[U][TM][2];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t k = kc + 32 * u;
      const bool ok = k < ke;
#pragma unroll
      for (int g = 0; g < NG; ++g)
        wb[u][g] = ok ? *(const uint4*)(bgrp + ((int64_t)g * nch + (k >> 5)) * 1024) : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int t = 0; t < TM; ++t) {
        const int m = 32 * t + c32;
        if (ok && m < p.M) {
          const uint16_t* ar = A + (int64_t)m * p.lda + k + 16 * h;
          af[u][t][0] = *(const bf16x8_t*)ar;
          af[u][t][1] = *(const bf16x8_t*)(ar + 8);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) af[u][t][0][e] = af[u][t][1][e] = (__bf16)0.f;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        const bf16x8_t b0 = fp8x8_to_bf16x8(wb[u][g].x, wb[u][g].y), b1 = fp8x8_to_bf16x8(wb[u][g].z, wb[u][g].w);
#pragma unroll
        for (int t = 0; t < TM; ++t) {
          acc[t][g] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[u][t][0], b0, acc[t][g], 0, 0, 0);
          acc[t][g] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[u][t][1], b1, acc[t][g], 0, 0, 0);
        }
      }
      if (do_ss) {
#pragma unroll
        for (int t = 0; t < TM; ++t)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float x0 = (float)af[u][t][0][e], x1 = (float)af[u][t][1][e];
            ss[t] += x0 * x0 + x1 * x1;
          }
      }
    }
  }
  // waves 1..3 hand their sums to wave 0
  if (wave > 0) {
#pragma unroll
    for (int t = 0; t < TM; ++t) {
#pragma unroll
      for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int r = 0; r < 16; ++r) red[wave - 1][t * NG + g][r][lane] = acc[t][g][r];
      if (do_ss) {
        const float v = ss[t] + __shfl_xor(ss[t], 32);
        if (h == 0) ssr[wave - 1][t][c32] = v;
      }
    }
  }
  __syncthreads();
  if (wave != 0) return;
  float* part = p.part + (int64_t)split * p.M * p.Npk;
#pragma unroll
  for (int t = 0; t < TM; ++t)
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int64_t col = ((int64_t)blockIdx.x * NG + g) * 32 + c32;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = t * NG + g;
        const float v = acc[t][g][r] + red[0][i][r][lane] + red[1][i][r][lane] + red[2][i][r][lane];
        const int m = 32 * t + 8 * (r >> 2) + 4 * h + (r & 3);
        if (m < p.M && col < p.Npk) part[(int64_t)m * p.Npk + col] = v;
      }
    }
  if (do_ss) {
#pragma unroll
    for (int t = 0; t < TM; ++t) {
      const float v = ss[t] + __shfl_xor(ss[t], 32) + ssr[0][t][c32] + ssr[1][t][c32] + ssr[2][t][c32];
      const int m = 32 * t + c32;
      if (h == 0 && m < p.M) p.sumsq_part[(int64_t)split * p.M + m] = v;
    }
  }
}

// acc_i(m, n) from the partials, scaled: s_i[n] * sum over splits.
__device__ __forceinline__ float fp8_acc(const Fp8K& p, int i, int64_t m, int64_t n) {
  const int64_t t = n / p.bn, j = n - t * p.bn;
  const int64_t row = (t * p.k.n_acc + i) * p.bn + j;
  float s = 0.f;
  for (int sp = 0; sp < p.splits; ++sp) s += p.part[((int64_t)sp * p.M + m) * p.Npk + row];
  return s * p.scale[(int64_t)i * p.N + n];
}

// One thread per (row m, output column n); every fused output op.
__global__ void __launch_bounds__(256) gemm_fp8_reduce_kernel(Fp8K p) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)p.M * p.N) return;
  const int64_t m = idx / p.N, n = idx - m * p.N;
  const GemmK& g = p.k;
  float rr = 1.f;
  if (g.sumsq) {
    float ss = 0.f;
    for (int sp = 0; sp < p.splits; ++sp) ss += p.sumsq_part[(int64_t)sp * p.M + m];
    rr = rsqrtf(ss * g.inv_k + g.eps);
    if (g.sumsq_out && n == 0) g.sumsq_out[m] = ss;
  }
  for (int o = 0; o < g.n_out; ++o) {
    const EpiOutK& eo = g.out[o];
    const int op = eo.op;
    float a = fp8_acc(p, eo.a, m, n);
    if ((g.rscale_mask >> eo.a) & 1u) a *= rr;
    float v;
    switch (op) {
      case TH_EPI_ACC:
        v = a;
        break;
      case TH_EPI_ROPE:
      case TH_EPI_ROPE_PAIR: {
        const int within = (int)(n % g.hd);
        float rot;
        if (op == TH_EPI_ROPE) {
          const int half = g.hd >> 1;
          const int64_t pn = within < half ? n + half : n - half;
          rot = fp8_acc(p, eo.a, m, pn) * (within < half ? -1.f : 1.f);
          if ((g.rscale_mask >> eo.a) & 1u) rot *= rr;
        } else {
          rot = fp8_acc(p, eo.b, m, n);
          if ((g.rscale_mask >> eo.b) & 1u) rot *= rr;
        }
        const int64_t toff = (m % g.period) * g.hd + within;
        v = a * g.rcos[toff] + rot * g.rsin[toff];
        break;
      }
      case TH_EPI_SILU:
        v = a * sigmoidf_(a);
        break;
      case TH_EPI_SWIGLU: {
        float b = fp8_acc(p, eo.b, m, n);
        if ((g.rscale_mask >> eo.b) & 1u) b *= rr;
        v = a * sigmoidf_(a) * b;
        break;
      }
      default: {  // TH_EPI_ADD, TH_EPI_SOFTPLUS_ADD, TH_EPI_MUL
        const float x = load_elem(g.extra[eo.e], m * g.ld_extra[eo.e] + n, g.extra_dtype[eo.e]);
        if (op == TH_EPI_MUL) {
          v = a * x;
        } else {
          v = a + x;
          if (op == TH_EPI_SOFTPLUS_ADD) v = softplusf_(v);
        }
        break;
      }
    }
    store_elem(eo.ptr, m * eo.ld + n, eo.dtype, v);
  }
}

// Split count: about one workgroup per CU, each wave at least 256 of K.
static int fp8_groups(int64_t Npk) { return Npk % 64 == 0 ? 2 : 1; }

static int fp8_splits(int64_t Npk, int64_t K) {
  const int64_t cus = device_cus() > 0 ? device_cus() : 256;
  const int64_t nb = Npk / (32 * fp8_groups(Npk));
  int64_t s = cdiv(cus, nb);
  s = std::min(s, std::max((int64_t)1, K / 1024));
  return (int)std::max((int64_t)1, std::min(s, (int64_t)64));
}

int64_t fp8_workspace_bytes(int64_t M, int64_t Npk, int64_t K) {
  const int s = fp8_splits(Npk, K);
  return (int64_t)s * M * (Npk + 1) * 4;
}

int launch_gemm_fp8(const GemmK& k, int64_t Npk, const float* scale, float* ws, int64_t ws_bytes,
                    hipStream_t stream) {
  Fp8K p{};
  p.k = k;
  p.A = k.A;
  p.lda = k.lda;
  p.B = k.B;
  p.ldb = k.ldb;
  p.M = k.M;
  p.N = k.N;
  p.K = k.K;
  p.Npk = Npk;
  p.bn = k.bn;
  p.scale = scale;
  p.splits = fp8_splits(Npk, k.K);
  p.ksplit = cdiv(cdiv(k.K, p.splits), 128) * 128;  // four waves x a multiple of 32
  p.splits = (int)cdiv(k.K, p.ksplit);
  const int64_t need = (int64_t)p.splits * k.M * (Npk + 1) * 4;
  TH_CHECK_ARG(ws && ws_bytes >= need, "th_gemm: fp8 weights need a workspace of %lld bytes (got %lld)",
               (long long)need, (long long)ws_bytes);
  p.part = ws;
  p.sumsq_part = k.sumsq ? ws + (int64_t)p.splits * k.M * Npk : nullptr;
  const int ng = fp8_groups(Npk);
  const dim3 g1((unsigned)(Npk / (32 * ng)), (unsigned)p.splits);
  if (k.M <= 64) {
    if (ng == 2)
      hipLaunchKernelGGL((gemm_fp8_splitk_kernel<2, 2, 4>), g1, dim3(256), 0, stream, p);
    else
      hipLaunchKernelGGL((gemm_fp8_splitk_kernel<2, 1, 4>), g1, dim3(256), 0, stream, p);
  } else {
    if (ng == 2)
      hipLaunchKernelGGL((gemm_fp8_splitk_kernel<4, 2, 2>), g1, dim3(256), 0, stream, p);
    else
      hipLaunchKernelGGL((gemm_fp8_splitk_kernel<4, 1, 2>), g1, dim3(256), 0, stream, p);
  }
  TH_CHECK_LAUNCH();
  hipLaunchKernelGGL(gemm_fp8_reduce_kernel, dim3((unsigned)cdiv(k.M * k.N, 256)), dim3(256), 0, stream, p);
  TH_CHECK_LAUNCH();
  return TH_OK;
}

}  // namespace th
