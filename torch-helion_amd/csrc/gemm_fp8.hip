// gemm kind with fp8 (OCP e4m3) weights and bf16 activations for few rows
// (M <= 128, the decode step): acc_i[m, n] = s_i[n] * sum_k x[m, k] q_i[k, n],
// q_i the e4m3 weights packed by th_gemm_pack_rhs, s_i the per-output-channel
// fp32 scales. No counterpart kernel in the reference (its IR has no fp8 type);
// the math is the gemm kind of codegen/interpret.py:22-35 on dequantised weights.
//
// Such GEMMs stream every weight byte from HBM once and do little arithmetic
// per byte, so the work is split along K as well as N until the whole GPU is
// pulling bandwidth. Every e4m3 value is a bf16 value: the weights are
// converted exactly (v_cvt_scalef32_pk_bf16_fp8) and multiplied on
// v_mfma_f32_32x32x16_bf16 with fp32 accumulation.
//
// Main path (K a multiple of 128, n_acc 1 or 2, bn = 128 / n_acc):
//   fp8_gain_prep_kernel    with an activation-side RMSNorm gain: the rows
//                           scaled once, bf16(x g), and their unscaled sums
//                           of squares, into the workspace;
//   gemm_fp8_lds_kernel     one workgroup of eight waves per (128-column packed
//                           tile, K split); four column groups of 32 x two K
//                           halves, sharing the activation slices, which
//                           stream through rotating LDS buffers by direct
//                           loads while each wave's weights (contiguous KiB
//                           blocks of the fragment-major packing) go to
//                           registers; a single split finishes its tiles in
//                           the kernel;
//   gemm_fp8_reduce4_kernel with several splits: sums them in a fixed order
//                           (deterministic), 4 columns per thread, and applies
//                           s_i[n], the RMS row scale and the fused output ops.
// Other shapes:
//   gemm_fp8_splitk_kernel  one workgroup per (32 packed columns, K range), the
//                           four waves splitting the range; per 32-K chunk a
//                           wave loads one contiguous KiB of weights, a lane
//                           32 contiguous activation bytes (the K order inside a
//                           chunk is permuted identically for both operands);
//                           fp32 partial sums per split go to the workspace
//                           (and, from the first column block, partial row sums
//                           of squares);
//   gemm_fp8_reduce_kernel  one thread per output element, same sums and ops.
#include <type_traits>
#include <utility>

#include "common.h"
#include "gemm_internal.h"

namespace th {

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;

// f(integral_constant<int, I>) for I = 0, 1, ... in order (compile-time slot indices)
template <int... I, class F>
__device__ __forceinline__ void unroll_seq(std::integer_sequence<int, I...>, F&& f) {
  (f(std::integral_constant<int, I>()), ...);
}


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
    if (p.k.gain) {
      // activation-side RMSNorm gain: the sum of squares is taken first, from
      // the unscaled row, then the operands become bf16(x * g)
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t k = kc + 32 * u;
        if (k >= ke) continue;
        const float4* gp = (const float4*)(p.k.gain + k + 16 * h);
        const float4 g4[4] = {gp[0], gp[1], gp[2], gp[3]};
        const float* g = (const float*)g4;
#pragma unroll
        for (int t = 0; t < TM; ++t)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float x0 = (float)af[u][t][0][e], x1 = (float)af[u][t][1][e];
            if (do_ss) ss[t] += x0 * x0 + x1 * x1;
            af[u][t][0][e] = (__bf16)(x0 * g[e]);
            af[u][t][1][e] = (__bf16)(x1 * g[8 + e]);
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
      if (do_ss && !p.k.gain) {
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

// Every fused output op of element (m, n) (outputs whose column window
// [cb, ce) holds n, stored at n - cb, extras read there too); accf(i, n') is
// accumulator i at output column n' (partials summed over the splits,
// per-column scale applied), rr the row's RMS scale (1 without sumsq).
template <class AccF>
__device__ __forceinline__ void fp8_emit(const Fp8K& p, int64_t m, int64_t n, float rr, AccF accf) {
  const GemmK& g = p.k;
  for (int o = 0; o < g.n_out; ++o) {
    const EpiOutK& eo = g.out[o];
    if (n < eo.cb || n >= eo.ce) continue;  // column window: stored at n - cb
    const int64_t gc = n - eo.cb;
    const int op = eo.op;
    float a = accf(eo.a, n);
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
          rot = accf(eo.a, pn) * (within < half ? -1.f : 1.f);
          if ((g.rscale_mask >> eo.a) & 1u) rot *= rr;
        } else {
          rot = accf(eo.b, n);
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
        float b = accf(eo.b, n);
        if ((g.rscale_mask >> eo.b) & 1u) b *= rr;
        v = a * sigmoidf_(a) * b;
        break;
      }
      default: {  // TH_EPI_ADD, TH_EPI_SOFTPLUS_ADD, TH_EPI_MUL
        const float x = load_elem(g.extra[eo.e], m * g.ld_extra[eo.e] + gc, g.extra_dtype[eo.e]);
        if (op == TH_EPI_MUL) {
          v = a * x;
        } else {
          v = a + x;
          if (op == TH_EPI_SOFTPLUS_ADD) v = softplusf_(v);
        }
        break;
      }
    }
    store_elem(eo.ptr, m * eo.ld + gc, eo.dtype, v);
  }
}

// Every output op of row m, columns n4 .. n4+3 (n4 a multiple of 4, the 4
// columns inside one packed tile and one RoPE half-head, column windows on
// multiples of 8); sum4(i, nn, rot) is accumulator i at columns nn .. nn+3,
// scaled (rot: nn is the RoPE partner's columns, not n4); n_acc is 1 or 2;
// rrf() the row's RMS scale; gather() issues the loads sum4 and rrf fold, if
// any. Two phases: every load (gather's, then the RoPE tables and the
// extras) goes out before the stores, so a thread waits for about one round
// of memory latency per distinct extra, not one per output and split; then
// one 4-wide store per output. With gain_out, output gain_index is stored as
// bf16(bf16(v) * gain_out[n]); the return value is the sum of its four
// bf16(v)^2 (0 without gain_out).
template <class Sum4, class RowScale, class Gather>
__device__ __forceinline__ float fp8_emit4(const Fp8K& p, int64_t m, int64_t n4, RowScale rrf, Sum4 sum4,
                                           Gather gather) {
  const GemmK& g = p.k;
  const int valid = (int)min((int64_t)4, p.N - n4);
  // the rotation partner of each accumulator some ROPE output here reads
  bool rope_acc[2] = {false, false};
  bool tab = false;
  for (int o = 0; o < g.n_out; ++o) {
    const EpiOutK& eo = g.out[o];
    if (n4 < eo.cb || n4 >= eo.ce) continue;
    if (eo.op == TH_EPI_ROPE) rope_acc[eo.a & 1] = true;
    if (eo.op == TH_EPI_ROPE || eo.op == TH_EPI_ROPE_PAIR) tab = true;
  }
  const int within = g.hd > 0 ? (int)n4 % g.hd : 0;
  const int half = g.hd >> 1;
  const int64_t pn = within < half ? n4 + half : n4 - half;
  const int toff = tab ? ((int)m % g.period) * g.hd + within : 0;
  gather();
  const float4 zero4 = make_float4(0.f, 0.f, 0.f, 0.f);
  float4 cs = zero4, sn = zero4;
  if (tab) {
    cs = make_float4(g.rcos[toff], g.rcos[toff + 1], g.rcos[toff + 2], g.rcos[toff + 3]);
    sn = make_float4(g.rsin[toff], g.rsin[toff + 1], g.rsin[toff + 2], g.rsin[toff + 3]);
  }
  const float4 gq = g.gain_out != nullptr ? *(const float4*)(g.gain_out + n4) : zero4;
  // extras (after gather's loads, so the first one's conversion waits for
  // all of them at once; an extra two outputs share is loaded once)
  float4 xe[TH_MAX_OUT];
#pragma unroll
  for (int o = 0; o < TH_MAX_OUT; ++o) {
    xe[o] = zero4;
    if (o >= g.n_out) continue;
    const EpiOutK& eo = g.out[o];
    const bool uses_e = eo.op == TH_EPI_ADD || eo.op == TH_EPI_SOFTPLUS_ADD || eo.op == TH_EPI_MUL;
    if (!uses_e || n4 < eo.cb || n4 >= eo.ce) continue;
    int same = -1;
#pragma unroll
    for (int o2 = 0; o2 < o; ++o2) {
      const EpiOutK& e2 = g.out[o2];
      const bool u2 = e2.op == TH_EPI_ADD || e2.op == TH_EPI_SOFTPLUS_ADD || e2.op == TH_EPI_MUL;
      if (same < 0 && u2 && e2.e == eo.e && e2.cb == eo.cb && e2.ce == eo.ce) same = o2;
    }
    if (same >= 0) {
#pragma unroll
      for (int o2 = 0; o2 < o; ++o2)
        if (o2 == same) xe[o] = xe[o2];
    } else {
      xe[o] = load4(g.extra[eo.e], m * g.ld_extra[eo.e] + (n4 - eo.cb), g.extra_dtype[eo.e], g.extra_vec[eo.e] != 0,
                    (int)min((int64_t)valid, eo.ce - n4));
    }
  }
  float ssg = 0.f;
  // the sums (the shared-activation kernel's packings have one or two accumulators)
  const float4 c0 = sum4(0, n4, false);
  const float4 c1 = g.n_acc > 1 ? sum4(1, n4, false) : c0;
  const float4 rot0 = rope_acc[0] ? sum4(0, pn, true) : zero4;
  const float4 rot1 = rope_acc[1] ? sum4(1, pn, true) : zero4;
  const float rr = rrf();
  auto sel = [&](int i) { return i == 1 ? c1 : c0; };
  auto scl = [](float4 v, float f) { return make_float4(v.x * f, v.y * f, v.z * f, v.w * f); };
  // emit
#pragma unroll
  for (int o = 0; o < TH_MAX_OUT; ++o) {
    if (o >= g.n_out) continue;
    const EpiOutK& eo = g.out[o];
    if (n4 < eo.cb || n4 >= eo.ce) continue;
    const float4 a = ((g.rscale_mask >> eo.a) & 1u) ? scl(sel(eo.a), rr) : sel(eo.a);
    float4 v;
    switch (eo.op) {
      case TH_EPI_ACC:
        v = a;
        break;
      case TH_EPI_ROPE:
      case TH_EPI_ROPE_PAIR: {
        float4 r;
        if (eo.op == TH_EPI_ROPE) {
          const float sg = within < half ? -1.f : 1.f;
          r = scl(eo.a == 1 ? rot1 : rot0, ((g.rscale_mask >> eo.a) & 1u) ? sg * rr : sg);
        } else {
          r = ((g.rscale_mask >> eo.b) & 1u) ? scl(sel(eo.b), rr) : sel(eo.b);
        }
        v = make_float4(a.x * cs.x + r.x * sn.x, a.y * cs.y + r.y * sn.y, a.z * cs.z + r.z * sn.z,
                        a.w * cs.w + r.w * sn.w);
        break;
      }
      case TH_EPI_SILU:
        v = make_float4(a.x * sigmoidf_(a.x), a.y * sigmoidf_(a.y), a.z * sigmoidf_(a.z), a.w * sigmoidf_(a.w));
        break;
      case TH_EPI_SWIGLU: {
        const float4 b = ((g.rscale_mask >> eo.b) & 1u) ? scl(sel(eo.b), rr) : sel(eo.b);
        v = make_float4(a.x * sigmoidf_(a.x) * b.x, a.y * sigmoidf_(a.y) * b.y, a.z * sigmoidf_(a.z) * b.z,
                        a.w * sigmoidf_(a.w) * b.w);
        break;
      }
      default: {  // TH_EPI_ADD, TH_EPI_SOFTPLUS_ADD, TH_EPI_MUL
        const float4 x = xe[o];
        if (eo.op == TH_EPI_MUL) {
          v = make_float4(a.x * x.x, a.y * x.y, a.z * x.z, a.w * x.w);
        } else {
          v = make_float4(a.x + x.x, a.y + x.y, a.z + x.z, a.w + x.w);
          if (eo.op == TH_EPI_SOFTPLUS_ADD)
            v = make_float4(softplusf_(v.x), softplusf_(v.y), softplusf_(v.z), softplusf_(v.w));
        }
        break;
      }
    }
    if (g.gain_out != nullptr && o == g.gain_index) {
      // the value the output would hold, then times the next RMSNorm's gain
      auto rb = [](float f) { return __uint_as_float((uint32_t)f32_to_bf16(f) << 16); };
      const float4 r = make_float4(rb(v.x), rb(v.y), rb(v.z), rb(v.w));
      ssg = ((r.x * r.x + r.y * r.y) + r.z * r.z) + r.w * r.w;
      v = make_float4(r.x * gq.x, r.y * gq.y, r.z * gq.z, r.w * gq.w);
    }
    store4(eo.ptr, m * eo.ld + (n4 - eo.cb), eo.dtype, eo.vec != 0, (int)min((int64_t)valid, eo.ce - n4), v);
  }
  return ssg;
}

// The outputs of packed tile t (output columns t bn .. +bn of every
// accumulator) from the workgroup's finished sums, staged in LDS as
// tl[m][i bn + j] (row stride ld floats), with the tile's per-column scales
// at sc[i bn + j]; rrs holds the M row scales. One thread per (row, 4
// columns).
__device__ __forceinline__ void fp8_tile_out(const Fp8K& p, int t, int tid, int nthr, const float* tl, int ld,
                                             const float* sc, const float* rrs) {
  const int M = (int)p.M, bn = (int)p.bn, q4 = bn >> 2;
  const int64_t n0 = (int64_t)t * bn;
  for (int e = tid; e < M * q4; e += nthr) {
    const int m = e / q4;
    const int64_t n4 = n0 + ((e - m * q4) << 2);
    if (n4 >= p.N) continue;
    const float* row = tl + m * ld - n0;
    const float* scr = sc - n0;
    fp8_emit4(p, m, n4, [&] { return rrs[m]; }, [&](int i, int64_t nn, bool) {
      const float4 v = *(const float4*)(row + i * bn + nn);
      const float4 s4 = *(const float4*)(scr + i * bn + nn);
      return make_float4(v.x * s4.x, v.y * s4.y, v.z * s4.z, v.w * s4.w);
    }, [] {});
  }
}

// grid (Npk / (128 NG), splits), eight waves per workgroup. Waves w and
// w + 4 own the same 32 NG packed columns and take the two K halves of every
// slice (intra-workgroup split-K, summed in LDS at the end), so two waves
// share each SIMD: one wave's LDS round trips and barrier waits overlap the
// other's MFMAs (one wave per SIMD leaves the MFMA pipe mostly idle).
// Activation slices (KS of K for all 32 TM rows) stream into NBUF rotating
// LDS buffers by direct loads, cooperatively, while each wave loads its own
// weights (NG KiB per 32-K chunk, fragment-major) into registers, both P
// slices ahead of the MFMAs; one barrier per slice frees the buffer slice
// j + P lands in.
// LDS slice layout: row r (one activation row, 2 KS bytes) holds its 16-byte
// chunk c in slot c ^ (r % 16), so the 32-row operand reads (one chunk per
// lane) hit distinct banks; the permutation is applied on the load side and
// the direct loads write 1 KiB (1024 / (2 KS) rows) linearly per instruction.
// An activation-side RMSNorm gain never reaches this kernel: the launcher
// first scales the rows once (fp8_gain_prep_kernel) and hands over their sums
// of squares (p.ss_pre), instead of every workgroup rescaling the same rows.
template <int TM, int NG, int KS>  // 32-row tiles of M (M <= 32 TM); 32-column groups per wave; K per slice
__global__ void __launch_bounds__(512) gemm_fp8_lds_kernel(Fp8K p) {
  constexpr int ROWS = 32 * TM;
  constexpr int RB = 2 * KS;           // bytes per activation row of a slice
  constexpr int SLB = ROWS * RB;       // bytes per activation slice
  constexpr int NWV = 8;               // waves per workgroup: 4 column groups x 2 K halves
  constexpr int NT = 64 * NWV;         // threads per workgroup
  constexpr int P = 2;                 // slices in flight ahead of the MFMAs (measured best of 2, 3, 5)
  constexpr int NBUF = P + 1;          // slice buffers (LDS) and weight register slots
  constexpr int ALD = SLB / 1024 / NWV;  // activation loads per wave per slice
  constexpr int RPI = 1024 / RB;       // rows per activation load
  constexpr int LPR = RB / 16;         // lanes per row in an activation load
  constexpr int NCH = KS / 32;         // 32-K chunks per slice
  constexpr int NCHH = NCH / 2;        // chunks per K half
  constexpr int WLD = NCHH * NG;       // weight loads per wave per slice
  constexpr int PARTS = NT / ROWS;     // threads per row in the sum of squares
  constexpr int CPP = LPR / PARTS;     // 16-byte chunks per such thread and slice
  static_assert(ALD >= 1 && NCH % 2 == 0 && CPP >= 1, "shape of the eight-wave pipeline");
  __shared__ __attribute__((aligned(16))) char sa[NBUF * SLB];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kh = wave >> 2, wc = wave & 3;  // K half, column group
  const int h = lane >> 5, c32 = lane & 31;
  const int split = blockIdx.y;
  const int64_t kb = (int64_t)split * p.ksplit;
  const int nsl = (int)((min(p.K, kb + p.ksplit) - kb) / KS);
  const int64_t nch = p.ldb / 32;
  const int64_t g0 = ((int64_t)blockIdx.x * 4 + wc) * NG;  // first 32-row group of this wave
  const uint8_t* bw = (const uint8_t*)p.B + (g0 * nch + kb / 32 + kh * NCHH) * 1024 + 16 * lane;
  const char* abase = (const char*)p.A + kb * 2;
  // row sums of squares (unless handed over): every workgroup when it
  // finishes its tile itself, else the first column block of each split
  const bool do_ss = p.k.sumsq && !p.ss_pre && (p.fused || blockIdx.x == 0);
  // row sums handed over as the lhs producer's parts (up to 16): loaded by
  // every thread at the start (rows and parts clamped into range: no branch,
  // so the compiler keeps its additions, and their wait, at the tile's end)
  // and added up there, in row_sumsq's order, by the row's first thread
  const bool pre_rs = p.k.sumsq && p.ss_pre == 2 && p.fused && p.k.n_rs_parts <= 16;
  float4 rsp[4];
  if (pre_rs) {
    const int64_t rr = min((int64_t)(tid / PARTS), p.M - 1);
    const float4* q = (const float4*)(p.k.rs_parts + rr * p.k.ld_rs_parts);
    const int nq4 = p.k.n_rs_parts >> 2;
#pragma unroll
    for (int i = 0; i < 4; ++i) rsp[i] = q[i < nq4 ? i : 0];
  }

  // activation load q of this wave fills slice rows RPI (ALD wave + q) + lane / LPR,
  // slot lane % LPR; rows past M re-read row M - 1 (their sums are dropped)
  uint32_t aoff[ALD];
#pragma unroll
  for (int q = 0; q < ALD; ++q) {
    const int r = RPI * (ALD * wave + q) + lane / LPR;
    const int rr = min(r, (int)p.M - 1);
    aoff[q] = (uint32_t)rr * (uint32_t)p.lda * 2u + (uint32_t)(((lane % LPR) ^ (r & 15)) << 4);
  }

  uint4 wb[NBUF][NCHH][NG];
  f32x16_t acc[TM][NG];
#pragma unroll
  for (int t = 0; t < TM; ++t)
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[t][g][r] = 0.f;
  float ss = 0.f;

  // slice j goes to LDS buffer j % NBUF and weight slot j % NBUF;
  // workgroups start their K walk at different slices (rotated), so the
  // weight streams of concurrent workgroups do not advance in lockstep
  const int rot = (int)((blockIdx.x * 5u) % (unsigned)nsl);
  auto issue = [&](int j0, auto slot) {
    constexpr int SL = decltype(slot)::value;
    const int j = j0 + rot < nsl ? j0 + rot : j0 + rot - nsl;
    const char* asrc = abase + (int64_t)j * KS * 2;
    char* ad = sa + SL * SLB + ALD * wave * 1024;
#pragma unroll
    for (int q = 0; q < ALD; ++q)
      __builtin_amdgcn_global_load_lds((const void*)(asrc + aoff[q]), (lds_ptr_t)(ad + q * 1024), 16, 0, 0);
    const uint8_t* wsrc = bw + (int64_t)j * NCH * 1024;
#pragma unroll
    for (int c = 0; c < NCHH; ++c)
#pragma unroll
      for (int g = 0; g < NG; ++g) wb[SL][c][g] = *(const uint4*)(wsrc + ((int64_t)g * nch + c) * 1024);
  };
  auto compute = [&](auto slot) {
    constexpr int SL = decltype(slot)::value;
    const char* ab = sa + SL * SLB + c32 * RB;
    // this wave's K half of the slice: chunks kh NCHH .. kh NCHH + NCHH - 1;
    // every A fragment is read before the first MFMA
    bf16x8_t a[NCHH][TM][2];
#pragma unroll
    for (int c = 0; c < NCHH; ++c)
#pragma unroll
      for (int t = 0; t < TM; ++t) {
        const int cg = kh * NCHH + c;
        a[c][t][0] = *(const bf16x8_t*)(ab + t * 32 * RB + (((4 * cg + 2 * h) ^ (c32 & 15)) << 4));
        a[c][t][1] = *(const bf16x8_t*)(ab + t * 32 * RB + (((4 * cg + 2 * h + 1) ^ (c32 & 15)) << 4));
      }
#pragma unroll
    for (int c = 0; c < NCHH; ++c) {
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        const bf16x8_t b0 = fp8x8_to_bf16x8(wb[SL][c][g].x, wb[SL][c][g].y);
        const bf16x8_t b1 = fp8x8_to_bf16x8(wb[SL][c][g].z, wb[SL][c][g].w);
#pragma unroll
        for (int t = 0; t < TM; ++t) {
          acc[t][g] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[c][t][0], b0, acc[t][g], 0, 0, 0);
          acc[t][g] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[c][t][1], b1, acc[t][g], 0, 0, 0);
        }
      }
    }
    // reads first, then the MFMAs (the scheduler would otherwise sink each
    // read to its first use): at most 8 reads are outstanding for M <= 64
    if constexpr (NCHH * TM * 2 <= 8) {
      __builtin_amdgcn_sched_group_barrier(0x100, NCHH * TM * 2, 0);       // DS reads
      __builtin_amdgcn_sched_group_barrier(0x008, NCHH * TM * 2 * NG, 0);  // MFMAs
    }
    if (do_ss) {
      const int row = tid / PARTS, part = tid % PARTS;
      const char* ar = sa + SL * SLB + row * RB;
#pragma unroll
      for (int cc = 0; cc < CPP; ++cc) {
        const bf16x8_t v = *(const bf16x8_t*)(ar + (((part * CPP + cc) ^ (row & 15)) << 4));
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = (float)v[e];
          ss += x * x;
        }
      }
    }
  };
  // Every step issues one slice (past the end: the last slice again, an L2
  // re-read into a buffer nobody reads), so the in-flight count is the same
  // at every wait and the compiler needs no waits of its own.
  // A step past the last slice (j >= nsl, padding the last trip) waits and
  // issues like the others but computes nothing: every trip is then the same
  // straight-line code, and no conditional step makes the compiler drain all
  // loads in flight at the loop's exit.
  auto step = [&](int j, auto slot) {
    constexpr int SL = decltype(slot)::value;
    // slice j has landed (slices j + 1 .. j + P - 1 may still be in flight)
    // and every wave is done with slice j - 1, whose buffer slice j + P reuses
    wait_vmcnt<(P - 1) * (ALD + WLD)>();
    barrier_keep_loads();
    issue(min(j + P, nsl - 1), std::integral_constant<int, (SL + P) % NBUF>());
    if (j < nsl) compute(slot);
  };

  unroll_seq(std::make_integer_sequence<int, P>(), [&](auto s) { issue(min((int)s, nsl - 1), s); });
  // whole trips of NBUF steps (the last one padded): one in-flight pattern at every wait
  for (int j = 0; j < nsl; j += NBUF)
    unroll_seq(std::make_integer_sequence<int, NBUF>(), [&](auto s) { step(j + (int)s, s); });
  wait_vmcnt<0>();  // no direct-to-LDS load may land after the workgroup ends

  // the two K halves meet: waves 4..7 hand their sums to waves 0..3 through
  // the (now free) slice buffers, in a fixed order (half 0 + half 1)
  static_assert(4 * TM * NG * 16 * 64 * 4 <= NBUF * SLB, "half sums fit the slice buffers");
  {
    float* xs = (float*)sa;
    __syncthreads();  // every wave is done reading the slice buffers
    if (kh == 1) {
#pragma unroll
      for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int g = 0; g < NG; ++g)
#pragma unroll
          for (int r = 0; r < 16; ++r) xs[(((wc * TM + t) * NG + g) * 16 + r) * 64 + lane] = acc[t][g][r];
    }
    __syncthreads();
    if (kh == 0) {
#pragma unroll
      for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int g = 0; g < NG; ++g)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[t][g][r] += xs[(((wc * TM + t) * NG + g) * 16 + r) * 64 + lane];
    }
  }
  if (do_ss) {
#pragma unroll
    for (int o = 1; o < PARTS; o <<= 1) ss += __shfl_xor(ss, o);
  }
  if (!p.fused) {
    float* part = p.part + (int64_t)split * p.M * p.Npk;
    if (kh == 0) {
#pragma unroll
      for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          const int64_t col = (g0 + g) * 32 + c32;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int m = 32 * t + 8 * (r >> 2) + 4 * h + (r & 3);
            if (m < p.M) part[(int64_t)m * p.Npk + col] = acc[t][g][r];
          }
        }
    }
    const int row = tid / PARTS;
    if (do_ss && tid % PARTS == 0 && row < p.M) p.sumsq_part[(int64_t)split * p.M + row] = ss;
    return;
  }
  // One split, every output op inside the tile: finish it here. The
  // accumulators go to the (now free) slice buffers as tl[m][packed column],
  // row stride 132 floats, followed by the row scales (one LDS object keeps
  // the compiler's LDS alias tracking exact, so it adds no waits on the
  // direct loads).
  constexpr int LDT = 128 * NG + 4;
  static_assert(ROWS * LDT * 4 + ROWS * 4 + 128 * NG * 4 <= NBUF * SLB, "tile staging fits the slice buffers");
  float* tl = (float*)sa;
  float* rrs = tl + ROWS * LDT;
  float* scl = rrs + ROWS;  // the tile's 128 NG per-column scales, packed-column order
  __syncthreads();
  for (int c = tid; c < 128 * NG; c += NT) {
    const int i = c / (int)p.bn, j = c - i * (int)p.bn;
    const int64_t n = (int64_t)blockIdx.x * p.bn + j;
    scl[c] = n < p.N ? p.scale[(int64_t)i * p.N + n] : 0.f;
  }
  if (kh == 0) {
#pragma unroll
    for (int t = 0; t < TM; ++t)
#pragma unroll
      for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = 32 * t + 8 * (r >> 2) + 4 * h + (r & 3);
          tl[m * LDT + (wc * NG + g) * 32 + c32] = acc[t][g][r];
        }
  }
  if (tid % PARTS == 0 && tid / PARTS < p.M) {
    const int row = tid / PARTS;
    float rr = 1.f;
    if (p.k.sumsq) {
      float s = ss;
      if (pre_rs) {
        s = rsp[0].x;
        s += rsp[0].y;
        s += rsp[0].z;
        s += rsp[0].w;
#pragma unroll
        for (int i = 1; i < 4; ++i) {
          const bool in = i < (p.k.n_rs_parts >> 2);
          float t = s + rsp[i].x;
          t += rsp[i].y;
          t += rsp[i].z;
          t += rsp[i].w;
          s = in ? t : s;
        }
      } else if (p.ss_pre == 2) {
        s = row_sumsq(p.k, row, 0.f);
      } else if (p.ss_pre) {
        s = p.sumsq_part[row];
      }
      rr = rsqrtf(s * p.k.inv_k + p.k.eps);
      if (p.k.sumsq_out && blockIdx.x == 0) p.k.sumsq_out[row] = s;
    }
    rrs[row] = rr;
  }
  __syncthreads();
  fp8_tile_out(p, (int)blockIdx.x, tid, NT, tl, LDT, scl, rrs);
}

// The activation-side RMSNorm gain, once per call: row m of the operand
// becomes bf16(x[m, k] * g[k]) (fp32 product, round to nearest even) and the
// row's sum of squares (of the unscaled x) goes to split 0's sum slot, the
// other splits' slots to zero, where the kernels and the reduce pass read the
// sums. One workgroup per row; a thread takes 8-element chunks 8 (tid + 256 u),
// u < U, of each 8192-wide span, all of whose loads are issued before the
// first is used (one memory round trip per span). K a multiple of 8, rows
// 16-byte aligned.
template <int U>
__global__ void __launch_bounds__(256) fp8_gain_prep_kernel(const uint16_t* x, int64_t lda, const float* g, int64_t K,
                                                            uint16_t* xg, float* ss, int64_t M, int splits) {
  __shared__ float red[4];
  const int64_t m = blockIdx.x;
  const int tid = threadIdx.x;
  const uint16_t* xr = x + m * lda;
  uint16_t* yr = xg + m * K;
  float acc = 0.f;
  for (int64_t k0 = 0; k0 < K; k0 += 8 * 256 * U) {
    u32x4_t v[U];
    f32x4_t ga[U], gb[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t k = k0 + 8 * (tid + 256 * u);
      if (k < K) {
        v[u] = *(const u32x4_t*)(xr + k);
        ga[u] = *(const f32x4_t*)(g + k);
        gb[u] = *(const f32x4_t*)(g + k + 4);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t k = k0 + 8 * (tid + 256 * u);
      if (k >= K) continue;
      const float gg[8] = {ga[u][0], ga[u][1], ga[u][2], ga[u][3], gb[u][0], gb[u][1], gb[u][2], gb[u][3]};
      u32x4_t o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = __uint_as_float(v[u][e] << 16), hi = __uint_as_float(v[u][e] & 0xffff0000u);
        acc += lo * lo + hi * hi;
        const bf16x2_t pr = {(__bf16)(lo * gg[2 * e]), (__bf16)(hi * gg[2 * e + 1])};
        o[e] = __builtin_bit_cast(uint32_t, pr);
      }
      *(u32x4_t*)(yr + k) = o;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
  if ((tid & 63) == 0) red[tid >> 6] = acc;
  __syncthreads();
  if (tid == 0) ss[m] = (red[0] + red[1]) + (red[2] + red[3]);
  for (int s = 1 + tid; s < splits; s += 256) ss[(int64_t)s * M + m] = 0.f;
}

// acc_i(m, n) from the partials, scaled: s_i[n] * sum over splits.
__device__ __forceinline__ float fp8_acc(const Fp8K& p, int i, int64_t m, int64_t n) {
  const int64_t t = n / p.bn, j = n - t * p.bn;
  const int64_t row = (t * p.k.n_acc + i) * p.bn + j;
  float s = 0.f;
  for (int sp = 0; sp < p.splits; ++sp) s += p.part[((int64_t)sp * p.M + m) * p.Npk + row];
  return s * p.scale[(int64_t)i * p.N + n];
}

// Per-wave split-K kernel's second pass: one thread per (row m, output
// column n); every fused output op.
__global__ void __launch_bounds__(256) gemm_fp8_reduce_kernel(Fp8K p) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)p.M * p.N) return;
  const int64_t m = idx / p.N, n = idx - m * p.N;
  const GemmK& g = p.k;
  float rr = 1.f;
  if (g.sumsq) {
    float ss = 0.f;
    if (p.ss_pre == 2)
      ss = row_sumsq(g, m, 0.f);
    else
      for (int sp = 0; sp < p.splits; ++sp) ss += p.sumsq_part[(int64_t)sp * p.M + m];
    rr = rsqrtf(ss * g.inv_k + g.eps);
    if (g.sumsq_out && n == 0) g.sumsq_out[m] = ss;
  }
  fp8_emit(p, m, n, rr, [&](int i, int64_t nn) { return fp8_acc(p, i, m, nn); });
}

// Second pass after a multi-split launch of the shared-activation kernel:
// one thread per (row m, 4 consecutive output columns), float4 partial loads,
// sums in split order, 4-wide stores. S > 0: exactly S splits, every partial
// the thread adds (its columns, the RoPE partner's, the row's sums of squares)
// loaded before the first is added, with the extras and RoPE tables: one
// memory round trip. S = 0: any split count, a loop per sum. Requires
// N % 4 == 0 and a power-of-two bn (so 4 columns share a tile). With
// gain_out (N a multiple of 1024, so every wave is whole and inside one row),
// each wave sums its 256 columns' bf16(v)^2 into ss_parts_out.
template <int S>
__global__ void __launch_bounds__(256) gemm_fp8_reduce4_kernel(Fp8K p) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t nq = p.N >> 2;
  if (idx >= p.M * nq) return;
  const int64_t m = idx / nq, n4 = (idx - m * nq) << 2;
  const GemmK& g = p.k;
  const int na = g.n_acc;
  const int sh = __builtin_ctz((unsigned)p.bn);
  const int64_t plane = p.M * p.Npk;
  auto part_ptr = [&](int i, int64_t nn) {
    const int64_t t = nn >> sh, j = nn & (p.bn - 1);
    return p.part + m * p.Npk + ((t * na + i) << sh) + j;
  };
  auto row_scale = [&](float ss) {
    if (g.sumsq_out && n4 == 0) g.sumsq_out[m] = ss;
    return rsqrtf(ss * g.inv_k + g.eps);
  };
  // the wave's part of the gain output's row sum of squares (lane order fixed)
  auto store_ss_part = [&](float v) {
    if (g.gain_out == nullptr) return;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) v += __shfl_xor(v, off);
    if ((threadIdx.x & 63) == 0) g.ss_parts_out[m * g.ld_ss_parts_out + (n4 >> 8)] = v;
  };
  if constexpr (S == 0) {
    const int ns = p.splits;
    // accumulator i at output columns nn .. nn+3 (nn a multiple of 4), scaled
    auto sum4 = [&](int i, int64_t nn, bool) {
      const float* q = part_ptr(i, nn);
      float4 acc = *(const float4*)q;
#pragma unroll 8
      for (int sp = 1; sp < ns; ++sp) {
        const float4 v = *(const float4*)(q + sp * plane);
        acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
      }
      const float4 sc = *(const float4*)(p.scale + (int64_t)i * p.N + nn);
      return make_float4(acc.x * sc.x, acc.y * sc.y, acc.z * sc.z, acc.w * sc.w);
    };
    float rr = 1.f;
    if (g.sumsq) {
      float ss = 0.f;
      if (p.ss_pre == 2) {
        ss = row_sumsq(g, m, 0.f);
      } else {
        ss = p.sumsq_part[m];
        for (int sp = 1; sp < ns; ++sp) ss += p.sumsq_part[(int64_t)sp * p.M + m];
      }
      rr = row_scale(ss);
    }
    store_ss_part(fp8_emit4(p, m, n4, [&] { return rr; }, sum4, [] {}));
  } else {
    // the accumulators and RoPE partners this thread's outputs read
    bool rope_acc[2] = {false, false};
    for (int o = 0; o < g.n_out; ++o) {
      const EpiOutK& eo = g.out[o];
      if (n4 >= eo.cb && n4 < eo.ce && eo.op == TH_EPI_ROPE) rope_acc[eo.a & 1] = true;
    }
    const int within = g.hd > 0 ? (int)n4 % g.hd : 0;
    const int64_t pn = within < (g.hd >> 1) ? n4 + (g.hd >> 1) : n4 - (g.hd >> 1);
    // (zero where not loaded: an undefined value there would let the compiler
    // move the first additions up between the loads, each with its own wait)
    float4 pa[2][S], pr[2][S], sa[2], sr[2];
    float ps[S];
#pragma unroll
    for (int i = 0; i < 2; ++i) sa[i] = sr[i] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int sp = 0; sp < S; ++sp) {
      pa[0][sp] = pa[1][sp] = pr[0][sp] = pr[1][sp] = make_float4(0.f, 0.f, 0.f, 0.f);
      ps[sp] = 0.f;
    }
    auto gather = [&] {
      if (g.sumsq && p.ss_pre != 2) {
#pragma unroll
        for (int sp = 0; sp < S; ++sp) ps[sp] = p.sumsq_part[(int64_t)sp * p.M + m];
      }
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        if (i < na) {
          const float* q = part_ptr(i, n4);
#pragma unroll
          for (int sp = 0; sp < S; ++sp) pa[i][sp] = *(const float4*)(q + sp * plane);
          sa[i] = *(const float4*)(p.scale + (int64_t)i * p.N + n4);
        }
        if (i < na && rope_acc[i]) {
          const float* q = part_ptr(i, pn);
#pragma unroll
          for (int sp = 0; sp < S; ++sp) pr[i][sp] = *(const float4*)(q + sp * plane);
          sr[i] = *(const float4*)(p.scale + (int64_t)i * p.N + pn);
        }
      }
    };
    // the same sums, in the same order, as the S = 0 form
    auto sum4 = [&](int i, int64_t, bool rot) {
      float4 acc = rot ? pr[i][0] : pa[i][0];
#pragma unroll
      for (int sp = 1; sp < S; ++sp) {
        const float4 v = rot ? pr[i][sp] : pa[i][sp];
        acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
      }
      const float4 sc = rot ? sr[i] : sa[i];
      return make_float4(acc.x * sc.x, acc.y * sc.y, acc.z * sc.z, acc.w * sc.w);
    };
    auto rrf = [&] {
      if (!g.sumsq) return 1.f;
      if (p.ss_pre == 2) return row_scale(row_sumsq(g, m, 0.f));
      float ss = ps[0];
#pragma unroll
      for (int sp = 1; sp < S; ++sp) ss += ps[sp];
      return row_scale(ss);
    };
    store_ss_part(fp8_emit4(p, m, n4, rrf, sum4, gather));
  }
}

// Split count: about one workgroup per CU, each wave at least 256 of K.
static int fp8_groups(int64_t Npk) { return Npk % 64 == 0 ? 2 : 1; }

// The shared-activation kernel: one workgroup per packed tile of 128 columns
// (bn = 128 / n_acc), K in whole 128-wide slices. Split count: about one
// workgroup per CU, a single split once the tiles alone nearly fill the GPU
// (that launch finishes its tiles itself, without the reduce kernel).
static bool fp8_lds_ok(int64_t Npk, int64_t K, int bn, int n_acc) {
  return K % 128 == 0 && (n_acc == 1 || n_acc == 2) && bn * n_acc == 128 && Npk % 128 == 0;
}

static int fp8_lds_splits(int64_t Npk, int64_t K) {
  const int64_t nsl = K / 128;
  const int64_t cus = device_cus() > 0 ? device_cus() : 256;
  const int64_t nb = Npk / 128;
  if (4 * nb >= 3 * cus) return 1;
  // as many splits as keep the launch within one round of one workgroup per CU
  return (int)std::min(std::max((int64_t)1, cus / nb), std::min(nsl, (int64_t)16));
}

static int fp8_splits(int64_t Npk, int64_t K) {
  const int64_t cus = device_cus() > 0 ? device_cus() : 256;
  const int64_t nb = Npk / (32 * fp8_groups(Npk));
  int64_t s = cdiv(cus, nb);
  s = std::min(s, std::max((int64_t)1, K / 1024));
  return (int)std::max((int64_t)1, std::min(s, (int64_t)64));
}

// Workspace: [splits][M][Npk] partial sums, [splits][M] partial row sums of
// squares, then (shared-activation kernel) the gain-scaled operand bf16 [M][K],
// 256-byte aligned.
static int64_t fp8_gain_offset(int64_t M, int64_t Npk, int s) { return cdiv((int64_t)s * M * (Npk + 1) * 4, 256) * 256; }

int64_t fp8_workspace_bytes(int64_t M, int64_t Npk, int64_t K, int bn, int n_acc) {
  if (!fp8_lds_ok(Npk, K, bn, n_acc)) return (int64_t)fp8_splits(Npk, K) * M * (Npk + 1) * 4;
  const int s = fp8_lds_splits(Npk, K);
  return fp8_gain_offset(M, Npk, s) + M * K * 2;
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
  const bool lds = fp8_lds_ok(Npk, k.K, (int)k.bn, k.n_acc);
  p.splits = lds ? fp8_lds_splits(Npk, k.K) : fp8_splits(Npk, k.K);
  p.ksplit = cdiv(cdiv(k.K, p.splits), 128) * 128;  // whole slices / four waves x a multiple of 32
  p.splits = (int)cdiv(k.K, p.ksplit);
  const int64_t need = lds ? fp8_gain_offset(k.M, Npk, p.splits) + k.M * k.K * 2
                           : (int64_t)p.splits * k.M * (Npk + 1) * 4;
  TH_CHECK_ARG(ws && ws_bytes >= need, "th_gemm: fp8 weights need a workspace of %lld bytes (got %lld)",
               (long long)need, (long long)ws_bytes);
  p.part = ws;
  p.sumsq_part = k.sumsq ? ws + (int64_t)p.splits * k.M * Npk : nullptr;
  if (k.rs_parts != nullptr) p.ss_pre = 2;  // the row sums come from the lhs's producer
  // 4-column output groups: inside one tile and one RoPE half-head
  bool vec = k.N % 4 == 0 && (k.bn & (k.bn - 1)) == 0;
  for (int o = 0; o < k.n_out; ++o) {
    if (k.out[o].op == TH_EPI_ROPE && k.hd % 8 != 0) vec = false;
    if (k.out[o].op == TH_EPI_ROPE_PAIR && k.hd % 4 != 0) vec = false;
  }
  if (k.gain_out != nullptr && !(lds && vec)) {
    set_error("th_gemm: gain_out needs the shared-activation e4m3 kernel with 4-column outputs "
              "(K a multiple of 128, 128-column packed tiles)");
    return TH_ERR_UNSUPPORTED;
  }
  if (lds) {
    TH_CHECK_ARG(k.lda < (1 << 24), "th_gemm: fp8 lhs row stride must be under 2^24 elements");
    if (k.gain) {
      // the gain-scaled rows and their (unscaled) sums of squares, once
      TH_CHECK_ARG(k.sumsq, "th_gemm: lhs_gain needs the row sum of squares (sumsq)");
      TH_CHECK_ARG(k.lda % 8 == 0 && ((uintptr_t)k.A & 15) == 0,
                   "th_gemm: lhs_gain needs 16-byte aligned lhs rows");
      uint16_t* xg = (uint16_t*)((char*)ws + fp8_gain_offset(k.M, Npk, p.splits));
      hipLaunchKernelGGL(fp8_gain_prep_kernel<4>, dim3((unsigned)k.M), dim3(256), 0, stream, (const uint16_t*)k.A,
                         k.lda, k.gain, k.K, xg, p.sumsq_part, k.M, p.splits);
      TH_CHECK_LAUNCH();
      p.A = xg;
      p.lda = k.K;
      p.ss_pre = 1;
    }
    // one split finishes in the main kernel when RoPE partners stay in a tile
    // (and no output's row sums are taken: those need whole waves per row)
    bool local = p.splits == 1 && vec && k.gain_out == nullptr;
    for (int o = 0; o < k.n_out; ++o)
      if (k.out[o].op == TH_EPI_ROPE && k.bn % k.hd != 0) local = false;
    p.fused = local ? 1 : 0;
    const dim3 g1((unsigned)(Npk / 128), (unsigned)p.splits);
    if (k.M <= 32)
      hipLaunchKernelGGL((gemm_fp8_lds_kernel<1, 1, 128>), g1, dim3(512), 0, stream, p);
    else if (k.M <= 64)
      hipLaunchKernelGGL((gemm_fp8_lds_kernel<2, 1, 128>), g1, dim3(512), 0, stream, p);
    else
      hipLaunchKernelGGL((gemm_fp8_lds_kernel<4, 1, 128>), g1, dim3(512), 0, stream, p);
    TH_CHECK_LAUNCH();
    if (!p.fused) {
      if (vec) {
        const dim3 gr((unsigned)cdiv(k.M * (k.N / 4), 256));
        switch (p.splits) {
#define TH_FP8_RED4(S_) \
  case S_:              \
    hipLaunchKernelGGL(gemm_fp8_reduce4_kernel<S_>, gr, dim3(256), 0, stream, p); \
    break;
          TH_FP8_RED4(2) TH_FP8_RED4(3) TH_FP8_RED4(4) TH_FP8_RED4(5) TH_FP8_RED4(6) TH_FP8_RED4(7) TH_FP8_RED4(8)
#undef TH_FP8_RED4
          default:
            hipLaunchKernelGGL(gemm_fp8_reduce4_kernel<0>, gr, dim3(256), 0, stream, p);
        }
      }
      else
        hipLaunchKernelGGL(gemm_fp8_reduce_kernel, dim3((unsigned)cdiv(k.M * k.N, 256)), dim3(256), 0, stream, p);
      TH_CHECK_LAUNCH();
    }
    return TH_OK;
  }
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

// ------------------------------------------------------------ no-alloc entry
// Scratch memory of th_gemm_noalloc: the e4m3 path's split-K partial sums (and
// partial row sums of squares) in a file-scope device array, one copy per GPU,
// held until the process ends. Host code never passes the array's name to a
// kernel or a copy (that is a host-side stand-in, not a device address): each
// device's address comes from hipGetSymbolAddress at th_init.
static __device__ __align__(256) float scratch[TH_GEMM_NOALLOC_SCRATCH_BYTES / 4];
static void* g_scratch[64];

int fp8_scratch_init_device(int device) {
  void* ptr = nullptr;
  TH_CHECK_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
  g_scratch[device] = ptr;
  return TH_OK;
}

}  // namespace th

using namespace th;

extern "C" int th_gemm_noalloc(const th_gemm_desc* d, void* stream) {
  TH_CHECK_ARG(d != nullptr, "th_gemm_noalloc: null descriptor");
  // bf16 / fp32 weights: th_gemm with no workspace (fp32 small grids then split K
  // inside each workgroup instead of through a workspace)
  if (d->in_dtype != TH_F8E4M3) {
    th_gemm_desc c = *d;
    c.workspace = nullptr;
    c.workspace_bytes = 0;
    return th_gemm(&c, stream);
  }
  const int64_t need = th_gemm_workspace_bytes(d->M, d->N, d->K, d->n_acc, d->in_dtype);
  TH_CHECK_ARG(need <= (int64_t)TH_GEMM_NOALLOC_SCRATCH_BYTES,
               "th_gemm_noalloc: M=%lld N=%lld K=%lld n_acc=%d need %lld bytes of scratch, above the fixed %lld "
               "(use th_gemm with a workspace)",
               (long long)d->M, (long long)d->N, (long long)d->K, d->n_acc, (long long)need,
               (long long)TH_GEMM_NOALLOC_SCRATCH_BYTES);
  int dev = -1;
  if (!device_ready() || hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64 || g_scratch[dev] == nullptr) {
    set_error("th_gemm_noalloc: th_init was not called for the current device");
    return TH_ERR_NOT_INIT;
  }
  th_gemm_desc c = *d;
  c.workspace = (float*)g_scratch[dev];
  c.workspace_bytes = TH_GEMM_NOALLOC_SCRATCH_BYTES;
  return th_gemm(&c, stream);
}
