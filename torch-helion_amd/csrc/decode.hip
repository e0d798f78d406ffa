// Decode-step attention over a KV cache (no counterpart kernel in the
// reference, which has no decode path; the math is softmax(q k^T * scale) v of
// optimizer/evaluate.py:139-146 for one query row per sequence, grouped KV
// heads as in the prefill kernel).
//
// One workgroup per (KV split, kv head, sequence) serves all G = Hq/Hkv query
// heads that share the kv head, so each cached K/V byte is read from HBM once.
// Each wave walks its own 32-key tiles of the split:
//   S^T = K Q^T   v_mfma_f32_32x32x16_bf16, K fragments straight from HBM
//                 (lane = one key row), Q^T held in registers (columns >= G
//                 are zero), so a lane owns one query column;
//   online softmax per query column (one lane^32 exchange);
//   O^T += V^T P^T  P^T taken from the S^T accumulators as they are, V staged
//                 into the wave's own LDS slice transposed, with the same
//                 within-k-step key order as the accumulators.
// No block barrier is needed inside the loop (every LDS slice is wave
// private). The four waves' partial (max, sum, o) are merged in LDS; with more
// than one split, a second kernel merges the splits.
#include "common.h"

namespace th {

struct DecK {
  const uint16_t* q;
  int64_t ldq;
  const uint16_t* k;
  int64_t ksb, kst;  // element strides of the K cache: sequence, token
  const uint16_t* v;
  int64_t vsb, vst;
  uint16_t* o;
  int64_t ldo;
  const int32_t* lengths;
  int fixed_len;
  int B, Hq, Hkv, G, nsplit;
  float scale_log2;
  float* part;  // [B][Hq][nsplit][D + 2]: m, l, o[D] (o unnormalised)
};

template <int D>
__global__ void __launch_bounds__(256) attn_decode_kernel(DecK p) {
  constexpr int NKS = D / 16;  // k steps of S^T = K Q^T
  constexpr int NDT = D / 32;  // 32-dim blocks of O^T
  constexpr int VROW = 32 * 2; // bytes per V^T row (one dim, 32 keys)
  constexpr int VSLICE = D * VROW;
  constexpr int GMAX = 16;
  __shared__ __attribute__((aligned(16))) char vsm[4 * VSLICE];
  __shared__ float mw[4][GMAX], lw[4][GMAX];
  __shared__ float ow[4][GMAX][D];

  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hl = lane >> 5, col = lane & 31;
  const int G = p.G;
  const int len = p.lengths ? p.lengths[b] : p.fixed_len;
  const int per = (len + p.nsplit - 1) / p.nsplit;
  const int s0 = split * per, s1 = min(len, s0 + per);

  // Q^T fragments: column col = query head kvh*G + col (zero for col >= G)
  bf16x8_t qf[NKS];
  const uint16_t* qrow = p.q + (int64_t)b * p.ldq + (int64_t)(kvh * G + col) * D;
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    if (col < G) {
      qf[ks] = *(const bf16x8_t*)(qrow + 16 * ks + 8 * hl);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[ks][e] = (__bf16)0.f;
    }
  }

  const uint16_t* kb = p.k + (int64_t)b * p.ksb + (int64_t)kvh * D;
  const uint16_t* vb = p.v + (int64_t)b * p.vsb + (int64_t)kvh * D;
  char* sv = vsm + wave * VSLICE;

  f32x16_t oacc[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[t][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  for (int t0 = s0 + 32 * wave; t0 < s1; t0 += 128) {
    // K fragments (row = key t0 + col) and this lane's share of the V tile
    bf16x8_t kf[NKS];
    const int key = t0 + col;
    const bool kok = key < s1;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      if (kok) {
        kf[ks] = *(const bf16x8_t*)(kb + (int64_t)key * p.kst + 16 * ks + 8 * hl);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) kf[ks][e] = (__bf16)0.f;
      }
    }
    // V^T: lane stages key pairs pr (keys 2pr, 2pr+1) for 16-byte dim chunks c
    constexpr int CH = D / 8;              // 16-byte chunks per V row
    constexpr int UNITS = 16 * CH / 64;    // (pair, chunk) units per lane
#pragma unroll
    for (int u = 0; u < UNITS; ++u) {
      const int id = lane + 64 * u;
      const int pr = id / CH, c = id - pr * CH;
      const int ka = t0 + 2 * pr, kb2 = ka + 1;
      const uint4 va = ka < s1 ? *(const uint4*)(vb + (int64_t)ka * p.vst + 8 * c) : make_uint4(0, 0, 0, 0);
      const uint4 vc = kb2 < s1 ? *(const uint4*)(vb + (int64_t)kb2 * p.vst + 8 * c) : make_uint4(0, 0, 0, 0);
      const uint32_t a[4] = {va.x, va.y, va.z, va.w};
      const uint32_t h[4] = {vc.x, vc.y, vc.z, vc.w};
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int d = 8 * c + q;
        const uint32_t lo = (q & 1) ? (a[q >> 1] >> 16) : (a[q >> 1] & 0xffffu);
        const uint32_t hi = (q & 1) ? (h[q >> 1] >> 16) : (h[q >> 1] & 0xffffu);
        const int sw = ((d >> 1) & 7) << 1;
        *(uint32_t*)(sv + d * VROW + ((pr ^ sw) << 2)) = lo | (hi << 16);
      }
    }
    // S^T = K Q^T
    f32x16_t s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks], qf[ks], s, 0, 0, 0);
    // online softmax per query column (keys of this column: this lane and lane^32)
    float mloc = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kk = t0 + 8 * (r >> 2) + 4 * hl + (r & 3);
      const float x = kk < s1 ? s[r] * p.scale_log2 : -INFINITY;
      s[r] = x;
      mloc = fmaxf(mloc, x);
    }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
    const float m_new = fmaxf(m_run, mloc);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2f(m_run - m_use);
    m_run = m_new;
    float lsum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float e = exp2f(s[r] - m_use);
      s[r] = e;
      lsum += e;
    }
    l_run = l_run * alpha + lsum;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[t][r] *= alpha;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // O^T += V^T P^T, two k steps of 16 keys
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      bf16x8_t pf;
#pragma unroll
      for (int e = 0; e < 8; ++e) pf[e] = (__bf16)s[8 * hh + e];
      const int w0 = 8 * hh + 2 * hl;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const int d = 32 * dt + col;
        const int sw = ((d >> 1) & 7) << 1;
        const char* vrow = sv + d * VROW;
        const uint2 lo = *(const uint2*)(vrow + ((w0 ^ sw) << 2));
        const uint2 hi = *(const uint2*)(vrow + (((w0 + 4) ^ sw) << 2));
        bf16x8_t vf;
        uint32_t* vw = (uint32_t*)&vf;
        vw[0] = lo.x; vw[1] = lo.y; vw[2] = hi.x; vw[3] = hi.y;
        oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, oacc[dt], 0, 0, 0);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // merge the four waves
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  if (col < G) {
    if (hl == 0) {
      mw[wave][col] = m_run;
      lw[wave][col] = l_tot;
    }
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) ow[wave][col][32 * dt + 8 * (r >> 2) + 4 * hl + (r & 3)] = oacc[dt][r];
  }
  __syncthreads();
  for (int e = tid; e < G * D; e += 256) {
    const int j = e / D, d = e - j * D;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) mx = fmaxf(mx, mw[w][j]);
    const float mu = mx == -INFINITY ? 0.f : mx;
    float l = 0.f, o = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float f = exp2f(mw[w][j] - mu);
      l += lw[w][j] * f;
      o += ow[w][j][d] * f;
    }
    const int hq = kvh * G + j;
    if (p.nsplit == 1) {
      p.o[(int64_t)b * p.ldo + (int64_t)hq * D + d] = f32_to_bf16(l > 0.f ? o / l : 0.f);
    } else {
      float* pp = p.part + (((int64_t)b * p.Hq + hq) * p.nsplit + split) * (D + 2);
      if (d == 0) {
        pp[0] = mx;
        pp[1] = l;
      }
      pp[2 + d] = o;
    }
  }
}

// Merge the splits of one (sequence, query head): o = sum_s o_s 2^(m_s - m) / sum_s l_s 2^(m_s - m).
template <int D>
__global__ void __launch_bounds__(D) attn_decode_merge_kernel(DecK p) {
  const int hq = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  const float* pp = p.part + ((int64_t)b * p.Hq + hq) * p.nsplit * (D + 2);
  float mx = -INFINITY;
  for (int s = 0; s < p.nsplit; ++s) mx = fmaxf(mx, pp[s * (D + 2)]);
  const float mu = mx == -INFINITY ? 0.f : mx;
  float l = 0.f, o = 0.f;
  for (int s = 0; s < p.nsplit; ++s) {
    const float f = exp2f(pp[s * (D + 2)] - mu);
    l += pp[s * (D + 2) + 1] * f;
    o += pp[s * (D + 2) + 2 + d] * f;
  }
  p.o[(int64_t)b * p.ldo + (int64_t)hq * D + d] = f32_to_bf16(l > 0.f ? o / l : 0.f);
}

static int decode_splits(int batch, int heads_kv, int max_len, int requested) {
  if (requested > 0) return requested;
  // about four workgroups per CU, each split at least 256 keys
  const int cus = device_cus() > 0 ? device_cus() : 256;
  int s = (int)cdiv(4 * cus, (int64_t)batch * heads_kv);
  s = std::min(s, (int)cdiv(max_len, 256));
  return std::max(1, std::min(s, 64));
}

}  // namespace th

using namespace th;

extern "C" int64_t th_attention_decode_workspace_bytes(int32_t batch, int32_t heads_q, int32_t heads_kv,
                                                       int32_t head_dim, int32_t max_len, int32_t n_split) {
  if (batch <= 0 || heads_q <= 0 || heads_kv <= 0 || head_dim <= 0 || max_len <= 0 || n_split < 0) return -1;
  const int s = decode_splits(batch, heads_kv, max_len, n_split);
  return s == 1 ? 0 : (int64_t)batch * heads_q * s * (head_dim + 2) * 4;
}

extern "C" int th_attention_decode(const th_decode_desc* d, void* stream) {
  TH_CHECK_ARG(d != nullptr, "th_attention_decode: null descriptor");
  TH_CHECK_ARG(d->batch > 0 && d->heads_q > 0 && d->heads_kv > 0 && d->max_len > 0,
               "th_attention_decode: sizes must be positive");
  TH_CHECK_ARG(d->heads_q % d->heads_kv == 0 && d->heads_q / d->heads_kv <= 16,
               "th_attention_decode: heads_q=%d must be a multiple of heads_kv=%d, at most 16 per kv head",
               d->heads_q, d->heads_kv);
  TH_CHECK_ARG(d->head_dim == 64 || d->head_dim == 128, "th_attention_decode: head_dim %d unsupported", d->head_dim);
  TH_CHECK_ARG(d->dtype == TH_BF16, "th_attention_decode: only bf16 q / cache / o");
  TH_CHECK_ARG(d->q && d->k_cache && d->v_cache && d->o, "th_attention_decode: null tensor pointer");
  TH_CHECK_ARG(d->lengths != nullptr || (d->fixed_len > 0 && d->fixed_len <= d->max_len),
               "th_attention_decode: fixed_len must be in 1..max_len when lengths is null");
  const int64_t row = (int64_t)d->heads_kv * d->head_dim;
  TH_CHECK_ARG(d->k_stride_t >= row && d->v_stride_t >= row && d->k_stride_b >= d->k_stride_t * d->max_len &&
                   d->v_stride_b >= d->v_stride_t * d->max_len,
               "th_attention_decode: cache strides too small for [batch][max_len][heads_kv][head_dim]");
  TH_CHECK_ARG(d->ld_q >= (int64_t)d->heads_q * d->head_dim && d->ld_o >= (int64_t)d->heads_q * d->head_dim,
               "th_attention_decode: q/o row strides smaller than heads_q*head_dim");
  TH_CHECK_ARG(d->ld_q % 8 == 0 && d->k_stride_t % 8 == 0 && d->v_stride_t % 8 == 0 && d->k_stride_b % 8 == 0 &&
                   d->v_stride_b % 8 == 0,
               "th_attention_decode: strides must be multiples of 8 elements");
  TH_CHECK_ARG((((uintptr_t)d->q | (uintptr_t)d->k_cache | (uintptr_t)d->v_cache) & 15) == 0,
               "th_attention_decode: q and caches must be 16-byte aligned");
  const int ns = decode_splits(d->batch, d->heads_kv, d->max_len, d->n_split);
  TH_CHECK_ARG(ns <= d->max_len, "th_attention_decode: n_split %d above max_len", ns);
  if (ns > 1) {
    const int64_t need = (int64_t)d->batch * d->heads_q * ns * (d->head_dim + 2) * 4;
    TH_CHECK_ARG(d->workspace && d->workspace_bytes >= need, "th_attention_decode: workspace %lld < %lld bytes",
                 (long long)d->workspace_bytes, (long long)need);
  }
  if (!device_ready()) {
    set_error("th_attention_decode: th_init was not called for the current device");
    return TH_ERR_NOT_INIT;
  }
  DecK k{};
  k.q = (const uint16_t*)d->q; k.ldq = d->ld_q;
  k.k = (const uint16_t*)d->k_cache; k.ksb = d->k_stride_b; k.kst = d->k_stride_t;
  k.v = (const uint16_t*)d->v_cache; k.vsb = d->v_stride_b; k.vst = d->v_stride_t;
  k.o = (uint16_t*)d->o; k.ldo = d->ld_o;
  k.lengths = d->lengths; k.fixed_len = d->fixed_len;
  k.B = d->batch; k.Hq = d->heads_q; k.Hkv = d->heads_kv; k.G = d->heads_q / d->heads_kv; k.nsplit = ns;
  k.scale_log2 = d->scale * 1.4426950408889634f;
  k.part = d->workspace;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(ns, d->heads_kv, d->batch);
  if (d->head_dim == 128)
    hipLaunchKernelGGL(attn_decode_kernel<128>, grid, dim3(256), 0, s, k);
  else
    hipLaunchKernelGGL(attn_decode_kernel<64>, grid, dim3(256), 0, s, k);
  TH_CHECK_LAUNCH();
  if (ns > 1) {
    const dim3 g2(d->heads_q, d->batch);
    if (d->head_dim == 128)
      hipLaunchKernelGGL(attn_decode_merge_kernel<128>, g2, dim3(128), 0, s, k);
    else
      hipLaunchKernelGGL(attn_decode_merge_kernel<64>, g2, dim3(64), 0, s, k);
    TH_CHECK_LAUNCH();
  }
  return TH_OK;
}
