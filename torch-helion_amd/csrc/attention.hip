// OpIR `attention` kind: softmax(q k^T * scale) v per (batch, head) over
// token-major [B*S, H*d] tensors (reference semantics: optimizer/evaluate.py:139-146;
// Helion template it replaces: codegen/emit.py:327-357), extended with a
// causal flag and grouped KV heads.
//
// bf16 prefill kernel (gfx950): one workgroup = 4 waves = 128 queries of one
// (batch, q-head); kv tiles of 64 keys are staged through LDS, double
// buffered. Each wave computes S^T = K Q^T with v_mfma_f32_32x32x16_bf16 so a
// lane owns one query column: the online-softmax max/sum needs a single
// lane^32 exchange and P^T is already in the B-operand layout of the P V
// product O^T = V^T P^T (the kv order inside one 16-wide k step is permuted,
// identically for V^T, which is harmless for a contraction). V is written to
// LDS transposed (kv contiguous) with an XOR swizzle that keeps the two
// 8-byte reads per MFMA operand conflict-free. Causal workgroups are issued
// longest-first; a wave skips kv tiles entirely above its diagonal.
#include "common.h"

namespace th {

struct AttnK {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  int64_t ldq, ldk, ldv, ldo;
  int B, Sq, Skv, Hq, Hkv, group, nqb, causal, off;
  float scale_log2;
};

template <int D>
__global__ void __launch_bounds__(256, 2) attn_fwd_bf16_kernel(AttnK p) {
  constexpr int BQ = 128, BKV = 64;
  constexpr int KCH = D / 8;             // 16-byte chunks per K row
  constexpr int KROW = D * 2;            // bytes per K row in LDS
  constexpr int VROW = BKV * 2;          // bytes per V^T row (one d) in LDS
  constexpr int KT_BYTES = BKV * KROW;
  constexpr int VT_BYTES = D * VROW;
  constexpr int STAGE = KT_BYTES + VT_BYTES;
  constexpr int OROW = D + 4;            // fp32 staging row for the output
  constexpr int O_BYTES = 4 * 32 * OROW * 4;
  constexpr int SMEM = 2 * STAGE > O_BYTES ? 2 * STAGE : O_BYTES;
  constexpr int KLD = BKV * KCH / 256;   // K chunks per thread per tile
  constexpr int VPAIRS = KCH / 8;        // V row pairs per thread per tile
  constexpr int NKS = D / 16;            // k steps of S^T = K Q^T
  constexpr int NDT = D / 32;            // 32-row blocks of O^T
  __shared__ __attribute__((aligned(16))) char smem[SMEM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, col = lane & 31;
  const int bh_count = p.B * p.Hq;
  const int qb = p.nqb - 1 - (int)(blockIdx.x / bh_count);
  const int bh = (int)(blockIdx.x % bh_count);
  const int b = bh / p.Hq, hq = bh - b * p.Hq, hk = hq / p.group;
  const int q0 = qb * BQ;
  const int q0w = q0 + wave * 32;
  const int qrow = q0w + col;

  const uint16_t* qbase = p.q + (int64_t)b * p.Sq * p.ldq + (int64_t)hq * D;
  const uint16_t* kbase = p.k + (int64_t)b * p.Skv * p.ldk + (int64_t)hk * D;
  const uint16_t* vbase = p.v + (int64_t)b * p.Skv * p.ldv + (int64_t)hk * D;

  bf16x8_t qf[NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    const int d = 16 * ks + 8 * hl;
    if (qrow < p.Sq) {
      qf[ks] = *(const bf16x8_t*)(qbase + (int64_t)qrow * p.ldq + d);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[ks][e] = (__bf16)0.f;
    }
  }

  int last_kv = p.Skv - 1;
  if (p.causal) last_kv = min(last_kv, q0 + BQ - 1 + p.off);
  const int ntiles = last_kv < 0 ? 0 : last_kv / BKV + 1;

  uint4 rk[KLD], rv[VPAIRS][2];
  auto gload = [&](int it) {
    const int k0 = it * BKV;
#pragma unroll
    for (int i = 0; i < KLD; ++i) {
      const int c = tid + 256 * i;
      const int row = c / KCH, ch = c - row * KCH;
      const int kv = k0 + row;
      rk[i] = kv < p.Skv ? *(const uint4*)(kbase + (int64_t)kv * p.ldk + ch * 8) : make_uint4(0, 0, 0, 0);
    }
    const int dc = tid % KCH;
#pragma unroll
    for (int i = 0; i < VPAIRS; ++i) {
      const int pr = tid / KCH + (256 / KCH) * i;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int kv = k0 + 2 * pr + e;
        rv[i][e] = kv < p.Skv ? *(const uint4*)(vbase + (int64_t)kv * p.ldv + dc * 8) : make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto sstore = [&](int buf) {
    char* sk = smem + buf * STAGE;
    char* sv = sk + KT_BYTES;
#pragma unroll
    for (int i = 0; i < KLD; ++i) {
      const int c = tid + 256 * i;
      const int row = c / KCH, ch = c - row * KCH;
      *(uint4*)(sk + row * KROW + ((ch ^ (row % KCH)) << 4)) = rk[i];
    }
    const int dc = tid % KCH;
#pragma unroll
    for (int i = 0; i < VPAIRS; ++i) {
      const int pr = tid / KCH + (256 / KCH) * i;
      const uint32_t a[4] = {rv[i][0].x, rv[i][0].y, rv[i][0].z, rv[i][0].w};
      const uint32_t c2[4] = {rv[i][1].x, rv[i][1].y, rv[i][1].z, rv[i][1].w};
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int d = dc * 8 + q;
        const uint32_t lo = (q & 1) ? (a[q >> 1] >> 16) : (a[q >> 1] & 0xffffu);
        const uint32_t hi = (q & 1) ? (c2[q >> 1] >> 16) : (c2[q >> 1] & 0xffffu);
        const int sw = ((d >> 1) & 15) << 1;
        *(uint32_t*)(sv + d * VROW + ((pr ^ sw) << 2)) = lo | (hi << 16);
      }
    }
  };

  f32x16_t oacc[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[t][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  if (ntiles > 0) {
    gload(0);
    sstore(0);
  }
  __syncthreads();
  for (int it = 0; it < ntiles; ++it) {
    const int cur = it & 1;
    if (it + 1 < ntiles) gload(it + 1);
    const int k0 = it * BKV;
    const bool active = !p.causal || k0 <= q0w + 31 + p.off;
    if (active) {
      const char* sk = smem + cur * STAGE;
      const char* sv = sk + KT_BYTES;
      f32x16_t s[2];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[t][r] = 0.f;
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int row = 32 * t + col;
          const int ch = 2 * ks + hl;
          const bf16x8_t kf = *(const bf16x8_t*)(sk + row * KROW + ((ch ^ (row % KCH)) << 4));
          s[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[ks], s[t], 0, 0, 0);
        }
      }
      // Online softmax per query column on raw scores; c = scale * log2(e) > 0 is
      // folded into the exponent, exp2(s c - m). The running max m moves only when
      // a tile's max exceeds it by more than 8 (log2 units): probabilities stay
      // below 2^8 and the O rescale is skipped while no lane of the wave moves.
      const float c = p.scale_log2;
      const bool need_mask = (k0 + BKV > p.Skv) || (p.causal && k0 + BKV - 1 > q0w + p.off);
      float mloc = -INFINITY;
      if (need_mask) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int kv = k0 + 32 * t + 8 * (r >> 2) + 4 * hl + (r & 3);
            if (kv >= p.Skv || (p.causal && kv > qrow + p.off)) s[t][r] = -INFINITY;
            mloc = fmaxf(mloc, s[t][r]);
          }
      } else {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) mloc = fmaxf(mloc, s[t][r]);
      }
      mloc = fmaxf(mloc, __shfl_xor(mloc, 32)) * c;
      const bool move = mloc > m_run + 8.f;
      float alpha = 1.f;
      if (move) {
        alpha = __builtin_amdgcn_exp2f(m_run - mloc);
        m_run = mloc;
      }
      const float nm = m_run == -INFINITY ? 0.f : -m_run;
      float lsum = 0.f;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float e = __builtin_amdgcn_exp2f(fmaf(s[t][r], c, nm));
          s[t][r] = e;
          lsum += e;
        }
      l_run = l_run * alpha + lsum;
      if (__any(move)) {
#pragma unroll
        for (int t = 0; t < NDT; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[t][r] *= alpha;
      }
      // O^T += V^T P^T over 4 k steps of 16 keys
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int t = ks >> 1, hh = ks & 1;
        bf16x8_t pf;
#pragma unroll
        for (int e = 0; e < 8; ++e) pf[e] = (__bf16)s[t][8 * hh + e];
        const int w0 = 16 * t + 8 * hh + 2 * hl;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          const int d = 32 * dt + col;
          const int sw = ((d >> 1) & 15) << 1;
          const char* vrow = sv + d * VROW;
          const uint2 lo = *(const uint2*)(vrow + ((w0 ^ sw) << 2));
          const uint2 hi = *(const uint2*)(vrow + (((w0 + 4) ^ sw) << 2));
          bf16x8_t vf;
          uint32_t* vw = (uint32_t*)&vf;
          vw[0] = lo.x; vw[1] = lo.y; vw[2] = hi.x; vw[3] = hi.y;
          oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, oacc[dt], 0, 0, 0);
        }
      }
    }
    if (it + 1 < ntiles) sstore(cur ^ 1);
    __syncthreads();
  }

  // normalise and write through LDS so rows are stored contiguously
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  float* ostage = (float*)smem + wave * 32 * OROW;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = 32 * dt + 8 * (r >> 2) + 4 * hl + (r & 3);
      ostage[col * OROW + d] = oacc[dt][r] * inv;
    }
  __syncthreads();
  uint16_t* obase = p.o + (int64_t)b * p.Sq * p.ldo + (int64_t)hq * D;
  constexpr int C4 = D / 4;
  for (int u = lane; u < 32 * C4; u += 64) {
    const int r = u / C4, c4 = (u - r * C4) * 4;
    const int qr = q0w + r;
    if (qr >= p.Sq) continue;
    const float4 x = *(const float4*)(ostage + r * OROW + c4);
    uint2 w;
    w.x = (uint32_t)f32_to_bf16(x.x) | ((uint32_t)f32_to_bf16(x.y) << 16);
    w.y = (uint32_t)f32_to_bf16(x.z) | ((uint32_t)f32_to_bf16(x.w) << 16);
    *(uint2*)(obase + (int64_t)qr * p.ldo + c4) = w;
  }
}

// fp32 attention: one thread per query row, online softmax over all keys.
// Used for fp32 programs (the small fp32 configurations are latency bound).
struct AttnF32K {
  const float* q;
  const float* k;
  const float* v;
  float* o;
  int64_t ldq, ldk, ldv, ldo;
  int B, Sq, Skv, Hq, Hkv, group, D, causal, off;
  float scale;
};

template <int D>
__global__ void __launch_bounds__(64) attn_fwd_f32_kernel(AttnF32K p) {
  const int bh = blockIdx.y;
  const int b = bh / p.Hq, hq = bh - b * p.Hq, hk = hq / p.group;
  const int qi = blockIdx.x * 64 + threadIdx.x;
  if (qi >= p.Sq) return;
  const float* qr = p.q + ((int64_t)b * p.Sq + qi) * p.ldq + (int64_t)hq * D;
  float qv[D], acc[D];
#pragma unroll
  for (int d = 0; d < D; ++d) { qv[d] = qr[d]; acc[d] = 0.f; }
  float m = -INFINITY, l = 0.f;
  int last = p.Skv - 1;
  if (p.causal) last = min(last, qi + p.off);
  for (int j = 0; j <= last; ++j) {
    const float* kr = p.k + ((int64_t)b * p.Skv + j) * p.ldk + (int64_t)hk * D;
    float s = 0.f;
#pragma unroll
    for (int d = 0; d < D; ++d) s += qv[d] * kr[d];
    s *= p.scale;
    const float mn = fmaxf(m, s);
    const float alpha = __expf(m - mn);
    const float e = __expf(s - mn);
    m = mn;
    l = l * alpha + e;
    const float* vr = p.v + ((int64_t)b * p.Skv + j) * p.ldv + (int64_t)hk * D;
#pragma unroll
    for (int d = 0; d < D; ++d) acc[d] = acc[d] * alpha + e * vr[d];
  }
  float* orow = p.o + ((int64_t)b * p.Sq + qi) * p.ldo + (int64_t)hq * D;
  const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
  for (int d = 0; d < D; ++d) orow[d] = acc[d] * inv;
}

}  // namespace th

using namespace th;

extern "C" int th_attention_prefill(const th_attn_desc* d, void* stream) {
  TH_CHECK_ARG(d != nullptr, "th_attention_prefill: null descriptor");
  TH_CHECK_ARG(d->batch > 0 && d->seq_q > 0 && d->seq_kv > 0 && d->heads_q > 0 && d->heads_kv > 0,
               "th_attention_prefill: sizes must be positive");
  TH_CHECK_ARG(d->heads_q % d->heads_kv == 0, "th_attention_prefill: heads_q=%d not a multiple of heads_kv=%d",
               d->heads_q, d->heads_kv);
  TH_CHECK_ARG(d->q && d->k && d->v && d->o, "th_attention_prefill: null tensor pointer");
  TH_CHECK_ARG(d->dtype == TH_BF16 || d->dtype == TH_F32, "th_attention_prefill: dtype %d unsupported", d->dtype);
  const int hd = d->head_dim;
  TH_CHECK_ARG(hd == 64 || hd == 128 || (d->dtype == TH_F32 && (hd == 32 || hd == 16)),
               "th_attention_prefill: head_dim %d unsupported", hd);
  TH_CHECK_ARG(d->ld_q >= (int64_t)d->heads_q * hd && d->ld_o >= (int64_t)d->heads_q * hd &&
                   d->ld_k >= (int64_t)d->heads_kv * hd && d->ld_v >= (int64_t)d->heads_kv * hd,
               "th_attention_prefill: row strides smaller than heads*head_dim");
  if (d->dtype == TH_BF16) {
    TH_CHECK_ARG(d->ld_q % 8 == 0 && d->ld_k % 8 == 0 && d->ld_v % 8 == 0 && d->ld_o % 4 == 0,
                 "th_attention_prefill: bf16 row strides must be multiples of 8 elements");
    TH_CHECK_ARG(((uintptr_t)d->q | (uintptr_t)d->k | (uintptr_t)d->v) % 16 == 0 && (uintptr_t)d->o % 8 == 0,
                 "th_attention_prefill: tensors must be 16-byte aligned");
  }
  TH_CHECK_ARG(d->dtype != TH_BF16 || d->scale > 0.f, "th_attention_prefill: bf16 kernel needs scale > 0 (got %g)",
               (double)d->scale);
  if (!device_ready()) {
    set_error("th_attention_prefill: th_init was not called for the current device");
    return TH_ERR_NOT_INIT;
  }
  hipStream_t s = (hipStream_t)stream;
  const float log2e = 1.4426950408889634f;
  if (d->dtype == TH_BF16) {
    AttnK k{};
    k.q = (const uint16_t*)d->q;
    k.k = (const uint16_t*)d->k;
    k.v = (const uint16_t*)d->v;
    k.o = (uint16_t*)d->o;
    k.ldq = d->ld_q; k.ldk = d->ld_k; k.ldv = d->ld_v; k.ldo = d->ld_o;
    k.B = d->batch; k.Sq = d->seq_q; k.Skv = d->seq_kv; k.Hq = d->heads_q; k.Hkv = d->heads_kv;
    k.group = d->heads_q / d->heads_kv;
    k.nqb = (int)cdiv(d->seq_q, 128);
    k.causal = d->causal ? 1 : 0;
    k.off = d->seq_kv - d->seq_q;
    k.scale_log2 = d->scale * log2e;
    const dim3 grid((unsigned)(k.nqb * d->batch * d->heads_q));
    if (hd == 128)
      hipLaunchKernelGGL(attn_fwd_bf16_kernel<128>, grid, dim3(256), 0, s, k);
    else
      hipLaunchKernelGGL(attn_fwd_bf16_kernel<64>, grid, dim3(256), 0, s, k);
  } else {
    AttnF32K k{};
    k.q = (const float*)d->q; k.k = (const float*)d->k; k.v = (const float*)d->v; k.o = (float*)d->o;
    k.ldq = d->ld_q; k.ldk = d->ld_k; k.ldv = d->ld_v; k.ldo = d->ld_o;
    k.B = d->batch; k.Sq = d->seq_q; k.Skv = d->seq_kv; k.Hq = d->heads_q; k.Hkv = d->heads_kv;
    k.group = d->heads_q / d->heads_kv; k.D = hd; k.causal = d->causal ? 1 : 0; k.off = d->seq_kv - d->seq_q;
    k.scale = d->scale;
    const dim3 grid((unsigned)cdiv(d->seq_q, 64), (unsigned)(d->batch * d->heads_q));
    switch (hd) {
      case 16: hipLaunchKernelGGL(attn_fwd_f32_kernel<16>, grid, dim3(64), 0, s, k); break;
      case 32: hipLaunchKernelGGL(attn_fwd_f32_kernel<32>, grid, dim3(64), 0, s, k); break;
      case 64: hipLaunchKernelGGL(attn_fwd_f32_kernel<64>, grid, dim3(64), 0, s, k); break;
      default: hipLaunchKernelGGL(attn_fwd_f32_kernel<128>, grid, dim3(64), 0, s, k); break;
    }
  }
  TH_CHECK_LAUNCH();
  return TH_OK;
}
