// Decode-step attention over a KV cache (no counterpart kernel in the
// reference, which has no decode path; the math is softmax(q k^T * scale) v of
// optimizer/evaluate.py:139-146 for one query row per sequence, grouped KV
// heads as in the prefill kernel).
//
// One workgroup per (KV split, kv head, sequence) serves all G = Hq/Hkv query
// heads that share the kv head (G <= 16), so each cached K/V byte is read from
// HBM once. Each of the four waves walks its own 32-key tiles of the split:
//   loads         K and V rows are read with D/8 lanes per row (whole rows per
//                 instruction), into registers one tile ahead of the tile
//                 being computed;
//   staging       the wave writes the landed tile into its own LDS slice,
//                 row-major with 16-byte chunks permuted per row, so no block
//                 barrier is needed in the loop;
//   S^T = K Q^T   v_mfma_f32_16x16x32_bf16 per 16-key block: K operands by
//                 ds_read_b128, Q^T in registers (columns >= G are zero), so
//                 lane l owns query column l % 16 and keys 4 (l / 16) .. +3
//                 of each block;
//   O^T += V^T P^T  v_mfma_f32_16x16x32_bf16 per 16 dims over the tile's 32
//                 keys: P^T is the two blocks' S^T accumulators as they are,
//                 V^T operands come from ds_read_b64_tr_b16 on the row-major V
//                 tile, in the same key order.
// The four waves' partial (max, sum, o) are merged in LDS; with more than one
// split, a second kernel merges the splits.
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
  int max_len;  // per-sequence lengths are clamped to 1..max_len (the cache slab)
  int B, Hq, Hkv, G, nsplit;
  float scale_log2;
  float* part;  // [B][Hq][nsplit][D + 2]: m, l, o[D] (o unnormalised)
};

typedef unsigned dec_u32x4 __attribute__((ext_vector_type(4)));
typedef short dec_s16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void wave_lds_order() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// LDS tile layout (one wave's slice: K tile, then V tile; 32 rows of 2 D bytes,
// 16-byte chunk c of row r in slot c ^ sw(r)):
//   K: ksw(r) = r % 16 (D = 128), (r / 2) % 8 (D = 64): an S^T operand read
//      (16 rows, one chunk per lane in each 16-lane group) hits distinct banks;
//   V: vsw(r) = 2 (r % 8) (D = 128), 2 ((r / 2) % 4) (D = 64): a transposing
//      read (16 rows, 32 bytes each) hits every bank twice.
// ds_read_b64_tr_b16, in each 16-lane group: output lane i, element e = the
// element i % 4 of the 8 bytes at source lane 4 e + i / 4's address. Source
// lane 4 e + j points at V row kb + e, columns d0 + 4 j .. +3, so output lane i
// holds keys kb .. kb+3 of column d0 + i.
template <int D>
__device__ __forceinline__ int dec_ksw(int r) { return D == 128 ? (r & 15) : ((r >> 1) & 7); }
template <int D>
__device__ __forceinline__ int dec_vsw(int r) { return D == 128 ? 2 * (r & 7) : 2 * ((r >> 1) & 3); }

template <int D>
__global__ void __launch_bounds__(256, 2) attn_decode_kernel(DecK p) {
  constexpr int NKS = D / 32;      // k steps of S^T = K Q^T per 16-key block
  constexpr int NDB = D / 16;      // 16-dim blocks of O^T
  constexpr int RB = D * 2;        // bytes per cached row (one token, one kv head)
  constexpr int KCH = D / 8;       // 16-byte chunks per row
  constexpr int RPI = 64 / KCH;    // rows per wave load instruction
  constexpr int NL = 32 / RPI;     // load instructions per tile per tensor
  constexpr int TB = 32 * RB;      // one tensor's tile
  constexpr int SLICE = 2 * TB;    // K tile then V tile
  constexpr int GMAX = 16;
  constexpr int OW_BYTES = 4 * GMAX * D * 4;
  constexpr int SMEM = 4 * SLICE > OW_BYTES ? 4 * SLICE : OW_BYTES;
  // periods (in load index i) of the K / V chunk permutations of row RPI i + lr
  constexpr int NKX = D == 128 ? 4 : 2;
  constexpr int NVX = D == 128 ? 2 : 1;
  __shared__ __attribute__((aligned(16))) char smem[SMEM];
  __shared__ float mw[4][GMAX], lw[4][GMAX];

  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qc = lane & 15, g = lane >> 4;  // query column, lane group
  const int G = p.G;
  const int len = p.lengths ? min(max(p.lengths[b], 1), p.max_len) : p.fixed_len;
  const int per = (len + p.nsplit - 1) / p.nsplit;
  const int s0 = split * per, s1 = min(len, s0 + per);

  // Q^T operands: column qc = query head kvh*G + qc (zero for qc >= G); k step
  // ks, lane group g holds dims 32 ks + 8 g .. +7
  bf16x8_t qf[NKS];
  const uint16_t* qrow = p.q + (int64_t)b * p.ldq + (int64_t)(kvh * G + qc) * D;
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    if (qc < G) {
      qf[ks] = *(const bf16x8_t*)(qrow + 32 * ks + 8 * g);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[ks][e] = (__bf16)0.f;
    }
  }

  const char* kbase = (const char*)(p.k + (int64_t)b * p.ksb + (int64_t)kvh * D);
  const char* vbase = (const char*)(p.v + (int64_t)b * p.vsb + (int64_t)kvh * D);
  char* sk = smem + wave * SLICE;
  char* sv = sk + TB;

  // This lane's share of a tile: rows RPI i + lr (i < NL), LDS slot lc. The
  // chunk permutation is applied on the load side (slot lc of row r holds
  // chunk lc ^ sw(r)), so the LDS writes are linear: 16-byte lane units at
  // i KB. Row offsets are 32-bit (strides under 2^24 elements).
  const int lr = lane / KCH, lc = lane % KCH;
  uint32_t kx[NKX], vx[NVX];
#pragma unroll
  for (int m = 0; m < NKX; ++m)
    kx[m] = (uint32_t)lr * (uint32_t)p.kst * 2u + (uint32_t)((lc ^ dec_ksw<D>(RPI * m + lr)) << 4);
#pragma unroll
  for (int m = 0; m < NVX; ++m)
    vx[m] = (uint32_t)lr * (uint32_t)p.vst * 2u + (uint32_t)((lc ^ dec_vsw<D>(RPI * m + lr)) << 4);
  const int64_t kstep = (int64_t)RPI * p.kst * 2, vstep = (int64_t)RPI * p.vst * 2;
  char* wk = sk + lane * 16;
  char* wv = sv + lane * 16;
  dec_u32x4 kr[NL], vr[NL];
  auto load = [&](int t) {
    const char* kt = kbase + (int64_t)t * p.kst * 2;
    const char* vt = vbase + (int64_t)t * p.vst * 2;
    if (t + 32 <= s1) {
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        kr[i] = *(const dec_u32x4*)(kt + i * kstep + kx[i % NKX]);
        vr[i] = *(const dec_u32x4*)(vt + i * vstep + vx[i % NVX]);
      }
    } else {
      // ragged last tile: rows past the split's end re-read its last row (in
      // bounds; their scores are masked to -inf, so P = 0)
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        const int r = RPI * i + lr;
        const int64_t row = min(t + r, s1 - 1);
        kr[i] = *(const dec_u32x4*)(kbase + row * p.kst * 2 + ((lc ^ dec_ksw<D>(r)) << 4));
        vr[i] = *(const dec_u32x4*)(vbase + row * p.vst * 2 + ((lc ^ dec_vsw<D>(r)) << 4));
      }
    }
  };

  // S^T operand reads: row 16 blk + qc, chunk 4 ks + g
  const char* rk = sk + qc * RB;
  // V^T operand reads: this lane is source lane 4 e + j of group g, reading
  // row 4 g + e (16 + 4 g + e for the second block), columns 16 db + 4 j .. +3
  const int e4 = (lane & 15) >> 2, j4 = lane & 3;
  const int vr0 = 4 * g + e4;
  const int vxo = dec_vsw<D>(vr0) >> 1;  // slot of chunk 2 db + j4/2 is 2 (db ^ vxo) + j4/2
  const char* rv = sv + vr0 * RB + (j4 >> 1) * 16 + (j4 & 1) * 8;

  f32x4_t oacc[NDB];
#pragma unroll
  for (int t = 0; t < NDB; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) oacc[t][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  int t0 = s0 + 32 * wave;
  if (t0 < s1) load(t0);
  for (; t0 < s1; t0 += 128) {
    // the slice is free (this wave's reads of the previous tile were issued
    // before these writes, and one wave's LDS operations complete in order)
    wave_lds_order();
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      *(dec_u32x4*)(wk + i * 1024) = kr[i];
      *(dec_u32x4*)(wv + i * 1024) = vr[i];
    }
    if (t0 + 128 < s1) load(t0 + 128);
    wave_lds_order();

    f32x4_t s[2];
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
      for (int r = 0; r < 4; ++r) s[blk][r] = 0.f;
      const int row = 16 * blk + qc;
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const bf16x8_t kf = *(const bf16x8_t*)(rk + 16 * blk * RB + (((4 * ks + g) ^ dec_ksw<D>(row)) << 4));
        s[blk] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[ks], s[blk], 0, 0, 0);
      }
    }
    // online softmax per query column: this lane holds 8 of the tile's 32 keys
    // (4 g + r and 16 + 4 g + r); the other 24 are in lanes qc + 16, 32, 48
    float mloc = -INFINITY;
    if (t0 + 32 <= s1) {
#pragma unroll
      for (int blk = 0; blk < 2; ++blk)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          s[blk][r] *= p.scale_log2;
          mloc = fmaxf(mloc, s[blk][r]);
        }
    } else {
#pragma unroll
      for (int blk = 0; blk < 2; ++blk)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int kk = t0 + 16 * blk + 4 * g + r;
          s[blk][r] = kk < s1 ? s[blk][r] * p.scale_log2 : -INFINITY;
          mloc = fmaxf(mloc, s[blk][r]);
        }
    }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
    const float m_new = fmaxf(m_run, mloc);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    m_run = m_new;
    float lsum = 0.f;
    bf16x8_t pf;
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float e = __builtin_amdgcn_exp2f(s[blk][r] - m_use);
        lsum += e;
        pf[4 * blk + r] = (__bf16)e;
      }
    l_run = l_run * alpha + lsum;
#pragma unroll
    for (int t = 0; t < NDB; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) oacc[t][r] *= alpha;
    // O^T += V^T P^T: k elements 0..3 = keys 4 g + 0..3, 4..7 = keys 16 + 4 g + 0..3
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int cofs = ((db ^ vxo) << 5);
      const dec_s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) dec_s16x4*)(rv + cofs));
      const dec_s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) dec_s16x4*)(rv + 16 * RB + cofs));
      const bf16x8_t vf = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      oacc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf, oacc[db], 0, 0, 0);
    }
  }

  // merge the four waves (the partial o rows reuse the tile slices)
  __syncthreads();
  float(*ow)[GMAX][D] = (float(*)[GMAX][D])smem;
  float l_tot = l_run + __shfl_xor(l_run, 16);
  l_tot += __shfl_xor(l_tot, 32);
  if (qc < G) {
    if (g == 0) {
      mw[wave][qc] = m_run;
      lw[wave][qc] = l_tot;
    }
#pragma unroll
    for (int db = 0; db < NDB; ++db)
      *(f32x4_t*)&ow[wave][qc][16 * db + 4 * g] = oacc[db];
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
  // one resident round (two workgroups per CU), each split at least 256 keys;
  // at the Llama-3-8B decode shape (batch 64, 8 kv heads, 4096 keys) one split
  // measured 186 us against 196-200 us for 2-16 splits
  const int cus = device_cus() > 0 ? device_cus() : 256;
  int s = (int)cdiv(2 * cus, (int64_t)batch * heads_kv);
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
  TH_CHECK_ARG(d->k_stride_t < (1 << 24) && d->v_stride_t < (1 << 24),
               "th_attention_decode: cache token strides must be under 2^24 elements");
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
  k.lengths = d->lengths; k.fixed_len = d->fixed_len; k.max_len = d->max_len;
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
