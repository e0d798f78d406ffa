// OpIR `attention` kind: softmax(q k^T * scale) v per (batch, head) over
// token-major [B*S, H*d] tensors (reference semantics: optimizer/evaluate.py:139-146;
// Helion template it replaces: codegen/emit.py:327-357), extended with a
// causal flag and grouped KV heads.
//
// bf16 prefill kernel (gfx950): one workgroup = 4 waves = 128 queries of one
// (batch, q-head); kv tiles of 64 keys stream into LDS by direct loads,
// double buffered. Each wave computes S^T = K Q^T with v_mfma_f32_32x32x16_bf16
// so a lane owns one query column: the online-softmax max/sum needs a single
// lane^32 exchange and P^T is already in the B-operand layout of the P V
// product O^T = V^T P^T (the kv order inside one 16-wide k step is permuted,
// identically for V^T, which is harmless for a contraction). V stays
// row-major in LDS; its transposed operands come from ds_read_b64_tr_b16.
// Causal workgroups are issued longest-first; a wave skips kv tiles entirely
// above its diagonal.
#include "common.h"

namespace th {

struct AttnK {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  int64_t ldq, ldk, ldv, ldo;
  int B, Sq, Skv, Hq, Hkv, group, nqb, causal, off;
  int xcd_map;  // (B * Hkv) % 8 == 0: every (batch, kv head) served by one XCD
  float scale_log2;
};

typedef short s16x4_t __attribute__((ext_vector_type(4)));

// K and V tiles stream from HBM straight into LDS (global_load_lds_dwordx4,
// 1 KB per wave instruction: 1024 / (2 D) rows), row-major with each row's
// 16-byte chunks permuted:
//   K row R: chunk c in slot c ^ (R % (D/8)): the 32-row reads of an S^T
//            operand (one chunk per lane) hit distinct banks.
//   V row R: chunk c in slot c ^ vsw(R), vsw(R) = 4 (R % 4) for D = 128 and
//            4 ((R / 2) % 2) for D = 64.
// V^T operands come from ds_read_b64_tr_b16: in each 16-lane group, output
// lane i, element e = the element i % 4 of the 8 bytes at source lane
// 4 e + i / 4's address. Source lane 4 e + j points at V row kb + e, columns
// d0 + 4 j .. +3, so output lane i holds keys kb .. kb+3 of column d0 + i; the
// swizzle puts the 4 rows of a group (and the two groups sharing them) on
// distinct banks. Rows past the last key re-read the last key: in bounds, and
// their scores are masked to -inf (P = 0).
template <int D>
__global__ void __launch_bounds__(256, 2) attn_fwd_bf16_kernel(AttnK p) {
  constexpr int BQ = 128, BKV = 64;
  constexpr int RB = D * 2;               // bytes per K or V row
  constexpr int KCH = D / 8;              // 16-byte chunks per row
  constexpr int RPI = 1024 / RB;          // rows per 1 KB load
  constexpr int NLOAD = BKV / RPI / 4;    // loads per wave per tile, per tensor
  constexpr int KT_BYTES = BKV * RB;
  constexpr int STAGE = 2 * KT_BYTES;     // K tile then V tile
  constexpr int OROW = D + 4;             // fp32 staging row for the output
  constexpr int O_BYTES = 4 * 32 * OROW * 4;
  constexpr int SMEM = 2 * STAGE > O_BYTES ? 2 * STAGE : O_BYTES;
  constexpr int NKS = D / 16;             // k steps of S^T = K Q^T
  constexpr int NDT = D / 32;             // 32-row blocks of O^T
  static_assert(NLOAD * RPI * 4 == BKV, "tile rows per wave");
  __shared__ __attribute__((aligned(16))) char smem[SMEM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hl = lane >> 5, col = lane & 31;
  const int bh_count = p.B * p.Hq;
  // Workgroups are dealt round-robin to the 8 XCDs (workgroup i to XCD i % 8),
  // each with its own L2. With xcd_map, XCD x owns (B Hkv / 8) whole (batch, kv
  // head) pairs, so the q heads of a GQA group and all q blocks that read one
  // K/V stream share one L2; within an XCD the q blocks still run longest first.
  int qb, b, hq;
  if (p.xcd_map) {
    const int xcd = (int)(blockIdx.x & 7), slot = (int)(blockIdx.x >> 3);
    const int per_qb = bh_count >> 3;  // one q block's workgroups per XCD
    const int qi = slot / per_qb, inner = slot - qi * per_qb;
    const int pl = inner / p.group;
    const int pair = xcd * ((p.B * p.Hkv) >> 3) + pl;
    b = pair / p.Hkv;
    hq = (pair - b * p.Hkv) * p.group + (inner - pl * p.group);
    qb = p.nqb - 1 - qi;
  } else {
    const int bh = (int)(blockIdx.x % bh_count);
    qb = p.nqb - 1 - (int)(blockIdx.x / bh_count);
    b = bh / p.Hq;
    hq = bh - b * p.Hq;
  }
  const int hk = hq / p.group;
  const int q0 = qb * BQ;
  const int q0w = q0 + wave * 32;
  const int qrow = q0w + col;

  const uint16_t* qbase = p.q + (int64_t)b * p.Sq * p.ldq + (int64_t)hq * D;
  const char* kbase = (const char*)(p.k + (int64_t)b * p.Skv * p.ldk + (int64_t)hk * D);
  const char* vbase = (const char*)(p.v + (int64_t)b * p.Skv * p.ldv + (int64_t)hk * D);

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

  // this lane's place in the tile loads: load n = NLOAD*wave + i covers rows RPI*n ..
  // Per-lane byte offsets of those rows within a tile (32-bit: 63 rows of a row
  // stride under 32 MiB) plus the chunk swizzle; a full tile adds them to a
  // uniform base, the ragged last tile clamps its rows to the last key.
  const int lrow = lane / KCH, slot = lane % KCH;
  auto vsw = [](int r) { return D == 128 ? 4 * (r & 3) : 4 * ((r >> 1) & 1); };
  uint32_t kro[NLOAD], vro[NLOAD];
#pragma unroll
  for (int i = 0; i < NLOAD; ++i) {
    const int row = RPI * (NLOAD * wave + i) + lrow;
    kro[i] = (uint32_t)row * (uint32_t)p.ldk * 2u + (uint32_t)((slot ^ (row % KCH)) << 4);
    vro[i] = (uint32_t)row * (uint32_t)p.ldv * 2u + (uint32_t)((slot ^ vsw(row)) << 4);
  }
  // (dma_load16: the compiler does not count these loads among the LDS
  // operations its read waits cover; the full wait at the top of every tile
  // covers them)
  const uint32_t lds0 = (uint32_t)(uintptr_t)smem;
  auto issue = [&](int it, int st) {
    const int k0 = it * BKV;
    const uint32_t sk = lds0 + st * STAGE;
    const char* kb = kbase + (int64_t)k0 * p.ldk * 2;
    const char* vb = vbase + (int64_t)k0 * p.ldv * 2;
    if (k0 + BKV <= p.Skv) {
#pragma unroll
      for (int i = 0; i < NLOAD; ++i) {
        const int n = NLOAD * wave + i;
        dma_load16(kb, kro[i], sk + n * 1024);
        dma_load16(vb, vro[i], sk + KT_BYTES + n * 1024);
      }
    } else {
      // ragged last tile: rows past the last key re-read the last key
#pragma unroll
      for (int i = 0; i < NLOAD; ++i) {
        const int n = NLOAD * wave + i;
        const int row = RPI * n + lrow;
        const uint32_t r = (uint32_t)min(row, p.Skv - 1 - k0);
        dma_load16(kb, r * (uint32_t)p.ldk * 2u + (uint32_t)((slot ^ (row % KCH)) << 4), sk + n * 1024);
        dma_load16(vb, r * (uint32_t)p.ldv * 2u + (uint32_t)((slot ^ vsw(row)) << 4), sk + KT_BYTES + n * 1024);
      }
    }
  };

  // V^T operand reads: this lane is source lane 4e + j of its 16-lane group
  const int e4 = (lane & 15) >> 2, j4 = lane & 3, g2 = (lane >> 4) & 1;
  const int ee = D == 128 ? e4 : (e4 >> 1);
  const int vrow_l = (4 * hl + e4) * RB + (j4 & 1) * 8;  // row part (keys +4hl+e) and the 8-byte half
  const int vc0 = 2 * g2 + (j4 >> 1);                   // chunk within the 32-column block, before the swizzle

  f32x16_t oacc[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[t][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  if (ntiles > 0) issue(0, 0);
  for (int it = 0; it < ntiles; ++it) {
    const int cur = it & 1;
    // tile it has landed everywhere, and every wave is done with stage cur ^ 1
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (it + 1 < ntiles) issue(it + 1, cur ^ 1);
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
          const bf16x8_t kf = *(const bf16x8_t*)(sk + row * RB + ((ch ^ (row % KCH)) << 4));
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
          const float ex = __builtin_amdgcn_exp2f(fmaf(s[t][r], c, nm));
          s[t][r] = ex;
          lsum += ex;
        }
      l_run = l_run * alpha + lsum;
      if (__any(move)) {
#pragma unroll
        for (int t = 0; t < NDT; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[t][r] *= alpha;
      }
      // O^T += V^T P^T over 4 k steps of 16 keys. The lane's 8 P values are the
      // keys 16 hh + 4 hl + 0..3 and 16 hh + 8 + 4 hl + 0..3 of 32-key block t
      // (S^T's C layout); one transposing read fetches each group of 4.
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int t = ks >> 1, hh = ks & 1;
        bf16x8_t pf;
#pragma unroll
        for (int e = 0; e < 8; ++e) pf[e] = (__bf16)s[t][8 * hh + e];
        const char* vb = sv + (32 * t + 16 * hh) * RB + vrow_l;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          const int cofs = ((4 * (dt ^ ee) + vc0) << 4);
          const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) s16x4_t*)(vb + cofs));
          const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) s16x4_t*)(vb + 8 * RB + cofs));
          const bf16x8_t vf = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
          oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, oacc[dt], 0, 0, 0);
        }
      }
    }
  }
  __syncthreads();  // every wave is done with the stages before they hold the output

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
    w.x = pk_bf16x2(x.x, x.y);
    w.y = pk_bf16x2(x.z, x.w);
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
  float scale_log2;  // scale * log2(e) (matrix-core kernel)
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

// fp32 attention on the matrix cores (head_dim 64 or 128): one workgroup of KW
// waves per 32 queries of one (batch, q head); wave w takes the key blocks
// w, w + KW, ... (32 keys each) with its own online softmax, and the waves'
// partial results are merged through LDS at the end, in wave order. (One wave
// walking every block serially left C1's 8 x 4 query blocks latency-bound.)
// S^T = K Q^T and O^T += V^T P^T run on v_mfma_f32_32x32x2f32, so a lane owns
// one query column (l % 32) and the softmax statistics need one lane^32
// exchange, as in the bf16 kernel. Operands come straight from memory in the
// MFMA layouts (the fp32 configurations are small and L2-resident):
//   S^T step (chunk i, component c): lane l supplies K[key l%32][8i + 4(l/32) + c]
//     and Q[query l%32][the same d]: one float4 per chunk and lane, the
//     contraction index permuted identically on both sides;
//   O^T step (register r of S^T): lane l supplies P for key
//     8(r/4) + 4(l/32) + r%4 (its own S^T register) and V[that key][32t + l%32].
// The result goes out through LDS as whole rows.
template <int D, int KW>
__global__ void __launch_bounds__(64 * KW, 1) attn_fwd_f32_mfma_kernel(AttnF32K p) {
  constexpr int NCH = D / 8;   // float4 chunks per lane of a Q or K row
  constexpr int NDT = D / 32;  // 32-row tiles of O^T
  constexpr int OROW = D + 4;  // LDS row stride (floats) of a wave's partial output
  __shared__ __attribute__((aligned(16))) float so[KW * 32 * OROW];
  __shared__ float sm[KW * 32], sl[KW * 32];
  const int bh = blockIdx.y;
  const int b = bh / p.Hq, hq = bh - b * p.Hq, hk = hq / p.group;
  const int q0 = blockIdx.x * 32;
  const int tid = threadIdx.x, lane = tid & 63, qc = lane & 31, half = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const float* qb = p.q + (int64_t)b * p.Sq * p.ldq + (int64_t)hq * D;
  const float* kbase = p.k + (int64_t)b * p.Skv * p.ldk + (int64_t)hk * D;
  const float* vbase = p.v + (int64_t)b * p.Skv * p.ldv + (int64_t)hk * D;
  const int qrow = min(q0 + qc, p.Sq - 1);  // rows past Sq re-read the last one (never stored)
  float4 qf[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) qf[i] = *(const float4*)(qb + (int64_t)qrow * p.ldq + 8 * i + 4 * half);
  f32x16_t o[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[t][r] = 0.f;
  float m = -INFINITY, l = 0.f;
  // keys visible to the block's last query
  int kend = p.Skv;
  if (p.causal) kend = min(kend, q0 + 31 + p.off + 1);
  const int myq = q0 + qc;
  // K rows of a block (rows past Skv re-read the last key; masked below) and its
  // V operands (register r's key, columns 32t + l%32); the wave's next block's
  // are loaded while this one computes
  float4 kf[NCH], kn[NCH];
  float vf[NDT][16], vn[NDT][16];
  auto load_block = [&](int kb, float4 (&kx)[NCH], float (&vx)[NDT][16]) {
    const int krow = min(kb + qc, p.Skv - 1);
#pragma unroll
    for (int i = 0; i < NCH; ++i) kx[i] = *(const float4*)(kbase + (int64_t)krow * p.ldk + 8 * i + 4 * half);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = min(kb + 8 * (r >> 2) + 4 * half + (r & 3), p.Skv - 1);
#pragma unroll
      for (int t = 0; t < NDT; ++t) vx[t][r] = vbase[(int64_t)key * p.ldv + 32 * t + qc];
    }
  };
  const int kfirst = 32 * wave;
  if (kfirst < kend) load_block(kfirst, kn, vn);
  for (int kb = kfirst; kb < kend; kb += 32 * KW) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) kf[i] = kn[i];
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) vf[t][r] = vn[t][r];
    if (kb + 32 * KW < kend) load_block(kb + 32 * KW, kn, vn);
    f32x16_t st;
#pragma unroll
    for (int r = 0; r < 16; ++r) st[r] = 0.f;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      st = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[i].x, qf[i].x, st, 0, 0, 0);
      st = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[i].y, qf[i].y, st, 0, 0, 0);
      st = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[i].z, qf[i].z, st, 0, 0, 0);
      st = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[i].w, qf[i].w, st, 0, 0, 0);
    }
    // scores in log2 units, masked past the sequence and above the diagonal
    float mb = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = kb + 8 * (r >> 2) + 4 * half + (r & 3);
      const bool vis = key < p.Skv && (!p.causal || key <= myq + p.off);
      st[r] = vis ? st[r] * p.scale_log2 : -INFINITY;
      mb = fmaxf(mb, st[r]);
    }
    mb = fmaxf(mb, __shfl_xor(mb, 32));
    const float mn = fmaxf(m, mb);
    // (a column with no visible key yet keeps m = -inf: nothing to rescale, P = 0)
    const float alpha = mn == -INFINITY ? 1.f : exp2f(m - mn);
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      st[r] = mn == -INFINITY ? 0.f : exp2f(st[r] - mn);
      ps += st[r];
    }
    ps += __shfl_xor(ps, 32);
    l = l * alpha + ps;
    m = mn;
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) o[t][r] *= alpha;
#pragma unroll
      for (int r = 0; r < 16; ++r) o[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf[t][r], st[r], o[t], 0, 0, 0);
    }
  }
  // the wave's partial O^T (unnormalised; lane l holds column (query) l%32, rows
  // d = 32t + 8(r/4) + 4(l/32) + r%4) as rows of its LDS slab, with m and l
  float* sw = so + wave * 32 * OROW;
#pragma unroll
  for (int t = 0; t < NDT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) sw[qc * OROW + 32 * t + 8 * (r >> 2) + 4 * half + (r & 3)] = o[t][r];
  if (half == 0) {
    sm[wave * 32 + qc] = m;
    sl[wave * 32 + qc] = l;
  }
  __syncthreads();
  // merge, in wave order: O = sum_w 2^(m_w - m) O_w / sum_w 2^(m_w - m) l_w, m = max_w m_w;
  // each thread writes float4s of whole rows
  constexpr int F4 = D / 4;
  float* ob = p.o + (int64_t)b * p.Sq * p.ldo + (int64_t)hq * D;
  for (int e = tid; e < 32 * F4; e += 64 * KW) {
    const int rr = e / F4, c4 = e - rr * F4;
    const int qi = q0 + rr;
    if (qi >= p.Sq) continue;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < KW; ++w) mx = fmaxf(mx, sm[w * 32 + rr]);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    float lt = 0.f;
    if (mx != -INFINITY) {
#pragma unroll
      for (int w = 0; w < KW; ++w) {
        const float mw = sm[w * 32 + rr];
        const float sc = mw == -INFINITY ? 0.f : exp2f(mw - mx);
        const float4 x = *(const float4*)(so + (w * 32 + rr) * OROW + 4 * c4);
        lt += sc * sl[w * 32 + rr];
        acc.x += sc * x.x; acc.y += sc * x.y; acc.z += sc * x.z; acc.w += sc * x.w;
      }
    }
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    *(float4*)(ob + (int64_t)qi * p.ldo + 4 * c4) = make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
  }
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
    TH_CHECK_ARG(d->ld_k < ((int64_t)1 << 24) && d->ld_v < ((int64_t)1 << 24),
                 "th_attention_prefill: bf16 k/v row strides must be under 2^24 elements");
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
    k.xcd_map = (d->batch * d->heads_kv) % 8 == 0 ? 1 : 0;
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
    k.scale_log2 = d->scale * log2e;
    // head_dim 64 / 128 (16-byte aligned rows): the matrix-core kernel, 32 queries per wave;
    // 16 / 32: the scalar kernel, one query per lane
    const bool mfma = (hd == 64 || hd == 128) && d->ld_q % 4 == 0 && d->ld_k % 4 == 0 && d->ld_o % 4 == 0 &&
                      ((uintptr_t)d->q | (uintptr_t)d->k | (uintptr_t)d->o) % 16 == 0;
    if (mfma) {
      const dim3 grid((unsigned)cdiv(d->seq_q, 32), (unsigned)(d->batch * d->heads_q));
      if (hd == 64)
        hipLaunchKernelGGL((attn_fwd_f32_mfma_kernel<64, 4>), grid, dim3(256), 0, s, k);
      else
        hipLaunchKernelGGL((attn_fwd_f32_mfma_kernel<128, 4>), grid, dim3(256), 0, s, k);
    } else {
      const dim3 grid((unsigned)cdiv(d->seq_q, 64), (unsigned)(d->batch * d->heads_q));
      switch (hd) {
        case 16: hipLaunchKernelGGL(attn_fwd_f32_kernel<16>, grid, dim3(64), 0, s, k); break;
        case 32: hipLaunchKernelGGL(attn_fwd_f32_kernel<32>, grid, dim3(64), 0, s, k); break;
        case 64: hipLaunchKernelGGL(attn_fwd_f32_kernel<64>, grid, dim3(64), 0, s, k); break;
        default: hipLaunchKernelGGL(attn_fwd_f32_kernel<128>, grid, dim3(64), 0, s, k); break;
      }
    }
  }
  TH_CHECK_LAUNCH();
  return TH_OK;
}
