// Mamba-2 SSD scan (ssd / ssd_chunked kinds) and the depthwise causal conv1d.
//
// Scan, per (batch b, head h), in three launches:
//   1. ssd_state_kernel   one workgroup per chunk: the running sum ``cl`` of
//      dt*A inside the chunk (an LDS scan), w_l = dt_l exp(cl_last - cl_l) and
//      the chunk state S_c[p, n] = sum_l x_l[p] w_l B_l[n];
//   2. ssd_carry_kernel   per state element, sequentially over chunks:
//      H_0 = 0, H_{c+1} = exp(tot_c) H_c + S_c (tot_c = the chunk's total decay);
//   3. ssd_out_kernel     one workgroup per (chunk, 64-row block): the state
//      term exp(cl_t) C_t . H_c, the within-chunk term
//      sum_{s<=t} (C_t . B_s) exp(cl_t - cl_s) dt_s x_s, plus D x_t, times gate.
// Every exponent is a difference of running sums within a chunk or a chunk
// total, so no exponent is positive except through round-off. All arithmetic is
// fp32 (VALU), operands are staged in LDS; states live in a caller workspace.
//
// The reference's own ``ssd`` kind passes the running sum ``cum`` directly
// (already centred, reference optimizer/passes.py:501-525); only differences of
// it are used here, so its centring offset cancels.
#include <algorithm>

#include "common.h"

namespace th {

struct SsdK {
  int B, S, H, P, N, G, Q, nc, hpg, RB, dt_stride, dtype;
  const void* x; int64_t ldx;
  const void* b; int64_t ldb;
  const void* c; int64_t ldc;
  const void* dt; int64_t lddt;
  const void* cum; int64_t ldcum;
  const float* A;
  const float* D;
  const void* dskip; int64_t lddskip;
  const void* gate; int64_t ldgate; int gdt;
  void* y; int64_t ldy; int ydt;
  float* y32; int64_t ldy32;
  float* states;  // [B][H][nc][P*N]
  float* tot;     // [B][H][nc]
  int vec_epi;    // bf16 y (and gate), no dskip, 16-byte aligned rows: vector epilogue
  float* gtile;   // optional [B][G][nc][npair][64 lanes][16]: the chunks' G^T tiles (MFMA path)
  int npair;      // tiles per chunk: (Q/32)(Q/32 + 1)/2
  const float* ygain;  // optional [H*P]: y stored times this gain (vector epilogue), and
  float* rsp;          // the sums of squares of y before it per (token, 32-column block)
  int64_t ldrsp;
};

// Running sum of dA (or the given cum re-based) for chunk ``c`` into cl[0..Q),
// dt into dts[0..Q); rows past the end of the sequence get dt = 0 and repeat
// the last running sum. In two parts so that a kernel can issue other loads
// between this thread's loads and the scan that waits for them: the first
// keeps the loaded words raw (a conversion there would wait for the load).
// 256 threads.
struct RunSumIn {
  uint32_t dt, cum, base;  // bf16 in the low half or fp32 bits, by p.dtype
  float a;                 // A[h] (the dA path)
};

__device__ __forceinline__ uint32_t load_raw(const void* q, int64_t i, int dtype) {
  return dtype == TH_BF16 ? (uint32_t)((const uint16_t*)q)[i] : ((const uint32_t*)q)[i];
}

__device__ __forceinline__ float raw_f32(uint32_t w, int dtype) {
  return __uint_as_float(dtype == TH_BF16 ? w << 16 : w);
}

__device__ __forceinline__ RunSumIn chunk_running_sum_load(const SsdK& p, int b, int h, int c) {
  const int tid = threadIdx.x;
  const int t0 = c * p.Q;
  const int rows = min(p.Q, p.S - t0);
  // Every load is issued on both sides of the cum test (without cum they all
  // read dt's first element, unused): a register left unloaded on one side
  // makes the compiler wait for the other side's load there.
  const bool cm = p.cum != nullptr;
  const void* cs = cm ? p.cum : p.dt;
  RunSumIn r{0u, 0u, 0u, cm ? 0.f : p.A[h]};
  const int l = min(min(tid, p.Q - 1), rows - 1);
  const int64_t tok = (int64_t)b * p.S + t0 + l;
  r.dt = load_raw(p.dt, tok * p.lddt + (int64_t)h * p.dt_stride, p.dtype);
  r.cum = load_raw(cs, cm ? tok * p.ldcum + (int64_t)h * p.dt_stride : 0, p.dtype);
  // re-base on the running sum just before the chunk (its first row for chunk 0,
  // where no earlier state exists and only differences are used)
  const int64_t row = (int64_t)b * p.S + (c == 0 ? 0 : t0 - 1);
  r.base = load_raw(cs, cm ? row * p.ldcum + (int64_t)h * p.dt_stride : 0, p.dtype);
  return r;
}

// Needs 4 floats of scratch in ``tmp``.
__device__ __forceinline__ void chunk_running_sum_finish(const SsdK& p, int h, int c, const RunSumIn& r, float* cl,
                                                         float* dts, float* tmp) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rows = min(p.Q, p.S - c * p.Q);
  const bool in = tid < p.Q && tid < rows;
  const float d = raw_f32(r.dt, p.dtype);
  if (p.cum == nullptr) {
    // inclusive scan: within each wave by shuffles, then the earlier waves' totals
    float x = in ? d * r.a : 0.f;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float y = __shfl_up(x, off, 64);
      if (lane >= off) x += y;
    }
    if (lane == 63) tmp[wave] = x;
    __syncthreads();
    float pre = 0.f;
    for (int w = 0; w < wave; ++w) pre += tmp[w];
    if (tid < p.Q) cl[tid] = x + pre;
  } else {
    if (tid < p.Q) cl[tid] = raw_f32(r.cum, p.dtype) - raw_f32(r.base, p.dtype);
  }
  if (tid < p.Q) dts[tid] = in ? d : 0.f;
  __syncthreads();
}

__device__ void chunk_running_sum(const SsdK& p, int b, int h, int c, float* cl, float* dts, float* tmp) {
  chunk_running_sum_finish(p, h, c, chunk_running_sum_load(p, b, h, c), cl, dts, tmp);
}

__global__ void __launch_bounds__(256) ssd_state_kernel(SsdK p) {
  extern __shared__ float sm[];
  float* cl = sm;            // 256
  float* dts = cl + 256;     // 256
  float* tmp = dts + 256;    // 512
  float* xs = tmp + 512;     // 32 * P
  float* bs = xs + 32 * p.P; // 32 * N
  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const int g = h / p.hpg;
  chunk_running_sum(p, b, h, c, cl, dts, tmp);
  const int t0 = c * p.Q;
  const int rows = min(p.Q, p.S - t0);
  const float last = cl[p.Q - 1];
  const int PN = p.P * p.N;
  const int no = PN / 256;  // P*N is a multiple of 256 (checked on the host)
  float acc[64];
#pragma unroll
  for (int i = 0; i < 64; ++i) acc[i] = 0.f;
  for (int l0 = 0; l0 < rows; l0 += 32) {
    for (int e = tid; e < 32 * p.P; e += 256) {
      const int ll = e / p.P, pp = e - ll * p.P;
      const int l = l0 + ll;
      float v = 0.f;
      if (l < rows) {
        const int64_t tok = (int64_t)b * p.S + t0 + l;
        v = load_elem(p.x, tok * p.ldx + (int64_t)h * p.P + pp, p.dtype) * dts[l] * __expf(last - cl[l]);
      }
      xs[e] = v;
    }
    for (int e = tid; e < 32 * p.N; e += 256) {
      const int ll = e / p.N, nn = e - ll * p.N;
      const int l = l0 + ll;
      bs[e] = l < rows ? load_elem(p.b, ((int64_t)b * p.S + t0 + l) * p.ldb + (int64_t)g * p.N + nn, p.dtype) : 0.f;
    }
    __syncthreads();
    for (int ll = 0; ll < 32; ++ll) {
#pragma unroll
      for (int i = 0; i < 64; ++i) {
        if (i < no) {
          const int o = tid + 256 * i;
          const int pp = o / p.N, nn = o - pp * p.N;
          acc[i] += xs[ll * p.P + pp] * bs[ll * p.N + nn];
        }
      }
    }
    __syncthreads();
  }
  float* st = p.states + (((int64_t)b * p.H + h) * p.nc + c) * PN;
#pragma unroll
  for (int i = 0; i < 64; ++i)
    if (i < no) st[tid + 256 * i] = acc[i];
  if (tid == 0) p.tot[((int64_t)b * p.H + h) * p.nc + c] = last;
}

__global__ void __launch_bounds__(256) ssd_carry_kernel(SsdK p) {
  const int h = blockIdx.y, b = blockIdx.z;
  const int PN = p.P * p.N;
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e >= PN) return;
  float* st = p.states + ((int64_t)b * p.H + h) * p.nc * PN;
  const float* tot = p.tot + ((int64_t)b * p.H + h) * p.nc;
  float carry = 0.f;
  for (int c = 0; c < p.nc; ++c) {
    const float s = st[(int64_t)c * PN + e];
    st[(int64_t)c * PN + e] = carry;
    carry = (c == 0 ? 0.f : __expf(tot[c]) * carry) + s;
  }
}

__global__ void __launch_bounds__(256) ssd_out_kernel(SsdK p) {
  extern __shared__ float sm[];
  const int RB = p.RB, P = p.P, N = p.N;
  float* cl = sm;                       // 256
  float* dts = cl + 256;                // 256
  float* tmp = dts + 256;               // 512
  float* cs = tmp + 512;                // RB * (N+1)
  float* region = cs + RB * (N + 1);    // Hs [P*(N+1)]  |  Bs [RB*(N+1)] + Xs [RB*(P+1)] + M [RB*(RB+1)]
  float* hs = region;
  float* bsm = region;
  float* xsm = bsm + RB * (N + 1);
  float* msm = xsm + RB * (P + 1);
  const int nrb = p.Q / RB;
  const int c = blockIdx.x / nrb, rbi = blockIdx.x - c * nrb;
  const int h = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const int g = h / p.hpg;
  chunk_running_sum(p, b, h, c, cl, dts, tmp);
  const int t0 = c * p.Q;
  const int rows = min(p.Q, p.S - t0);
  const int r0 = rbi * RB;
  if (r0 >= rows) return;  // whole row block past the end of the sequence (uniform per workgroup)
  const int tpr = 256 / RB;            // threads per output row
  const int pc = P / tpr;              // columns per thread
  const int r = tid / tpr, q = tid - r * tpr;
  const int64_t tok0 = (int64_t)b * p.S + t0;
  float acc[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) acc[i] = 0.f;

  for (int e = tid; e < RB * N; e += 256) {
    const int rr = e / N, nn = e - rr * N;
    cs[rr * (N + 1) + nn] = (r0 + rr < rows) ? load_elem(p.c, (tok0 + r0 + rr) * p.ldc + (int64_t)g * N + nn, p.dtype) : 0.f;
  }
  // state entering the chunk (zero for the first chunk)
  if (c > 0) {
    const float* st = p.states + (((int64_t)b * p.H + h) * p.nc + c) * (int64_t)(P * N);
    for (int e = tid; e < P * N; e += 256) {
      const int pp = e / N, nn = e - pp * N;
      hs[pp * (N + 1) + nn] = st[e];
    }
    __syncthreads();
    const float* crow = cs + r * (N + 1);
    for (int n = 0; n < N; ++n) {
      const float cv = crow[n];
#pragma unroll
      for (int i = 0; i < 32; ++i)
        if (i < pc) acc[i] += cv * hs[(q + tpr * i) * (N + 1) + n];
    }
    const float sc = __expf(cl[r0 + r]);
#pragma unroll
    for (int i = 0; i < 32; ++i) acc[i] *= sc;
  }
  __syncthreads();
  // within the chunk: row blocks jb <= rbi
  for (int jb = 0; jb <= rbi; ++jb) {
    const int j0 = jb * RB;
    for (int e = tid; e < RB * N; e += 256) {
      const int jj = e / N, nn = e - jj * N;
      bsm[jj * (N + 1) + nn] = (j0 + jj < rows) ? load_elem(p.b, (tok0 + j0 + jj) * p.ldb + (int64_t)g * N + nn, p.dtype) : 0.f;
    }
    for (int e = tid; e < RB * P; e += 256) {
      const int jj = e / P, pp = e - jj * P;
      xsm[jj * (P + 1) + pp] = (j0 + jj < rows) ? load_elem(p.x, (tok0 + j0 + jj) * p.ldx + (int64_t)h * P + pp, p.dtype) : 0.f;
    }
    __syncthreads();
    // M[r][j] = (C_r . B_j) exp(cl_r - cl_j) dt_j  for j <= r
    for (int e = tid; e < RB * RB; e += 256) {
      const int rr = e / RB, jj = e - rr * RB;
      float m = 0.f;
      if (j0 + jj <= r0 + rr && j0 + jj < rows) {
        float dot = 0.f;
        const float* crow = cs + rr * (N + 1);
        const float* brow = bsm + jj * (N + 1);
        for (int n = 0; n < N; ++n) dot += crow[n] * brow[n];
        m = dot * __expf(cl[r0 + rr] - cl[j0 + jj]) * dts[j0 + jj];
      }
      msm[rr * (RB + 1) + jj] = m;
    }
    __syncthreads();
    const float* mrow = msm + r * (RB + 1);
    for (int j = 0; j < RB; ++j) {
      const float m = mrow[j];
#pragma unroll
      for (int i = 0; i < 32; ++i)
        if (i < pc) acc[i] += m * xsm[j * (P + 1) + q + tpr * i];
    }
    __syncthreads();
  }
  if (r0 + r >= rows) return;
  const int64_t tok = tok0 + r0 + r;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    if (i >= pc) continue;
    const int pp = q + tpr * i;
    const int64_t col = (int64_t)h * P + pp;
    const float xv = load_elem(p.x, tok * p.ldx + col, p.dtype);
    float v = acc[i];
    if (p.dskip) v += xv * load_elem(p.dskip, tok * p.lddskip + col, p.dtype);
    else if (p.D) v += xv * p.D[h];
    if (p.gate) v *= load_elem(p.gate, tok * p.ldgate + col, p.gdt);
    store_elem(p.y, tok * p.ldy + col, p.ydt, v);
    if (p.y32) p.y32[tok * p.ldy32 + col] = v;
  }
}

// ------------------------------------------------------ bf16 MFMA scan path
// Same three-step scan with every product on v_mfma_f32_32x32x16_bf16 (bf16
// operands, fp32 accumulation). Operand layouts of the 32x32x16 MFMA, lane l,
// g = l/32:
//   A (32 x 16): row l%32, k = 8g .. 8g+8       B (16 x 32): col l%32, same k
//   C (32 x 32): register r holds row 8*(r/4) + 4g + r%4, col l%32.
// A and B fragments have the same shape, so a C result read lane-wise is, as
// it stands, the A or B operand of a next product whose k index runs over its
// rows: registers 0..7 are k-step 0 and 8..15 k-step 1, with the k order
// row(r) of the C layout. Both operands of such a product must come out of a
// C layout (or be stored in that order) so their k orders agree.
//
// Token-major tiles (32 tokens x 32 columns of x or B) become operands with k
// over tokens through an identity product: D = X I copies X exactly (bf16 in,
// one nonzero product per fp32 sum) into the C layout, lane = column,
// register = token. Nothing is transposed through LDS.
//
// Computed fp32 operands (w_l x_l, the masked decay products and the carried
// state) enter as hi + lo, hi = bf16(v), lo = bf16(v - hi), ~16 mantissa bits;
// x, B, C are bf16 already.

typedef __attribute__((ext_vector_type(2))) float f32x2_t;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

// two fp32 -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ bf16x8_t pk8(const float* v) {
  const uint4 w = make_uint4(pk_bf16(v[0], v[1]), pk_bf16(v[2], v[3]), pk_bf16(v[4], v[5]), pk_bf16(v[6], v[7]));
  return __builtin_bit_cast(bf16x8_t, w);
}

__device__ __forceinline__ void unpk8(const uint4& w, float* f) {
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    f[2 * q] = __uint_as_float(ws[q] << 16);
    f[2 * q + 1] = __uint_as_float(ws[q] & 0xffff0000u);
  }
}

// lo = bf16(v - hi) from the rounded v: the subtraction is kept out of FMA
// contraction, which the compiler would otherwise decide per kernel instance
// (fusing it with the product that formed v), so every kernel and route that
// splits the same values gets the same bits.
__device__ __forceinline__ void pk8_split(const float* v, bf16x8_t& hi, bf16x8_t& lo) {
#pragma clang fp contract(off)
  const uint4 h = make_uint4(pk_bf16(v[0], v[1]), pk_bf16(v[2], v[3]), pk_bf16(v[4], v[5]), pk_bf16(v[6], v[7]));
  float f[8], r[8];
  unpk8(h, f);
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = v[i] - f[i];
  hi = __builtin_bit_cast(bf16x8_t, h);
  lo = pk8(r);
}

// Branch-free guarded load: out-of-range lanes read element 0 (always valid)
// and return zeros, so a batch of loads issues back to back.
__device__ __forceinline__ bf16x8_t ldg_bf16x8(const void* base, int64_t elem, bool ok) {
  const uint4 v = *(const uint4*)((const uint16_t*)base + (ok ? elem : 0));
  const uint4 z = make_uint4(0, 0, 0, 0);
  return __builtin_bit_cast(bf16x8_t, ok ? v : z);
}

__device__ __forceinline__ int crow_of(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

// B operand of the identity product for k-step kk: 1.0 at k = column (lane % 32).
__device__ __forceinline__ bf16x8_t eye_frag(int lane, int kk) {
  const int j = (lane & 31) - 16 * kk - 8 * (lane >> 5);
  uint32_t w[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) w[q] = (j == 2 * q ? 0x3F80u : 0u) | (j == 2 * q + 1 ? 0x3F800000u : 0u);
  return __builtin_bit_cast(bf16x8_t, make_uint4(w[0], w[1], w[2], w[3]));
}

// 32 rows (lane%32) x 32 columns, given as the two 16-column A fragments -> C layout.
__device__ __forceinline__ f32x16_t relayout(bf16x8_t a0, bf16x8_t a1, bf16x8_t e0, bf16x8_t e1) {
  f32x16_t d;
#pragma unroll
  for (int r = 0; r < 16; ++r) d[r] = 0.f;
  d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, e0, d, 0, 0, 0);
  d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, e1, d, 0, 0, 0);
  return d;
}

// G^T tiles of chunk c, group g: tile (tb, sb), sb <= tb, at pair index
// tb (tb + 1) / 2 + sb, is G^T = B_s C_t^T over the chunk's 32-token blocks t
// (tb) and s (sb), in the MFMA C layout (lane = t, register r = s row
// 8 (r / 4) + 4 (lane / 32) + r % 4), 16 floats per lane. The same loads (C
// rows past the chunk zero, B rows clamped to its last row) and the same MFMA
// chain as the output kernel's own, so either route gives the same bits. With
// one B/C group per several heads every head of a chunk shares the tiles; the
// pairs are dealt round robin over (head within the group, wave), so the
// workgroups of a group share the work.
template <int KS>  // state_dim / 16
__device__ void ssd_g_tiles(const SsdK& p, int b, int g, int hg, int c, int rows) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, gl = lane >> 5, r32 = lane & 31;
  const int64_t tok0 = (int64_t)b * p.S + (int64_t)c * p.Q;
  const int64_t ccol = (int64_t)g * p.N + 8 * gl;
  const char* bbase = (const char*)p.b + (tok0 * p.ldb + (int64_t)g * p.N) * 2;
  const uint32_t ldb2 = (uint32_t)p.ldb * 2, ccol2 = 16 * gl;
  float* gtb = p.gtile + (((int64_t)b * p.G + g) * p.nc + c) * (int64_t)p.npair * 1024;
  const int ntb = (rows + 31) >> 5;
  for (int pi = hg * 4 + wave; pi < ntb * (ntb + 1) / 2; pi += 4 * p.hpg) {
    int tb = 0;
    while ((tb + 1) * (tb + 2) / 2 <= pi) ++tb;
    const int sb = pi - tb * (tb + 1) / 2, t = tb * 32 + r32;
    bf16x8_t cf[KS], bfr[KS];
    const uint32_t sr = (uint32_t)min(sb * 32 + r32, rows - 1);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      cf[ks] = ldg_bf16x8(p.c, (tok0 + t) * p.ldc + ccol + ks * 16, t < rows);
      bfr[ks] = *(const bf16x8_t*)(bbase + (sr * ldb2 + ccol2) + 32 * ks);
    }
    f32x16_t gt;
#pragma unroll
    for (int r = 0; r < 16; ++r) gt[r] = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) gt = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[ks], cf[ks], gt, 0, 0, 0);
    float4* dst = (float4*)(gtb + (int64_t)pi * 1024 + lane * 16);
#pragma unroll
    for (int q = 0; q < 4; ++q) dst[q] = make_float4(gt[4 * q], gt[4 * q + 1], gt[4 * q + 2], gt[4 * q + 3]);
  }
}

// S_c[p][n] = sum_l (w_l x_l[p]) B_l[n],  w_l = dt_l exp(cl_last - cl_l)  (exponent <= 0).
// One workgroup per (chunk, head, batch): wave w owns p-tile w % PT and
// n-tiles w / PT + j * (4 / PT), j < NTW, and walks the chunk in 32-token
// blocks, each x / B block moved into operand order by relayout().
// The blocks come through a ring of kStateRing LDS stages filled by
// direct-to-LDS loads (no registers held for loads in flight; each byte read
// once per workgroup, where two waves share every x and B fragment): stage =
// x block (32 x P bf16) then B block (32 x N), as 16-byte chunks in load
// order, load i covering columns 16 i .. 16 i + 15 of one of them, lane l at
// row l % 32, columns 16 i + 8 (l / 32) .. + 7, so each operand fragment is
// one lane-contiguous 16-byte LDS read. The first stages are issued before
// the running sum. Rows past the chunk's end re-read its last row (their
// weight w_l is zero). NL = loads per wave per stage, (P + N) / 64 rounded
// up; a wave with fewer repeats its last (the same bytes to the same place).
// Occupancy floor: four waves per SIMD (at most 128 VGPRs) for NTW 1 and 2;
// with P = 64, N = 128 four workgroups then fit the LDS (4 x 39 KiB).
constexpr int kStateRing = 3;
template <int NTW, int NL>
__global__ void __launch_bounds__(256, NTW <= 2 ? 4 : 1) ssd_state2_kernel(SsdK p) {
  __shared__ float cl[256], dts[256], tmp[4], wl[256];
  extern __shared__ __align__(16) char ring[];
  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z, tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = h / p.hpg, gl = lane >> 5, r32 = lane & 31;
  const int Q = p.Q, t0 = c * Q, rows = min(Q, p.S - t0);
  const int nsb = (rows + 31) >> 5;
  const int64_t tok0 = (int64_t)b * p.S + t0;
  const int XI = p.P >> 4, NI = XI + (p.N >> 4);  // loads per stage: x, then x + B
  const uint32_t SB = (uint32_t)NI * 1024;         // stage bytes
  const char* xbase = (const char*)p.x + (tok0 * p.ldx + (int64_t)h * p.P) * 2;
  const char* bbase = (const char*)p.b + (tok0 * p.ldb + (int64_t)g * p.N) * 2;
  const uint32_t lds0 = (uint32_t)(uintptr_t)ring;
  // this wave's loads: index n, and its 16-byte column offset within x or B
  int ln[NL];
  uint32_t lcol[NL];
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    ln[i] = min(wave + 4 * i, NI - 1);
    const int ci = ln[i] < XI ? ln[i] : ln[i] - XI;
    lcol[i] = (uint32_t)(32 * ci + 16 * gl);
  }
  auto issue = [&](int sb) {
    const uint32_t r = (uint32_t)min(sb * 32 + r32, rows - 1);
    const uint32_t xo = r * (uint32_t)p.ldx * 2u, bo = r * (uint32_t)p.ldb * 2u;
    const uint32_t st = lds0 + (uint32_t)(sb % kStateRing) * SB;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      if (ln[i] < XI) dma_load16(xbase, xo + lcol[i], st + (uint32_t)ln[i] * 1024);
      else dma_load16(bbase, bo + lcol[i], st + (uint32_t)ln[i] * 1024);
    }
  };
#pragma unroll
  for (int sb = 0; sb < kStateRing - 1; ++sb)
    if (sb < nsb) issue(sb);
  chunk_running_sum(p, b, h, c, cl, dts, tmp);
  const float last = cl[Q - 1];
  if (tid < Q) wl[tid] = dts[tid] * __expf(last - cl[tid]);
  __syncthreads();
  const int PT = p.P >> 5, NT = p.N >> 5, WPP = 4 / PT;
  const int pt = wave % PT, nt0 = wave / PT;
  const bf16x8_t e0 = eye_frag(lane, 0), e1 = eye_frag(lane, 1);
  f32x16_t acc[NTW];
#pragma unroll
  for (int j = 0; j < NTW; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
  for (int sb = 0; sb < nsb; ++sb) {
    // this wave's loads of block sb have landed (those of sb + 1 may not
    // have); after the barrier every wave's have, and every wave is done
    // reading block sb - 1, whose stage block sb + 2 refills
    if (sb + 1 < nsb) wait_vmcnt<NL>();
    else wait_vmcnt<0>();
    barrier_keep_loads();
    if (sb + kStateRing - 1 < nsb) issue(sb + kStateRing - 1);
    const char* st = ring + (sb % kStateRing) * SB + lane * 16;
    const bf16x8_t xa0 = *(const bf16x8_t*)(st + (2 * pt) * 1024);
    const bf16x8_t xa1 = *(const bf16x8_t*)(st + (2 * pt + 1) * 1024);
    const f32x16_t xr = relayout(xa0, xa1, e0, e1);
    float v[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 w4 = *(const float4*)&wl[sb * 32 + 8 * q + 4 * gl];
      v[4 * q] = xr[4 * q] * w4.x;
      v[4 * q + 1] = xr[4 * q + 1] * w4.y;
      v[4 * q + 2] = xr[4 * q + 2] * w4.z;
      v[4 * q + 3] = xr[4 * q + 3] * w4.w;
    }
    bf16x8_t xh0, xl0, xh1, xl1;
    pk8_split(v, xh0, xl0);
    pk8_split(v + 8, xh1, xl1);
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
      const int nt = nt0 + j * WPP;
      if (nt >= NT) continue;
      const bf16x8_t ba0 = *(const bf16x8_t*)(st + (XI + 2 * nt) * 1024);
      const bf16x8_t ba1 = *(const bf16x8_t*)(st + (XI + 2 * nt + 1) * 1024);
      const f32x16_t br = relayout(ba0, ba1, e0, e1);
      float bv[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) bv[r] = br[r];
      const bf16x8_t bb0 = pk8(bv), bb1 = pk8(bv + 8);
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xh0, bb0, acc[j], 0, 0, 0);
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xl0, bb0, acc[j], 0, 0, 0);
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xh1, bb1, acc[j], 0, 0, 0);
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xl1, bb1, acc[j], 0, 0, 0);
    }
  }
  float* sto = p.states + (((int64_t)b * p.H + h) * p.nc + c) * (int64_t)(p.P * p.N);
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    const int nt = nt0 + j * WPP;
    if (nt >= NT) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) sto[(int64_t)(pt * 32 + crow_of(r, lane)) * p.N + nt * 32 + r32] = acc[j][r];
  }
  if (tid == 0) p.tot[((int64_t)b * p.H + h) * p.nc + c] = last;
  // this workgroup's share of the chunk's G^T tiles (set for state_dim 128 only)
  if (p.gtile != nullptr) ssd_g_tiles<8>(p, b, g, h - g * p.hpg, c, rows);
}

// H_0 = 0, H_{c+1} = exp(tot_c) H_c + S_c, written for c >= 1 as the hi/lo bf16
// B fragments of the out kernel's state term: fragment (pt, ks, lane) is
// H[pt*32 + lane%32][16 ks + 8 (lane/32) + j], j < 8, hi (16 bytes) then lo.
// One thread per (p, 8 consecutive n), sequential over the chunks; blocks of
// 256 threads, or of 64 when that many would not reach every CU (the loads of
// a small grid then come from all of them: C2's carry 7.9 -> about 6 us).
__global__ void __launch_bounds__(256) ssd_carry2_kernel(SsdK p, uint4* hf) {
  const int h = blockIdx.y, b = blockIdx.z;
  const int N8 = p.N >> 3, KS = p.N >> 4, PN = p.P * p.N;
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= p.P * N8) return;
  const int pp = e / N8, n8 = e - pp * N8;
  const int frag = ((pp >> 5) * KS + (n8 >> 1)) * 64 + (pp & 31) + 32 * (n8 & 1);
  const int64_t bh = (int64_t)b * p.H + h;
  const float* st = p.states + bh * p.nc * PN + (int64_t)pp * p.N + n8 * 8;
  uint4* out = hf + bh * p.nc * (PN / 4) + 2 * frag;
  const float* tot = p.tot + bh * p.nc;
  float carry[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) carry[i] = 0.f;
  // the loads of up to 8 chunks are issued together; the recurrence then runs on registers
  for (int c0 = 0; c0 + 1 < p.nc; c0 += 8) {
    float4 sv[8][2];
    float dec[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int c = min(c0 + k, p.nc - 2);
      sv[k][0] = *(const float4*)(st + (int64_t)c * PN);
      sv[k][1] = *(const float4*)(st + (int64_t)c * PN + 4);
      dec[k] = tot[c];
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int c = c0 + k;
      if (c + 1 >= p.nc) break;
      const float e = c == 0 ? 0.f : __expf(dec[k]);
      const float s8[8] = {sv[k][0].x, sv[k][0].y, sv[k][0].z, sv[k][0].w,
                           sv[k][1].x, sv[k][1].y, sv[k][1].z, sv[k][1].w};
#pragma unroll
      for (int i = 0; i < 8; ++i) carry[i] = carry[i] * e + s8[i];
      bf16x8_t hi, lo;
      pk8_split(carry, hi, lo);
      uint4* o = out + (int64_t)(c + 1) * (PN / 4);
      o[0] = __builtin_bit_cast(uint4, hi);
      o[1] = __builtin_bit_cast(uint4, lo);
    }
  }
}

// One workgroup per (chunk, head, batch):
//   y_t = exp(cl_t) C_t H^T + sum_{s<=t} (C_t . B_s) exp(cl_t - cl_s) dt_s x_s + D x_t, times gate.
// x of the chunk is staged once in LDS as B fragments (relayout()). A unit is
// a 32-row t-block with NPT p-tiles; for each s-block s <= t the wave forms
// G^T = B_s C_t^T on the MFMA (lane = t, registers = s in C order), weighs it
// element-wise with the decay and uses it directly as the A operand of the
// product with x. Exponents are in base 2 on the raw v_exp_f32 (results below
// 2^-126 flush to zero). For an s-block before the t-block (first token t0)
// the decay factors as exp2(cl_t - cl_t0) exp2(cl_t0 - cl_s): the second
// factor, times dt_s, comes from a per-chunk table in LDS, and the first
// scales the finished rows of acc once per unit (together with the state
// term). Both factors are <= 1 because the running sum of dt A does not
// increase along the chunk (A < 0, dt > 0), so neither overflows where the
// direct exponent would not. Only the diagonal s-block takes the exponent
// per element, and is masked. The result goes out through a per-wave LDS
// tile as 16-byte rows (gate in, y out), 16 rows at a time.
// The carried state's hi/lo fragments (P N 4 bytes, the same for every unit
// of the block) are copied into LDS once, by direct-to-LDS loads issued at the
// start, instead of being re-read from L2 by each unit.
constexpr int kEpiStride = 36;  // floats per row of the per-wave 16 x 32 output tile

// G^T tile min(sb, tb) of a t-block's run of tiles (gtb: its first tile plus
// this lane's 16 floats), as the MFMA C-layout registers
__device__ __forceinline__ f32x16_t ssd_load_gtile(const float* gtb, int sb, int tb) {
  const float4* q = (const float4*)(gtb + (int64_t)min(sb, tb) * 1024);
  f32x16_t v;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float4 f = q[k];
    v[4 * k] = f.x; v[4 * k + 1] = f.y; v[4 * k + 2] = f.z; v[4 * k + 3] = f.w;
  }
  return v;
}

template <int KS, int NPT, bool GT>  // KS = state_dim / 16, NPT = p-tiles per unit, GT: G^T tiles given
__global__ void __launch_bounds__(256, 2) ssd_out2_kernel(SsdK p, const uint4* hf) {
  extern __shared__ float sm[];
  float* cl = sm;          // running sum of dA, in log2 units after set-up
  float* dts = cl + 256;
  float* epi = dts + 256;  // [4 waves][16][kEpiStride]; the running sum's scratch before that
  uint4* xs = (uint4*)(epi + 4 * 16 * kEpiStride);  // [Q/32][2][PT][64] B fragments of x
  uint4* hs = xs + (p.Q >> 5) * 2 * (p.P >> 5) * 64;  // [PT][KS][64][2] carried-state fragments
  float* wt = (float*)(hs + p.P * p.N / 4);           // decay weights, row tb at 16 tb (tb - 1)
  float* sg = wt + 16 * (p.Q >> 5) * ((p.Q >> 5) - 1);  // this head's P output gains (ygain)
  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z, tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = h / p.hpg, gl = lane >> 5, r32 = lane & 31;
  const int Q = p.Q, t0 = c * Q, rows = min(Q, p.S - t0);
  const int PT = p.P >> 5;
  const int64_t tok0 = (int64_t)b * p.S + t0;
  const int ntb = (rows + 31) >> 5;
  {
    // Set-up loads, all in flight together: dt for the running sum, this
    // wave's x tiles (at most 8), then the carried state into LDS (1 KiB per
    // wave-instruction, waited for with wait_vmcnt before the barrier that
    // precedes the first unit). The scan's barriers overlap their latency.
    const RunSumIn rin = chunk_running_sum_load(p, b, h, c);
    const bf16x8_t e0 = eye_frag(lane, 0), e1 = eye_frag(lane, 1);
    bf16x8_t xa[8][2];
#pragma unroll
    for (int k2 = 0; k2 < 8; ++k2) {
      const int u = wave + 4 * k2;
      const int sb = u / PT, pt = u - sb * PT;
      const int l = sb * 32 + r32;
      const bool ok = u < ntb * PT && l < rows;
      const int64_t at = (tok0 + l) * p.ldx + (int64_t)h * p.P + pt * 32 + 8 * gl;
      xa[k2][0] = ldg_bf16x8(p.x, at, ok);
      xa[k2][1] = ldg_bf16x8(p.x, at + 16, ok);
    }
    if (c > 0) {
      // (uniform addresses; the read-first-lanes keep them in scalar registers,
      // which the load's address and M0 operands require; the builtin returns
      // int, so each half goes through uint32_t before widening)
      const uint64_t sa = (uint64_t)(uintptr_t)(hf + (((int64_t)b * p.H + h) * p.nc + c) * (int64_t)(p.P * p.N / 4));
      const uint32_t shi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(sa >> 32));
      const uint32_t slo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)sa);
      const char* src = (const char*)(uintptr_t)(((uint64_t)shi << 32) | (uint64_t)slo);
      const uint32_t dst = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)hs);
      for (int k = wave; k < p.P * p.N / 256; k += 4) dma_load16(src + 1024 * k, 16 * lane, dst + 1024 * k);
    }
    chunk_running_sum_finish(p, h, c, rin, cl, dts, epi);
    if (tid < Q) cl[tid] *= 1.4426950408889634f;
#pragma unroll
    for (int k2 = 0; k2 < 8; ++k2) {
      const int u = wave + 4 * k2;
      if (u >= ntb * PT) break;
      const int sb = u / PT, pt = u - sb * PT;
      const f32x16_t d = relayout(xa[k2][0], xa[k2][1], e0, e1);
      float v[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) v[r] = d[r];
      xs[((sb * 2 + 0) * PT + pt) * 64 + lane] = __builtin_bit_cast(uint4, pk8(v));
      xs[((sb * 2 + 1) * PT + pt) * 64 + lane] = __builtin_bit_cast(uint4, pk8(v + 8));
    }
  }
  if (p.ygain && tid < (p.P >> 2)) ((float4*)sg)[tid] = ((const float4*)(p.ygain + (int64_t)h * p.P))[tid];
  __syncthreads();
  // wt[16 tb (tb - 1) + s] = exp2(cl_t0 - cl_s) dt_s for the s before t0 = 32 tb
  for (int tb = 1; tb < ntb; ++tb)
    for (int s = tid; s < 32 * tb; s += 256)
      wt[16 * tb * (tb - 1) + s] = __builtin_amdgcn_exp2f(cl[tb * 32] - cl[s]) * dts[s];
  wait_vmcnt<0>();  // this wave's share of the carried state has landed
  __syncthreads();
  const int PG = PT / NPT, U = ntb * PG;
  const int64_t ccol = (int64_t)g * p.N + 8 * gl;
  // B rows: a uniform base and 32-bit lane offsets (row stride below 2^22 elements)
  const char* bbase = (const char*)p.b + (tok0 * p.ldb + (int64_t)g * p.N) * 2;
  const uint32_t ldb2 = (uint32_t)p.ldb * 2, ccol2 = 16 * gl;
  const float dh = p.D ? p.D[h] : 0.f;
  float* ep = epi + wave * 16 * kEpiStride;
  // C rows of t-block tb (rows past the chunk's end read as zero)
  auto load_cf = [&](bf16x8_t* dst, int tb) {
    const int t = tb * 32 + r32;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) dst[ks] = ldg_bf16x8(p.c, (tok0 + t) * p.ldc + ccol + ks * 16, t < rows);
  };
  // With the G^T tiles given, C enters only the state term (chunks after the
  // first): a wave's first unit's rows load here, each later unit's while the
  // unit before it runs, once the state term has consumed the current ones.
  // The wave's units: i = 4 k + (k odd ? 3 - wave : wave), k = 0, 1, ...
  bf16x8_t cfn[KS];
  if constexpr (GT) {
    if (c > 0 && wave < U) load_cf(cfn, ntb - 1 - wave / PG);
  }
  for (int i = 0; i < U; ++i) {
    // units by decreasing work, dealt to the waves in snake order
    int w = i & 3;
    if ((i >> 2) & 1) w = 3 - w;
    if (w != wave) continue;
    const int tb = ntb - 1 - i / PG, pg = i % PG;
    const int t = tb * 32 + r32;
    bf16x8_t cf[KS];
    if constexpr (GT) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) cf[ks] = cfn[ks];
    } else {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) cf[ks] = ldg_bf16x8(p.c, (tok0 + t) * p.ldc + ccol + ks * 16, t < rows);
    }
    // the first two G^T tiles load under the state term
    f32x16_t gq[GT ? 2 : 1];
    const float* gtb = GT ? p.gtile + (((int64_t)b * p.G + g) * p.nc + c) * (int64_t)p.npair * 1024 +
                                (int64_t)(tb * (tb + 1) / 2) * 1024 + lane * 16
                          : nullptr;
    if constexpr (GT) {
      gq[0] = ssd_load_gtile(gtb, 0, tb);
      gq[1] = ssd_load_gtile(gtb, 1, tb);
    }
    f32x16_t acc[NPT];
#pragma unroll
    for (int j = 0; j < NPT; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
    // cl at the t-block's first token: the decay exp2(cl_t - cl_s) of every
    // earlier s factors as exp2(cl_t - cl_t0) exp2(cl_t0 - cl_s), both <= 1
    const float clt0 = cl[tb * 32];
    if (c > 0) {
#pragma unroll
      for (int j = 0; j < NPT; ++j) {
        const int pt = pg * NPT + j;
        uint4 hfr[KS][2];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const uint4* f = hs + 2 * ((pt * KS + ks) * 64 + lane);
          hfr[ks][0] = f[0];
          hfr[ks][1] = f[1];
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cf[ks], __builtin_bit_cast(bf16x8_t, hfr[ks][0]), acc[j], 0, 0, 0);
          acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cf[ks], __builtin_bit_cast(bf16x8_t, hfr[ks][1]), acc[j], 0, 0, 0);
        }
      }
      if constexpr (GT) {
        const int k = i >> 2, inext = 4 * (k + 1) + (((k + 1) & 1) ? 3 - wave : wave);
        if (inext < U) load_cf(cfn, ntb - 1 - inext / PG);
      }
      // state term exp2(cl_t) C_t H = exp2(cl_t - cl_t0) (exp2(cl_t0) C_t H): the
      // per-row factor is applied with the earlier s-blocks' terms below
      const float e0 = __builtin_amdgcn_exp2f(clt0);
#pragma unroll
      for (int j = 0; j < NPT; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][r] *= e0;
    }
    const float clt = cl[t];
    // B rows of s-block sb; rows past the chunk's end repeat its last row (their
    // products only reach masked or discarded outputs, and x there is zero)
    auto load_b = [&](bf16x8_t* bfr, int sb) {
      const uint32_t sr = (uint32_t)min(sb * 32 + r32, rows - 1);
      const char* bp = bbase + (sr * ldb2 + ccol2);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) bfr[ks] = *(const bf16x8_t*)(bp + 32 * ks);
    };
    // G^T = B_s C_t^T (lane = t, registers = s in C order)
    auto chain = [&](const bf16x8_t* bfr) {
      f32x16_t gt;
#pragma unroll
      for (int r = 0; r < 16; ++r) gt[r] = 0.f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) gt = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[ks], cf[ks], gt, 0, 0, 0);
      return gt;
    };
    // acc += M x_s, M (registers = s) split into bf16 hi + lo
    auto xprod = [&](const float* m, int sb) {
      bf16x8_t mh0, ml0, mh1, ml1;
      pk8_split(m, mh0, ml0);
      pk8_split(m + 8, mh1, ml1);
#pragma unroll
      for (int j = 0; j < NPT; ++j) {
        const int pt = pg * NPT + j;
        const bf16x8_t x0 = __builtin_bit_cast(bf16x8_t, xs[((sb * 2 + 0) * PT + pt) * 64 + lane]);
        const bf16x8_t x1 = __builtin_bit_cast(bf16x8_t, xs[((sb * 2 + 1) * PT + pt) * 64 + lane]);
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(mh0, x0, acc[j], 0, 0, 0);
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ml0, x0, acc[j], 0, 0, 0);
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(mh1, x1, acc[j], 0, 0, 0);
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ml1, x1, acc[j], 0, 0, 0);
      }
    };
    // an earlier s-block: M = G^T exp2(cl_t0 - cl_s) dt_s from the per-t-block table
    auto offdiag = [&](const f32x16_t& gt, int sb) {
      float m[16];
      const float* wr = wt + 16 * tb * (tb - 1) + sb * 32 + 4 * gl;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 w4 = *(const float4*)(wr + 8 * q);
        m[4 * q] = gt[4 * q] * w4.x;
        m[4 * q + 1] = gt[4 * q + 1] * w4.y;
        m[4 * q + 2] = gt[4 * q + 2] * w4.z;
        m[4 * q + 3] = gt[4 * q + 3] * w4.w;
      }
      xprod(m, sb);
    };
    // the diagonal s-block: full decay exp2(cl_t - cl_s) dt_s, masked to s <= t
    auto diag = [&](const f32x16_t& gt) {
      float m[16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int s0 = tb * 32 + 8 * q + 4 * gl;
        const float4 c4 = *(const float4*)&cl[s0];
        const float4 d4 = *(const float4*)&dts[s0];
        const float cs[4] = {c4.x, c4.y, c4.z, c4.w}, ds[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
        for (int i2 = 0; i2 < 4; ++i2) {
          const float v = gt[4 * q + i2] * __builtin_amdgcn_exp2f(clt - cs[i2]) * ds[i2];
          m[4 * q + i2] = 8 * q + 4 * gl + i2 <= r32 ? v : 0.f;
        }
      }
      xprod(m, tb);
    };
    // Earlier s-blocks, each G^T chain issued one step ahead of the weighting
    // and product that consume it (the MFMA chain runs under the VALU work),
    // and the B rows two steps ahead: a buffer is refilled as soon as its
    // chain has read it, a full step before the next chain waits for it. The
    // refills are unconditional (the last two re-read clamped rows) so that
    // every chain waits only for its own loads; a scheduling barrier keeps the
    // compiler from sinking them to their uses.
    f32x16_t g0, g1;
    if constexpr (GT) {
      // The chunk's G^T tiles were formed once per group by the state kernel:
      // each is loaded two s-blocks ahead of the weighting and product that
      // consume it (past the diagonal, the diagonal tile again).
      g0 = gq[0];
      g1 = gq[GT ? 1 : 0];
      int sb = 0;
      while (sb < tb) {
        offdiag(g0, sb);
        g0 = ssd_load_gtile(gtb, sb + 2, tb);
        if (++sb == tb) break;
        offdiag(g1, sb);
        g1 = ssd_load_gtile(gtb, sb + 2, tb);
        ++sb;
      }
    } else {
      bf16x8_t b0[KS], b1[KS];
      load_b(b0, 0);
      if (tb > 0) load_b(b1, 1);
      g0 = chain(b0);
      int sb = 0;
      while (sb < tb) {
        load_b(b0, sb + 2);
        __builtin_amdgcn_sched_barrier(0);
        g1 = chain(b1);  // s-block sb + 1
        offdiag(g0, sb);
        if (++sb == tb) break;
        load_b(b1, sb + 2);
        __builtin_amdgcn_sched_barrier(0);
        g0 = chain(b0);
        offdiag(g1, sb);
        ++sb;
      }
    }
    // rows t of acc: the factor exp2(cl_t - cl_t0) of the state and earlier terms
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 c4 = *(const float4*)&cl[tb * 32 + 8 * q + 4 * gl];
      const float ex[4] = {__builtin_amdgcn_exp2f(c4.x - clt0), __builtin_amdgcn_exp2f(c4.y - clt0),
                           __builtin_amdgcn_exp2f(c4.z - clt0), __builtin_amdgcn_exp2f(c4.w - clt0)};
#pragma unroll
      for (int j = 0; j < NPT; ++j)
#pragma unroll
        for (int i2 = 0; i2 < 4; ++i2) acc[j][4 * q + i2] *= ex[i2];
    }
    // the vector epilogue's gate rows, fetched under the diagonal block: lane
    // (row, c0) holds 8 columns of rows 16 hh + row of the t-block
    const int erow = lane >> 2, ec0 = 8 * (lane & 3);
    bool eok[2];
    int64_t etok[2];
    uint4 gw[NPT][2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int tr = tb * 32 + 16 * hh + erow;
      eok[hh] = tr < rows;
      etok[hh] = tok0 + (eok[hh] ? tr : 0);
    }
    if (p.vec_epi && p.gate) {
#pragma unroll
      for (int j = 0; j < NPT; ++j)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
          gw[j][hh] = *(const uint4*)((const uint16_t*)p.gate + etok[hh] * p.ldgate + (int64_t)h * p.P +
                                      (pg * NPT + j) * 32 + ec0);
    }
    if (tb & 1) diag(g1);
    else diag(g0);
#pragma unroll
    for (int j = 0; j < NPT; ++j) {
      const int pt = pg * NPT + j;
      float xv[16];
      unpk8(xs[((tb * 2 + 0) * PT + pt) * 64 + lane], xv);
      unpk8(xs[((tb * 2 + 1) * PT + pt) * 64 + lane], xv + 8);
      const int64_t col = (int64_t)h * p.P + pt * 32 + r32;
      if (p.vec_epi) {
        // C layout -> row-major 16-row tile in LDS -> 8 columns of one row per
        // lane; registers 8 hh .. 8 hh + 7 hold rows 16 hh .. 16 hh + 15
        const int row = erow, c0 = ec0;
        const int64_t oc = (int64_t)h * p.P + pt * 32 + c0;
        const bool* ok = eok;
        const int64_t* tok = etok;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
          for (int r = 0; r < 8; ++r)
            ep[(crow_of(8 * hh + r, lane) - 16 * hh) * kEpiStride + r32] = acc[j][8 * hh + r] + xv[8 * hh + r] * dh;
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
          __builtin_amdgcn_wave_barrier();
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
          float v[8];
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            const float4 f = *(const float4*)&ep[row * kEpiStride + c0 + 4 * q];
            v[4 * q] = f.x; v[4 * q + 1] = f.y; v[4 * q + 2] = f.z; v[4 * q + 3] = f.w;
          }
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
          __builtin_amdgcn_wave_barrier();
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
          if (p.gate) {
            float gv[8];
            unpk8(gw[j][hh], gv);
#pragma unroll
            for (int k2 = 0; k2 < 8; ++k2) v[k2] *= gv[k2];
          }
          if (p.ygain) {
            // the next RMSNorm's gain, applied here; its row scale is applied by the
            // consumer from these sums: a row's 32 columns of p-tile pt are in the
            // four lanes 4 row .. 4 row + 3, 8 each
            float s2 = 0.f;
#pragma unroll
            for (int k2 = 0; k2 < 8; ++k2) s2 += v[k2] * v[k2];
            s2 += __shfl_xor(s2, 1);
            s2 += __shfl_xor(s2, 2);
            if (ok[hh] && (lane & 3) == 0) p.rsp[tok[hh] * p.ldrsp + (int64_t)h * PT + pt] = s2;
            const float4 g0 = *(const float4*)&sg[pt * 32 + c0], g1 = *(const float4*)&sg[pt * 32 + c0 + 4];
            v[0] *= g0.x; v[1] *= g0.y; v[2] *= g0.z; v[3] *= g0.w;
            v[4] *= g1.x; v[5] *= g1.y; v[6] *= g1.z; v[7] *= g1.w;
          }
          if (ok[hh]) {
            *(uint4*)((uint16_t*)p.y + tok[hh] * p.ldy + oc) = __builtin_bit_cast(uint4, pk8(v));
            if (p.y32) {
              float4* y4 = (float4*)(p.y32 + tok[hh] * p.ldy32 + oc);
              y4[0] = make_float4(v[0], v[1], v[2], v[3]);
              y4[1] = make_float4(v[4], v[5], v[6], v[7]);
            }
          }
        }
      } else {
        // general dtypes / full D: every load of the 16 rows issues before any is used
        float dv[16], gv[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int tr = tb * 32 + crow_of(r, lane);
          const int64_t tok = tok0 + (tr < rows ? tr : 0);
          dv[r] = p.dskip ? load_elem(p.dskip, tok * p.lddskip + col, p.dtype) : dh;
          gv[r] = p.gate ? load_elem(p.gate, tok * p.ldgate + col, p.gdt) : 1.f;
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int tr = tb * 32 + crow_of(r, lane);
          const float v = (acc[j][r] + xv[r] * dv[r]) * gv[r];
          if (tr < rows) {
            const int64_t tok = tok0 + tr;
            store_elem(p.y, tok * p.ldy + col, p.ydt, v);
            if (p.y32) p.y32[tok * p.ldy32 + col] = v;
          }
        }
      }
    }
  }
}

// ------------------------------------------------------------------ conv1d
struct ConvK {
  int B, S, W, K, act, xdt, ydt;
  const void* x; int64_t ldx;
  const float* w;
  void* y; int64_t ldy;
  float* y32; int64_t ldy32;
};

__global__ void __launch_bounds__(256) conv1d_causal_kernel(ConvK p) {
  const int ch = blockIdx.y * 256 + threadIdx.x;
  const int64_t tok = blockIdx.x;  // b*S + t
  if (ch >= p.W) return;
  const int t = (int)(tok % p.S);
  float acc = 0.f;
  for (int j = 0; j < p.K; ++j) {
    const int tt = t - (p.K - 1) + j;
    if (tt < 0) continue;
    acc += p.w[(int64_t)ch * p.K + j] * load_elem(p.x, (tok - (p.K - 1) + j) * p.ldx + ch, p.xdt);
  }
  if (p.act == 1) acc = acc * sigmoidf_(acc);
  store_elem(p.y, tok * p.ldy + ch, p.ydt, acc);
  if (p.y32) p.y32[tok * p.ldy32 + ch] = acc;
}

// bf16 input, 8 channels (one 16-byte vector) x TT consecutive tokens of one
// sequence per thread: the TT + K - 1 input rows the run needs are loaded
// up front (the K - 1 rows before the run come from L2 for every run but the
// first of a sequence), the taps slide over registers, and every access is a
// 16-byte vector (32 bytes for fp32 outputs). Consecutive lanes take
// consecutive channel groups, so a wave reads whole 1 KiB row segments.
template <int K, int TT>
__global__ void __launch_bounds__(256) conv1d_vec_kernel(ConvK p, int cg, int runs) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int g = (int)(idx % cg);
  const int64_t r = idx / cg;  // run over (sequence, token block)
  if (r >= (int64_t)p.B * runs) return;
  const int bseq = (int)(r / runs);
  const int t0 = (int)(r - (int64_t)bseq * runs) * TT;
  const int ch = g * 8;
  float w[8][K];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
#pragma unroll
    for (int j = 0; j < K; ++j) w[c][j] = p.w[(int64_t)(ch + c) * K + j];
  }
  const int64_t base = (int64_t)bseq * p.S;
  uint4 rows[TT + K - 1];
#pragma unroll
  for (int i = 0; i < TT + K - 1; ++i) {
    const int t = t0 - (K - 1) + i;
    rows[i] = (t >= 0 && t < p.S) ? *(const uint4*)((const uint16_t*)p.x + (base + t) * p.ldx + ch)
                                  : make_uint4(0, 0, 0, 0);
  }
  auto unpack = [](const uint4& v, float* f) {
    const uint32_t ws[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      f[2 * q] = __uint_as_float(ws[q] << 16);
      f[2 * q + 1] = __uint_as_float(ws[q] & 0xffff0000u);
    }
  };
#pragma unroll
  for (int i = 0; i < TT; ++i) {
    const int t = t0 + i;
    if (t >= p.S) break;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < K; ++j) {
      float f[8];
      unpack(rows[i + j], f);
#pragma unroll
      for (int c = 0; c < 8; ++c) acc[c] += w[c][j] * f[c];
    }
    if (p.act == 1) {
#pragma unroll
      for (int c = 0; c < 8; ++c) acc[c] = acc[c] * sigmoidf_(acc[c]);
    }
    const int64_t tok = base + t;
    if (p.ydt == TH_BF16) {
      uint4 o;
      o.x = pk_bf16x2(acc[0], acc[1]);
      o.y = pk_bf16x2(acc[2], acc[3]);
      o.z = pk_bf16x2(acc[4], acc[5]);
      o.w = pk_bf16x2(acc[6], acc[7]);
      *(uint4*)((uint16_t*)p.y + tok * p.ldy + ch) = o;
    } else {
      float* yo = (float*)p.y + tok * p.ldy + ch;
      *(float4*)yo = make_float4(acc[0], acc[1], acc[2], acc[3]);
      *(float4*)(yo + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
    }
    if (p.y32) {
      float* yo = p.y32 + tok * p.ldy32 + ch;
      *(float4*)yo = make_float4(acc[0], acc[1], acc[2], acc[3]);
      *(float4*)(yo + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
    }
  }
}

static size_t state_lds(int P, int N) { return (size_t)(256 * 4 + 32 * P + 32 * N) * 4; }
// cl, dts | epilogue tiles (and the running sum's scratch) | x fragments |
// carried state | triangular decay-weight table
static size_t out2_lds(int Q, int P, int N) {
  const size_t nt = Q / 32;
  return 512 * 4 + 4 * 16 * kEpiStride * 4 + (size_t)Q * P * 2 + (size_t)P * N * 4 + 16 * nt * (nt - 1) * 4 +
         (size_t)P * 4;
}
static size_t out_lds(int RB, int P, int N) {
  const size_t intra = (size_t)RB * (N + 1) + (size_t)RB * (P + 1) + (size_t)RB * (RB + 1);
  const size_t inter = (size_t)P * (N + 1);
  return (size_t)(256 * 4 + RB * (N + 1) + std::max(intra, inter)) * 4;
}

constexpr size_t kMaxLds = 163840;  // 160 KiB per workgroup on gfx950

// Raise the dynamic-LDS limit of the scan kernels once per device (th_init),
// so that launching them needs no attribute call (and can be graph-captured).
int ssd_init_device() {
  const void* fns[] = {(const void*)ssd_state_kernel,             (const void*)ssd_out_kernel,
                       (const void*)ssd_out2_kernel<2, 1, false>, (const void*)ssd_out2_kernel<4, 1, false>,
                       (const void*)ssd_out2_kernel<8, 1, false>, (const void*)ssd_out2_kernel<2, 2, false>,
                       (const void*)ssd_out2_kernel<4, 2, false>, (const void*)ssd_out2_kernel<8, 2, false>,
                       (const void*)ssd_out2_kernel<8, 1, true>,  (const void*)ssd_out2_kernel<8, 2, true>};
  for (const void* f : fns) TH_CHECK_HIP(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxLds));
  return TH_OK;
}

}  // namespace th

using namespace th;

// Workspace: chunk states S [B][H][nc][P*N] fp32, chunk totals [B][H][nc]
// (padded to 4 floats), then the carried states as MFMA fragments (4 bytes
// per element, the MFMA path only).
static int64_t ssd_tot_floats(int64_t bhc) { return (bhc + 3) / 4 * 4; }
// G^T tiles: [B][G][nc][npair] tiles of 32 x 32 fp32
static int64_t ssd_gtile_bytes(int64_t batch, int64_t groups, int64_t nc, int64_t npair) {
  return batch * groups * nc * npair * 1024 * 4;
}

extern "C" int64_t th_ssd_workspace_bytes(int32_t batch, int32_t seq, int32_t heads, int32_t head_dim,
                                          int32_t state_dim, int32_t chunk) {
  if (batch <= 0 || seq <= 0 || heads <= 0 || head_dim <= 0 || state_dim <= 0 || chunk <= 0) return -1;
  const int64_t bhc = (int64_t)batch * heads * cdiv(seq, chunk);
  return (2 * bhc * head_dim * state_dim + ssd_tot_floats(bhc)) * 4;
}

// The shared G^T tiles pay for state_dim 128 (8 MFMAs saved per tile, 4 KiB
// reloaded in place of 8 KiB of B rows) with several heads per group. Measured
// on MI355X: N = 128, 256-row chunks, 32 heads per group, 8 x 2048 tokens, 14%
// faster; N = 64, 64-row chunks, 16 heads per group, 2 x 1024 tokens, 4% slower
// (there a tile costs as many bytes as the B rows it replaces).
static bool ssd_gtile_pays(int state_dim, int heads_per_group) { return state_dim == 128 && heads_per_group > 1; }

extern "C" int64_t th_ssd_gtile_workspace_bytes(int32_t batch, int32_t seq, int32_t heads, int32_t head_dim,
                                                int32_t state_dim, int32_t chunk, int32_t ngroups) {
  const int64_t base = th_ssd_workspace_bytes(batch, seq, heads, head_dim, state_dim, chunk);
  if (base < 0) return -1;
  const int g = ngroups > 0 ? ngroups : heads;
  if (heads % g != 0) return -1;
  if (!ssd_gtile_pays(state_dim, heads / g)) return base;
  const int64_t nt = cdiv(std::min(chunk, 256), 32);
  return base + ssd_gtile_bytes(batch, g, cdiv(seq, chunk), nt * (nt + 1) / 2);
}

extern "C" int th_ssd_chunked(const th_ssd_desc* d, void* stream) {
  TH_CHECK_ARG(d != nullptr, "th_ssd_chunked: null descriptor");
  TH_CHECK_ARG(d->batch > 0 && d->seq > 0 && d->heads > 0 && d->head_dim > 0 && d->state_dim > 0,
               "th_ssd_chunked: sizes must be positive");
  TH_CHECK_ARG(d->chunk > 0 && d->chunk <= 256 && (d->chunk <= 64 || d->chunk % 64 == 0),
               "th_ssd_chunked: chunk %d must be <= 64 or a multiple of 64 up to 256", d->chunk);
  const int g = d->ngroups > 0 ? d->ngroups : d->heads;
  TH_CHECK_ARG(d->heads % g == 0, "th_ssd_chunked: heads %d not a multiple of ngroups %d", d->heads, g);
  TH_CHECK_ARG(d->head_dim <= 128 && d->state_dim <= 128, "th_ssd_chunked: head_dim/state_dim above 128");
  TH_CHECK_ARG((d->head_dim * d->state_dim) % 256 == 0, "th_ssd_chunked: head_dim*state_dim must be a multiple of 256");
  TH_CHECK_ARG(d->dtype == TH_BF16 || d->dtype == TH_F32, "th_ssd_chunked: dtype unsupported");
  TH_CHECK_ARG(d->y_dtype == TH_BF16 || d->y_dtype == TH_F32, "th_ssd_chunked: y_dtype unsupported");
  TH_CHECK_ARG(d->x && d->b && d->c && d->dt && d->y && d->workspace, "th_ssd_chunked: null operand");
  TH_CHECK_ARG(d->cum != nullptr || d->A != nullptr, "th_ssd_chunked: needs A or cum");
  TH_CHECK_ARG(d->dt_stride >= 1, "th_ssd_chunked: dt_stride must be >= 1");
  TH_CHECK_ARG(!d->gate || d->gate_dtype == TH_BF16 || d->gate_dtype == TH_F32, "th_ssd_chunked: gate dtype");
  const int64_t need = th_ssd_workspace_bytes(d->batch, d->seq, d->heads, d->head_dim, d->state_dim, d->chunk);
  TH_CHECK_ARG(d->workspace_bytes >= need, "th_ssd_chunked: workspace %lld < %lld bytes", (long long)d->workspace_bytes,
               (long long)need);
  const int RB = std::min(d->chunk, 64);
  TH_CHECK_ARG(256 % RB == 0 && d->head_dim % (256 / RB) == 0 && d->head_dim / (256 / RB) <= 32,
               "th_ssd_chunked: head_dim %d does not fit the row-block mapping", d->head_dim);
  if (!device_ready()) {
    set_error("th_ssd_chunked: th_init was not called for the current device");
    return TH_ERR_NOT_INIT;
  }
  SsdK k{};
  k.B = d->batch; k.S = d->seq; k.H = d->heads; k.P = d->head_dim; k.N = d->state_dim; k.G = g;
  k.Q = d->chunk; k.nc = (int)cdiv(d->seq, d->chunk); k.hpg = d->heads / g; k.RB = RB; k.dt_stride = d->dt_stride;
  k.dtype = d->dtype;
  k.x = d->x; k.ldx = d->ld_x; k.b = d->b; k.ldb = d->ld_b; k.c = d->c; k.ldc = d->ld_c;
  k.dt = d->dt; k.lddt = d->ld_dt; k.cum = d->cum; k.ldcum = d->ld_cum; k.A = d->A; k.D = d->D;
  k.dskip = d->dskip; k.lddskip = d->ld_dskip; k.gate = d->gate; k.ldgate = d->ld_gate; k.gdt = d->gate_dtype;
  k.y = d->y; k.ldy = d->ld_y; k.ydt = d->y_dtype; k.y32 = d->y32; k.ldy32 = d->ld_y32;
  {
    auto a16 = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
    k.vec_epi = d->y_dtype == TH_BF16 && d->ld_y % 8 == 0 && a16(d->y) && !d->dskip &&
                (!d->gate || (d->gate_dtype == TH_BF16 && d->ld_gate % 8 == 0 && a16(d->gate))) &&
                (!d->y32 || (d->ld_y32 % 4 == 0 && a16(d->y32))) && d->head_dim % 32 == 0;
  }
  k.states = d->workspace;
  k.tot = d->workspace + (int64_t)k.B * k.H * k.nc * k.P * k.N;
  k.gtile = nullptr;
  k.npair = (k.Q / 32) * (k.Q / 32 + 1) / 2;
  k.ygain = d->y_gain;
  k.rsp = d->rs_parts;
  k.ldrsp = d->ld_rs_parts;
  hipStream_t s = (hipStream_t)stream;
  // MFMA path: bf16 operands, 32-wide p / n tiles, 16-byte aligned rows.
  auto al16 = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
  const bool mfma = d->dtype == TH_BF16 && (k.P == 32 || k.P == 64 || k.P == 128) &&
                    (k.N == 32 || k.N == 64 || k.N == 128) && k.Q % 32 == 0 && d->ld_x % 8 == 0 &&
                    d->ld_b % 8 == 0 && d->ld_c % 8 == 0 && d->ld_b < (1 << 22) && d->ld_x < (1 << 22) && al16(d->x) &&
                    al16(d->b) && al16(d->c) &&
                    out2_lds(k.Q, k.P, k.N) <= kMaxLds;
  if (d->y_gain) {
    // the gain and the sums live in the MFMA path's vector epilogue only
    TH_CHECK_ARG(mfma && k.vec_epi && !d->y32 && d->rs_parts && ((uintptr_t)d->y_gain & 15) == 0 &&
                     d->ld_rs_parts >= (int64_t)k.H * (k.P / 32),
                 "th_ssd_chunked: y_gain needs the bf16 MFMA path (16-byte aligned bf16 y, no y32 or dskip, "
                 "head_dim a multiple of 32), rs_parts and ld_rs_parts >= heads * head_dim / 32");
  }
  if (mfma) {
    const int64_t bhc = (int64_t)k.B * k.H * k.nc;
    uint4* hf = (uint4*)(d->workspace + bhc * k.P * k.N + ssd_tot_floats(bhc));
    // Several heads per B/C group and room for the tiles after the base workspace
    // (th_ssd_gtile_workspace_bytes): C_t B_s^T of a chunk is formed once per group.
    if (ssd_gtile_pays(k.N, k.hpg) && d->workspace_bytes >= need + ssd_gtile_bytes(k.B, g, k.nc, k.npair))
      k.gtile = (float*)((char*)d->workspace + need);
    const int PT = k.P / 32, NT = k.N / 32;
    const int ntw = (NT * PT + 3) / 4;
    const dim3 grid(k.nc, k.H, k.B);
    // the state kernel's ring: kStateRing stages of 32 x (P + N) bf16; loads
    // per wave per stage (P + N) / 64 rounded up
    const size_t lring = (size_t)kStateRing * 32 * (k.P + k.N) * 2;
    const int nl = (k.P + k.N + 63) / 64;
    if (ntw == 1 && nl == 1) hipLaunchKernelGGL((ssd_state2_kernel<1, 1>), grid, dim3(256), lring, s, k);
    else if (ntw == 1 && nl == 2) hipLaunchKernelGGL((ssd_state2_kernel<1, 2>), grid, dim3(256), lring, s, k);
    else if (ntw == 1) hipLaunchKernelGGL((ssd_state2_kernel<1, 3>), grid, dim3(256), lring, s, k);
    else if (ntw == 2) hipLaunchKernelGGL((ssd_state2_kernel<2, 3>), grid, dim3(256), lring, s, k);
    else hipLaunchKernelGGL((ssd_state2_kernel<4, 4>), grid, dim3(256), lring, s, k);
    TH_CHECK_LAUNCH();
    if (k.nc > 1) {
      const int64_t cus = device_cus() > 0 ? device_cus() : 256;
      const int ct = cdiv(k.P * k.N / 8, 256) * k.H * k.B < cus ? 64 : 256;
      hipLaunchKernelGGL(ssd_carry2_kernel, dim3((unsigned)cdiv(k.P * k.N / 8, ct), k.H, k.B), dim3(ct), 0, s, k, hf);
      TH_CHECK_LAUNCH();
    }
    const size_t l3 = out2_lds(k.Q, k.P, k.N);
    // a full 8-block chunk gives every wave two t-blocks: share each G^T tile over
    // two p-tiles (more accumulators would not fit two waves per SIMD)
    const int npt = k.Q / 32 >= 8 ? std::min(PT, 2) : 1;
#define TH_SSD_OUT2(KS_, NPT_)                                                                       \
  do {                                                                                               \
    if constexpr (KS_ == 8) {                                                                        \
      if (k.gtile) {                                                                                 \
        hipLaunchKernelGGL((ssd_out2_kernel<KS_, NPT_, true>), grid, dim3(256), l3, s, k, (const uint4*)hf); \
        break;                                                                                       \
      }                                                                                              \
    }                                                                                                \
    hipLaunchKernelGGL((ssd_out2_kernel<KS_, NPT_, false>), grid, dim3(256), l3, s, k, (const uint4*)hf);  \
  } while (0)
#define TH_SSD_OUT2_KS(NPT_)                \
  do {                                      \
    if (k.N == 32) TH_SSD_OUT2(2, NPT_);    \
    else if (k.N == 64) TH_SSD_OUT2(4, NPT_); \
    else TH_SSD_OUT2(8, NPT_);              \
  } while (0)
    if (npt == 1) TH_SSD_OUT2_KS(1);
    else TH_SSD_OUT2_KS(2);
#undef TH_SSD_OUT2_KS
#undef TH_SSD_OUT2
    TH_CHECK_LAUNCH();
    return TH_OK;
  }
  const size_t l1 = state_lds(k.P, k.N), l3 = out_lds(RB, k.P, k.N);
  TH_CHECK_ARG(l1 <= kMaxLds && l3 <= kMaxLds, "th_ssd_chunked: shape needs more than 160 KiB of LDS");
  hipLaunchKernelGGL(ssd_state_kernel, dim3(k.nc, k.H, k.B), dim3(256), l1, s, k);
  TH_CHECK_LAUNCH();
  hipLaunchKernelGGL(ssd_carry_kernel, dim3((unsigned)cdiv(k.P * k.N, 256), k.H, k.B), dim3(256), 0, s, k);
  TH_CHECK_LAUNCH();
  hipLaunchKernelGGL(ssd_out_kernel, dim3(k.nc * (k.Q / RB), k.H, k.B), dim3(256), l3, s, k);
  TH_CHECK_LAUNCH();
  return TH_OK;
}

extern "C" int th_conv1d_causal(const th_conv_desc* d, void* stream) {
  TH_CHECK_ARG(d != nullptr, "th_conv1d_causal: null descriptor");
  TH_CHECK_ARG(d->batch > 0 && d->seq > 0 && d->width > 0 && d->kernel > 0 && d->kernel <= 8,
               "th_conv1d_causal: bad sizes (kernel must be 1..8)");
  TH_CHECK_ARG(d->x && d->w && d->y, "th_conv1d_causal: null operand");
  TH_CHECK_ARG((d->x_dtype == TH_BF16 || d->x_dtype == TH_F32) && (d->y_dtype == TH_BF16 || d->y_dtype == TH_F32),
               "th_conv1d_causal: dtype unsupported");
  TH_CHECK_ARG(d->ld_x >= d->width && d->ld_y >= d->width, "th_conv1d_causal: row stride < width");
  TH_CHECK_ARG(d->activation == 0 || d->activation == 1, "th_conv1d_causal: activation %d unknown", d->activation);
  if (!device_ready()) {
    set_error("th_conv1d_causal: th_init was not called for the current device");
    return TH_ERR_NOT_INIT;
  }
  ConvK k{};
  k.B = d->batch; k.S = d->seq; k.W = d->width; k.K = d->kernel; k.act = d->activation;
  k.xdt = d->x_dtype; k.ydt = d->y_dtype; k.x = d->x; k.ldx = d->ld_x; k.w = d->w;
  k.y = d->y; k.ldy = d->ld_y; k.y32 = d->y32; k.ldy32 = d->ld_y32;
  auto al16 = [](const void* q) { return q == nullptr || ((uintptr_t)q & 15) == 0; };
  const bool vec = k.K == 4 && k.xdt == TH_BF16 && k.W % 8 == 0 && k.ldx % 8 == 0 && k.ldy % 8 == 0 &&
                   (!k.y32 || k.ldy32 % 4 == 0) && al16(k.x) && al16(k.y) && al16(k.y32);
  if (vec) {
    // the longest token run (fewest halo re-reads) that still gives about two
    // 256-thread blocks per CU; small problems take short runs
    const int cg = k.W / 8;
    const int64_t want = (int64_t)std::max(device_cus(), 1) * 512;
    int tt = 16;
    while (tt > 1 && (int64_t)cg * k.B * cdiv(k.S, tt) < want) tt >>= 1;
    const int runs = (int)cdiv(k.S, tt);
    const dim3 grid((unsigned)cdiv((int64_t)cg * k.B * runs, 256));
    hipStream_t st = (hipStream_t)stream;
    switch (tt) {
      case 16: hipLaunchKernelGGL((conv1d_vec_kernel<4, 16>), grid, dim3(256), 0, st, k, cg, runs); break;
      case 8: hipLaunchKernelGGL((conv1d_vec_kernel<4, 8>), grid, dim3(256), 0, st, k, cg, runs); break;
      case 4: hipLaunchKernelGGL((conv1d_vec_kernel<4, 4>), grid, dim3(256), 0, st, k, cg, runs); break;
      case 2: hipLaunchKernelGGL((conv1d_vec_kernel<4, 2>), grid, dim3(256), 0, st, k, cg, runs); break;
      default: hipLaunchKernelGGL((conv1d_vec_kernel<4, 1>), grid, dim3(256), 0, st, k, cg, runs); break;
    }
  } else {
    hipLaunchKernelGGL(conv1d_causal_kernel, dim3((unsigned)((int64_t)k.B * k.S), (unsigned)cdiv(k.W, 256)), dim3(256),
                       0, (hipStream_t)stream, k);
  }
  TH_CHECK_LAUNCH();
  return TH_OK;
}
