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
#include <cstdlib>

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
};

// Running sum of dA (or the given cum re-based) for chunk ``c`` into cl[0..Q),
// dt into dts[0..Q); rows past the end of the sequence get dt = 0 and repeat
// the last running sum. Needs 2*256 floats of scratch in ``tmp``.
__device__ void chunk_running_sum(const SsdK& p, int b, int h, int c, float* cl, float* dts, float* tmp) {
  const int tid = threadIdx.x;
  const int t0 = c * p.Q;
  const int rows = min(p.Q, p.S - t0);
  float v = 0.f, dtv = 0.f;
  if (tid < p.Q) {
    const int l = min(tid, rows - 1);
    const int64_t tok = (int64_t)b * p.S + t0 + l;
    const float d = load_elem(p.dt, tok * p.lddt + (int64_t)h * p.dt_stride, p.dtype);
    dtv = tid < rows ? d : 0.f;
    if (p.cum == nullptr) {
      v = tid < rows ? d * p.A[h] : 0.f;
    } else {
      v = load_elem(p.cum, tok * p.ldcum + (int64_t)h * p.dt_stride, p.dtype);
    }
  }
  if (p.cum == nullptr) {
    // inclusive Hillis-Steele scan over Q <= 256 values
    float* a = tmp;
    float* bb = tmp + 256;
    a[tid] = v;
    __syncthreads();
    for (int off = 1; off < p.Q; off <<= 1) {
      float s = a[tid];
      if (tid >= off && tid < p.Q) s += a[tid - off];
      bb[tid] = s;
      __syncthreads();
      float* t = a; a = bb; bb = t;
    }
    if (tid < p.Q) cl[tid] = a[tid];
  } else {
    // re-base on the running sum just before the chunk (its first row for chunk 0,
    // where no earlier state exists and only differences are used)
    float base;
    if (c == 0) {
      base = load_elem(p.cum, ((int64_t)b * p.S) * p.ldcum + (int64_t)h * p.dt_stride, p.dtype);
    } else {
      base = load_elem(p.cum, ((int64_t)b * p.S + t0 - 1) * p.ldcum + (int64_t)h * p.dt_stride, p.dtype);
    }
    if (tid < p.Q) cl[tid] = v - base;
  }
  if (tid < p.Q) dts[tid] = dtv;
  __syncthreads();
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
// operands, fp32 accumulation). Operand layouts of the 32x32x16 MFMA, lane l:
//   A (32 x 16): row l%32, k = 8*(l/32) .. +8      B (16 x 32): col l%32, same k
//   C (32 x 32): register r holds row 8*(r/4) + 4*(l/32) + r%4, col l%32.
// The computed operands w_l x_l (chunk states), M = (C B^T) o L and the carried
// state H are fp32; each enters the MFMA as hi + lo, two bf16 parts with
// hi = bf16(v), lo = bf16(v - hi), so they carry ~16 mantissa bits. Inputs x,
// B, C are bf16 already; all sums are fp32.

__device__ __forceinline__ bf16x8_t pack8_bf16(const float* v) {
  uint4 w;
  w.x = (uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16);
  w.y = (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16);
  w.z = (uint32_t)f32_to_bf16(v[4]) | ((uint32_t)f32_to_bf16(v[5]) << 16);
  w.w = (uint32_t)f32_to_bf16(v[6]) | ((uint32_t)f32_to_bf16(v[7]) << 16);
  return __builtin_bit_cast(bf16x8_t, w);
}

__device__ __forceinline__ void split8_bf16(const float* v, bf16x8_t& hi, bf16x8_t& lo) {
  float h[8], l[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint16_t hb = f32_to_bf16(v[i]);
    h[i] = bf16_to_f32(hb);
    l[i] = v[i] - h[i];
  }
  hi = pack8_bf16(h);
  lo = pack8_bf16(l);
}

__device__ __forceinline__ bf16x8_t ldg_bf16x8(const void* base, int64_t elem, bool ok) {
  if (!ok) return __builtin_bit_cast(bf16x8_t, make_uint4(0, 0, 0, 0));
  return *(const bf16x8_t*)((const uint16_t*)base + elem);
}

__device__ __forceinline__ int crow_of(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

// Token-major bf16 rows [tok0 + l, col0 .. col0 + 8*C8) of chunk rows l < Q into
// an LDS matrix dst[col][l] (row stride QS), each value times wl[l] (or 1).
__device__ void stage_transposed(const void* src, int64_t ld, int64_t tok0, int64_t col0, int C8, int Q, int rows,
                                 const float* wl, uint16_t* dst, int QS, uint16_t* dst_lo = nullptr) {
  for (int e = threadIdx.x; e < Q * C8; e += 256) {
    const int l = e / C8, c8 = e - l * C8;
    uint4 raw = make_uint4(0, 0, 0, 0);
    if (l < rows) raw = *(const uint4*)((const uint16_t*)src + (tok0 + l) * ld + col0 + c8 * 8);
    const uint32_t ws[4] = {raw.x, raw.y, raw.z, raw.w};
    uint16_t* d = dst + (c8 * 8) * QS + l;
    if (wl) {
      const float w = wl[l];
      uint16_t* dl = dst_lo + (c8 * 8) * QS + l;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float v = __uint_as_float((i & 1) ? (ws[i >> 1] & 0xffff0000u) : (ws[i >> 1] << 16)) * w;
        const uint16_t hb = f32_to_bf16(v);
        d[i * QS] = hb;
        dl[i * QS] = f32_to_bf16(v - bf16_to_f32(hb));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        d[(2 * i) * QS] = (uint16_t)(ws[i] & 0xffffu);
        d[(2 * i + 1) * QS] = (uint16_t)(ws[i] >> 16);
      }
    }
  }
}

// S_c[p][n] = sum_l (w_l x_l[p]) B_l[n],  w_l = dt_l exp(cl_last - cl_l).
__global__ void __launch_bounds__(256) ssd_state_mfma_kernel(SsdK p) {
  extern __shared__ float sm[];
  float* cl = sm;          // 256
  float* dts = cl + 256;   // 256
  float* tmp = dts + 256;  // 512
  const int Q = p.Q, P = p.P, N = p.N, QS = Q + 8;
  uint16_t* xt = (uint16_t*)(tmp + 512);  // [P][QS]  w_l x_l (hi part), transposed
  uint16_t* xl = xt + P * QS;             // [P][QS]  its lo part
  uint16_t* bt = xl + P * QS;             // [N][QS]  B_l, transposed
  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z, tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = h / p.hpg;
  chunk_running_sum(p, b, h, c, cl, dts, tmp);
  const int t0 = c * Q;
  const int rows = min(Q, p.S - t0);
  const float last = cl[Q - 1];
  if (tid < Q) tmp[tid] = dts[tid] * __expf(last - cl[tid]);  // w_l (0 past the sequence end: dt = 0)
  __syncthreads();
  const int64_t tok0 = (int64_t)b * p.S + t0;
  stage_transposed(p.x, p.ldx, tok0, (int64_t)h * P, P >> 3, Q, rows, tmp, xt, QS, xl);
  stage_transposed(p.b, p.ldb, tok0, (int64_t)g * N, N >> 3, Q, rows, nullptr, bt, QS);
  __syncthreads();
  const int TN = N >> 5;
  float* st = p.states + (((int64_t)b * p.H + h) * p.nc + c) * (int64_t)(P * N);
  for (int tile = wave; tile < (P >> 5) * TN; tile += 4) {
    const int ti = tile / TN, tj = tile - ti * TN;
    f32x16_t acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
    const uint16_t* ar = xt + (ti * 32 + (lane & 31)) * QS + 8 * (lane >> 5);
    const uint16_t* arl = ar + P * QS;
    const uint16_t* br = bt + (tj * 32 + (lane & 31)) * QS + 8 * (lane >> 5);
    for (int k0 = 0; k0 < Q; k0 += 16) {
      const bf16x8_t bv = *(const bf16x8_t*)(br + k0);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*(const bf16x8_t*)(ar + k0), bv, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*(const bf16x8_t*)(arl + k0), bv, acc, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) st[(int64_t)(ti * 32 + crow_of(r, lane)) * N + tj * 32 + (lane & 31)] = acc[r];
  }
  if (tid == 0) p.tot[((int64_t)b * p.H + h) * p.nc + c] = last;
}

// One workgroup per chunk; each wave takes 32x32 output tiles (32 rows t,
// 32 columns p):
//   y = exp(cl_t) C_t H^T + sum_{s<=t} [(C_t . B_s) exp(cl_t - cl_s) dt_s] x_s + D x_t, times gate,
// where H is the state entering the chunk (the carry kernel's output).
template <int KS>  // state_dim / 16
__global__ void __launch_bounds__(256) ssd_out_mfma_kernel(SsdK p) {
  extern __shared__ float sm[];
  float* cl = sm;
  float* dts = cl + 256;
  float* tmp = dts + 256;
  const int Q = p.Q, P = p.P, N = KS * 16, QS = Q + 8;
  constexpr int MS = 40;                  // M scratch row stride (bf16)
  uint16_t* xt = (uint16_t*)(tmp + 512);  // [P][QS] x transposed
  uint16_t* ms = xt + P * QS;             // per wave [32][MS]
  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z, tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = h / p.hpg;
  chunk_running_sum(p, b, h, c, cl, dts, tmp);
  const int t0 = c * Q;
  const int rows = min(Q, p.S - t0);
  const int64_t tok0 = (int64_t)b * p.S + t0;
  stage_transposed(p.x, p.ldx, tok0, (int64_t)h * P, P >> 3, Q, rows, nullptr, xt, QS);
  __syncthreads();
  uint16_t* msw = ms + wave * 2 * 32 * MS;  // hi tile, then lo tile
  uint16_t* msl = msw + 32 * MS;
  const float* H = p.states + (((int64_t)b * p.H + h) * p.nc + c) * (int64_t)(P * N);
  const int TP = P >> 5, ntb = (rows + 31) >> 5;
  const int64_t ccol = (int64_t)g * N + 8 * (lane >> 5);
  for (int unit = wave; unit < ntb * TP; unit += 4) {
    const int tb = unit / TP, pt = unit - tb * TP;
    const int trow = tb * 32 + (lane & 31);
    bf16x8_t cf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) cf[ks] = ldg_bf16x8(p.c, (tok0 + trow) * p.ldc + ccol + ks * 16, trow < rows);
    f32x16_t acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
    if (c > 0) {
      const float* hr = H + (int64_t)(pt * 32 + (lane & 31)) * N + 8 * (lane >> 5);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const float4 h0 = *(const float4*)(hr + ks * 16), h1 = *(const float4*)(hr + ks * 16 + 4);
        const float hv[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
        bf16x8_t hh, hl;
        split8_bf16(hv, hh, hl);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cf[ks], hh, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cf[ks], hl, acc, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] *= __expf(cl[tb * 32 + crow_of(r, lane)]);
    }
    for (int sb = 0; sb <= tb; ++sb) {
      const int srow = sb * 32 + (lane & 31);
      f32x16_t gacc;
#pragma unroll
      for (int r = 0; r < 16; ++r) gacc[r] = 0.f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        gacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            cf[ks], ldg_bf16x8(p.b, (tok0 + srow) * p.ldb + ccol + ks * 16, srow < rows), gacc, 0, 0, 0);
      // M[t][s] = G o L, written to this wave's scratch as bf16 (A-operand layout on read)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int tr = crow_of(r, lane), t = tb * 32 + tr;
        const float m = (srow <= t && srow < rows) ? gacc[r] * __expf(cl[t] - cl[srow]) * dts[srow] : 0.f;
        const uint16_t mh = f32_to_bf16(m);
        msw[tr * MS + (lane & 31)] = mh;
        msl[tr * MS + (lane & 31)] = f32_to_bf16(m - bf16_to_f32(mh));
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
        const int mo = (lane & 31) * MS + k2 * 16 + 8 * (lane >> 5);
        const bf16x8_t bx = *(const bf16x8_t*)(xt + (pt * 32 + (lane & 31)) * QS + sb * 32 + k2 * 16 + 8 * (lane >> 5));
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*(const bf16x8_t*)(msw + mo), bx, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*(const bf16x8_t*)(msl + mo), bx, acc, 0, 0, 0);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    const int pp = pt * 32 + (lane & 31);
    const int64_t col = (int64_t)h * P + pp;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = tb * 32 + crow_of(r, lane);
      if (t >= rows) continue;
      const int64_t tok = tok0 + t;
      const float xv = load_elem(p.x, tok * p.ldx + col, p.dtype);
      float v = acc[r];
      if (p.dskip) v += xv * load_elem(p.dskip, tok * p.lddskip + col, p.dtype);
      else if (p.D) v += xv * p.D[h];
      if (p.gate) v *= load_elem(p.gate, tok * p.ldgate + col, p.gdt);
      store_elem(p.y, tok * p.ldy + col, p.ydt, v);
      if (p.y32) p.y32[tok * p.ldy32 + col] = v;
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

static size_t state_lds(int P, int N) { return (size_t)(256 * 4 + 32 * P + 32 * N) * 4; }
static size_t state_mfma_lds(int Q, int P, int N) { return 1024 * 4 + (size_t)(2 * P + N) * (Q + 8) * 2; }
static size_t out_mfma_lds(int Q, int P) { return 1024 * 4 + (size_t)P * (Q + 8) * 2 + 4 * 2 * 32 * 40 * 2; }
static size_t out_lds(int RB, int P, int N) {
  const size_t intra = (size_t)RB * (N + 1) + (size_t)RB * (P + 1) + (size_t)RB * (RB + 1);
  const size_t inter = (size_t)P * (N + 1);
  return (size_t)(256 * 4 + RB * (N + 1) + std::max(intra, inter)) * 4;
}

constexpr size_t kMaxLds = 163840;  // 160 KiB per workgroup on gfx950

// Raise the dynamic-LDS limit of the scan kernels once per device (th_init),
// so that launching them needs no attribute call (and can be graph-captured).
int ssd_init_device() {
  const void* fns[] = {(const void*)ssd_state_kernel, (const void*)ssd_out_kernel, (const void*)ssd_state_mfma_kernel,
                       (const void*)ssd_out_mfma_kernel<2>, (const void*)ssd_out_mfma_kernel<4>,
                       (const void*)ssd_out_mfma_kernel<8>};
  for (const void* f : fns) TH_CHECK_HIP(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxLds));
  return TH_OK;
}

// TH_SSD_VALU=1 keeps the fp32 VALU kernels for bf16 inputs too.
static bool ssd_force_valu() {
  static const bool v = [] {
    const char* e = getenv("TH_SSD_VALU");
    return e && e[0] == '1';
  }();
  return v;
}

}  // namespace th

using namespace th;

extern "C" int64_t th_ssd_workspace_bytes(int32_t batch, int32_t seq, int32_t heads, int32_t head_dim,
                                          int32_t state_dim, int32_t chunk) {
  if (batch <= 0 || seq <= 0 || heads <= 0 || head_dim <= 0 || state_dim <= 0 || chunk <= 0) return -1;
  const int64_t nc = cdiv(seq, chunk);
  return (int64_t)batch * heads * nc * ((int64_t)head_dim * state_dim + 1) * 4;
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
  k.states = d->workspace;
  k.tot = d->workspace + (int64_t)k.B * k.H * k.nc * k.P * k.N;
  hipStream_t s = (hipStream_t)stream;
  // MFMA path: bf16 operands, 32-multiple tiles, 16-byte aligned rows.
  auto al16 = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
  const bool mfma = d->dtype == TH_BF16 && k.P % 32 == 0 && k.P <= 128 && (k.N == 32 || k.N == 64 || k.N == 128) &&
                    k.Q % 32 == 0 && d->ld_x % 8 == 0 && d->ld_b % 8 == 0 && d->ld_c % 8 == 0 && al16(d->x) &&
                    al16(d->b) && al16(d->c) && state_mfma_lds(k.Q, k.P, k.N) <= kMaxLds &&
                    out_mfma_lds(k.Q, k.P) <= kMaxLds && !ssd_force_valu();
  if (mfma) {
    const size_t l1 = state_mfma_lds(k.Q, k.P, k.N), l3 = out_mfma_lds(k.Q, k.P);
    hipLaunchKernelGGL(ssd_state_mfma_kernel, dim3(k.nc, k.H, k.B), dim3(256), l1, s, k);
    TH_CHECK_LAUNCH();
    hipLaunchKernelGGL(ssd_carry_kernel, dim3((unsigned)cdiv(k.P * k.N, 256), k.H, k.B), dim3(256), 0, s, k);
    TH_CHECK_LAUNCH();
    if (k.N == 32)
      hipLaunchKernelGGL(ssd_out_mfma_kernel<2>, dim3(k.nc, k.H, k.B), dim3(256), l3, s, k);
    else if (k.N == 64)
      hipLaunchKernelGGL(ssd_out_mfma_kernel<4>, dim3(k.nc, k.H, k.B), dim3(256), l3, s, k);
    else
      hipLaunchKernelGGL(ssd_out_mfma_kernel<8>, dim3(k.nc, k.H, k.B), dim3(256), l3, s, k);
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
  hipLaunchKernelGGL(conv1d_causal_kernel, dim3((unsigned)((int64_t)k.B * k.S), (unsigned)cdiv(k.W, 256)), dim3(256), 0,
                     (hipStream_t)stream, k);
  TH_CHECK_LAUNCH();
  return TH_OK;
}
