// OpIR `gemm` kind on CDNA4 MFMA (reference semantics: codegen/interpret.py:22-35;
// Helion template it replaces: codegen/emit.py:71-221).
//
// Layout and tiling
//   lhs    [M, K] row-major (K contiguous), bf16 or fp32.
//   rhs    packed once by th_gemm_pack_rhs into a K-contiguous [Ncat, K] matrix
//          whose rows interleave the n_acc operands tile by tile: block tile n
//          holds rows (n*n_acc + i)*bn + j = column n*bn + j of operand i. A
//          block therefore computes every accumulator of its output columns with
//          one plain "A * B^T" main loop.
//   bf16:  v_mfma_f32_32x32x16_bf16 with fp32 accumulation, 64-wide K tiles,
//          three main loops chosen per shape by th_gemm:
//          * persistent (gemm_bf16_pk_kernel, large grids): one block per CU
//            walks output tiles in an XCD-aware order; 256-row tiles run eight
//            waves (two per SIMD), 128-row tiles four; each wave owns its rows
//            x half of every accumulator's columns (or, with ASPLIT, one whole
//            accumulator), so SwiGLU pairs and whole RoPE heads meet inside the
//            wave. Operand tiles go HBM -> LDS by direct loads
//            (global_load_lds_dwordx4) two stages deep, into an XOR-swizzled
//            layout (conflict-free ds_read_b128 of MFMA operands); the epilogue
//            of tile t overlaps the first loads of tile t+1;
//          * direct (gemm_bf16_dl_kernel, small grids): one block per output
//            tile, 64/128/256-row tiles, the same direct loads in a 2-8 stage
//            ring;
//          * staged (gemm_bf16_kernel): register-staged loads, for K not a
//            multiple of 64 or strides the 32-bit direct-load offsets cannot
//            reach.
//          The RMS sum of squares of lhs rows comes from the A fragments the
//          MFMAs already read, so it costs no extra traffic.
//   fp32:  64 x BNC x 16 tiles of v_mfma_f32_32x32x2f32.
//   Epilogue: accumulators are staged as fp32 through LDS one half-tile at a
//          time; every output op then reads its operands (its own column, the
//          RoPE partner column, other accumulators) from LDS and writes 4
//          consecutive columns per thread, so global stores are coalesced.
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "gemm_internal.h"

namespace th {

// Block id -> output tile. Consecutive workgroups are dealt round-robin to the
// 8 XCDs; remap so each XCD owns a contiguous range of logical tiles, then walk
// that range in groups of 8 tile-rows so neighbouring blocks on one XCD share
// lhs rows and rhs columns in that XCD's L2.
__device__ __forceinline__ void map_tile_id(int pid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int nb = tiles_m * tiles_n;
  if ((nb & 7) == 0) pid = (pid & 7) * (nb >> 3) + (pid >> 3);
  const int G = 8;
  const int group = pid / (G * tiles_n);
  const int first = group * G;
  const int gm = min(tiles_m - first, G);
  const int in_group = pid - group * G * tiles_n;
  tm = first + in_group % gm;
  tn = in_group / gm;
}

__device__ __forceinline__ void map_tile(int tiles_m, int tiles_n, int& tm, int& tn) {
  map_tile_id(blockIdx.x, tiles_m, tiles_n, tm, tn);
}

// 8 consecutive elements (one 16-byte bf16 or two 16-byte fp32 accesses when
// vec8, element by element for a ragged end or unaligned rows).
__device__ __forceinline__ void load8(const void* p, int64_t off, int dtype, bool vec8, int valid, float* v) {
  if (vec8 && valid >= 8) {
    if (dtype == TH_BF16) {
      const uint4 w = *(const uint4*)((const uint16_t*)p + off);
      const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        v[2 * q] = __uint_as_float(ws[q] << 16);
        v[2 * q + 1] = __uint_as_float(ws[q] & 0xffff0000u);
      }
    } else {
      const float4 a = *(const float4*)((const float*)p + off), b = *(const float4*)((const float*)p + off + 4);
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
    return;
  }
#pragma unroll
  for (int q = 0; q < 8; ++q) v[q] = q < valid ? load_elem(p, off + q, dtype) : 0.f;
}

__device__ __forceinline__ void store8(void* p, int64_t off, int dtype, bool vec8, int valid, const float* v) {
  if (vec8 && valid >= 8) {
    if (dtype == TH_BF16) {
      uint4 w;
      w.x = pk_bf16x2(v[0], v[1]);
      w.y = pk_bf16x2(v[2], v[3]);
      w.z = pk_bf16x2(v[4], v[5]);
      w.w = pk_bf16x2(v[6], v[7]);
      *(uint4*)((uint16_t*)p + off) = w;
    } else {
      *(float4*)((float*)p + off) = make_float4(v[0], v[1], v[2], v[3]);
      *(float4*)((float*)p + off + 4) = make_float4(v[4], v[5], v[6], v[7]);
    }
    return;
  }
#pragma unroll
  for (int q = 0; q < 8; ++q)
    if (q < valid) store_elem(p, off + q, dtype, v[q]);
}

// One output op over a 16-row slice of the per-wave epilogue (persistent
// kernel). Lane l takes columns c8 .. c8+8 (c8 = 8 (l % q8), q8 = hbn / 8
// octets per row) of rows r_l + pass * rp, pass < np. The op is a template
// argument, so each output runs one straight loop; every global operand of
// the slice (extra rows, RoPE table rows) is loaded before the first use.
// aoff / boff: slice columns where the op's accumulators a / b start.
template <int OP, bool SUMSQ>
__device__ __forceinline__ void epi_pair(const GemmK& p, const EpiOutK& eo, int o2, const float* wsl,
                                         int ws, int aoff, int boff, const float* rsrow, int64_t row0, int64_t col_w,
                                         int r_l, int c8, int np, int rp, int p0) {
  constexpr bool USES_E = OP == TH_EPI_ADD || OP == TH_EPI_SOFTPLUS_ADD || OP == TH_EPI_MUL;
  constexpr bool USES_T = OP == TH_EPI_ROPE || OP == TH_EPI_ROPE_PAIR;
  const int ia = eo.a, ib = eo.b;
  const bool sa = SUMSQ && ((p.rscale_mask >> ia) & 1u);
  const bool sb = SUMSQ && ib >= 0 && ((p.rscale_mask >> ib) & 1u);
  // columns fit 32 bits (N < 2^31): the window test and column offsets stay 32-bit
  const int gn = (int)col_w + c8;
  // the output's column window (multiples of 8: an octet is wholly in or out)
  const int valid = gn >= eo.cb && gn < eo.ce ? min(8, eo.ce - gn) : 0;
  const int gc = gn - eo.cb;  // output (and extra) column
  float xe[2][8], ye[2][8];
  if constexpr (USES_E || USES_T) {
    // RoPE table row of pass p0: one division per call, then a wrap per pass
    int tr0 = 0, tcol = 0;
    if constexpr (USES_T) {
      tr0 = (int)((row0 + r_l + (int64_t)p0 * rp) % p.period);
      tcol = gn % p.hd;
    }
#pragma unroll
    for (int pi = 0; pi < 2; ++pi) {
      const int ps = p0 + pi;
      const int64_t gm = row0 + r_l + ps * rp;
      if (ps >= np || gm >= p.M || valid <= 0) continue;
      if constexpr (USES_E) {
        const int e = eo.e;
        load8(p.extra[e], gm * p.ld_extra[e] + gc, p.extra_dtype[e], p.extra_vec8[e] != 0, valid, xe[pi]);
      } else {
        // head_dim is a multiple of 8, so the octet lies inside one head
        int tr = tr0 + pi * rp;
        while (tr >= p.period) tr -= p.period;
        const int64_t toff = (int64_t)tr * p.hd + tcol;
        const float4 c0 = *(const float4*)(p.rcos + toff), c1 = *(const float4*)(p.rcos + toff + 4);
        const float4 s0 = *(const float4*)(p.rsin + toff), s1 = *(const float4*)(p.rsin + toff + 4);
        xe[pi][0] = c0.x; xe[pi][1] = c0.y; xe[pi][2] = c0.z; xe[pi][3] = c0.w;
        xe[pi][4] = c1.x; xe[pi][5] = c1.y; xe[pi][6] = c1.z; xe[pi][7] = c1.w;
        ye[pi][0] = s0.x; ye[pi][1] = s0.y; ye[pi][2] = s0.z; ye[pi][3] = s0.w;
        ye[pi][4] = s1.x; ye[pi][5] = s1.y; ye[pi][6] = s1.z; ye[pi][7] = s1.w;
      }
    }
  }
#pragma unroll
  for (int pi = 0; pi < 2; ++pi) {
    const int ps = p0 + pi;
    const int r16 = r_l + ps * rp;
    const int64_t gm = row0 + r16;
    if (ps >= np || gm >= p.M || valid <= 0) continue;
    const float rr = SUMSQ ? rsrow[r16] : 1.f;
    const float* srow = wsl + r16 * ws;
    float a[8], v[8];
    {
      const float4 a0 = *(const float4*)(srow + aoff + c8), a1 = *(const float4*)(srow + aoff + c8 + 4);
      a[0] = a0.x; a[1] = a0.y; a[2] = a0.z; a[3] = a0.w; a[4] = a1.x; a[5] = a1.y; a[6] = a1.z; a[7] = a1.w;
    }
    if (sa) {
#pragma unroll
      for (int i = 0; i < 8; ++i) a[i] *= rr;
    }
    if constexpr (OP == TH_EPI_ACC) {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = a[i];
    } else if constexpr (OP == TH_EPI_SILU) {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = a[i] * sigmoidf_(a[i]);
    } else if constexpr (OP == TH_EPI_SWIGLU) {
      const float4 b0 = *(const float4*)(srow + boff + c8), b1 = *(const float4*)(srow + boff + c8 + 4);
      float bb[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
      const float rb = sb ? rr : 1.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = a[i] * sigmoidf_(a[i]) * (bb[i] * rb);
    } else if constexpr (OP == TH_EPI_ROPE || OP == TH_EPI_ROPE_PAIR) {
      float rot[8];
      if constexpr (OP == TH_EPI_ROPE) {
        // partner column within the head, per quad (half a head is a multiple of 4)
        const int half = p.hd >> 1;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const int within = (int)((gn + 4 * q) % p.hd);
          const int pc = within < half ? c8 + 4 * q + half : c8 + 4 * q - half;
          const float sg = within < half ? -1.f : 1.f;
          const float4 r4 = *(const float4*)(srow + aoff + pc);
          const float s2 = sa ? sg * rr : sg;
          rot[4 * q] = r4.x * s2; rot[4 * q + 1] = r4.y * s2; rot[4 * q + 2] = r4.z * s2; rot[4 * q + 3] = r4.w * s2;
        }
      } else {
        const float4 b0 = *(const float4*)(srow + boff + c8), b1 = *(const float4*)(srow + boff + c8 + 4);
        const float bb[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) rot[i] = sb ? bb[i] * rr : bb[i];
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = a[i] * xe[pi][i] + rot[i] * ye[pi][i];
    } else {  // ADD, SOFTPLUS_ADD, MUL
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if constexpr (OP == TH_EPI_MUL) v[i] = a[i] * xe[pi][i];
        else if constexpr (OP == TH_EPI_ADD) v[i] = a[i] + xe[pi][i];
        else v[i] = softplusf_(a[i] + xe[pi][i]);
      }
    }
    store8(eo.ptr, gm * eo.ld + gc, eo.dtype, eo.vec8 != 0, valid, v);
    if (o2 >= 0) {
      const EpiOutK& e2 = p.out[o2];
      store8(e2.ptr, gm * e2.ld + gc, e2.dtype, e2.vec8 != 0, valid, v);
    }
  }
}

// o2 (or -1): the index of a second output with the same values (the fp32
// copy of a bf16 output), stored from the same registers. (An index, not a
// pointer: taking the address of a kernel-argument field would copy the
// whole argument block to scratch memory.)
template <int OP, bool SUMSQ>
__device__ __forceinline__ void epi_slice(const GemmK& p, const EpiOutK& eo, int o2, const float* wsl,
                                          int ws, int aoff, int boff, const float* rsrow, int64_t row0, int64_t col_w,
                                          int r_l, int c8, int np, int rp) {
  // two passes at a time: their global operands load together, and at most 2 x 16
  // of them are live (np = 4 with all loaded up front spilled the 8-wave kernel)
  for (int p0 = 0; p0 < np; p0 += 2)
    epi_pair<OP, SUMSQ>(p, eo, o2, wsl, ws, aoff, boff, rsrow, row0, col_w, r_l, c8, np, rp, p0);
}

// Outputs o and o + 1 compute the same values (same op, operands and column
// window; only the destination differs).
__device__ __forceinline__ bool same_values(const EpiOutK& x, const EpiOutK& y) {
  return x.op == y.op && x.a == y.a && x.b == y.b && x.e == y.e && x.cb == y.cb && x.ce == y.ce;
}

// Every output op over `rows` staged rows of a whole column tile
// (slab[r * srow + i * bn + j] = acc_i(row0 + r, tile_n * bn + j)), the
// direct-loop kernel's epilogue when 256 threads tile it evenly: wave w owns
// the column strip of q8 / 4 octets (q8 = bn / 8) starting at octet w q8 / 4;
// each lane keeps one octet of the strip and walks rows lane / (q8 / 4) +
// k 256 / q8 with the per-wave epilogue's passes (one 16-byte store per pass,
// no per-element index division). A wave skips every output whose column
// window misses its strip, so a tile holding several narrow outputs (a merged
// launch) costs each wave only the outputs it holds. Returns false (nothing
// done) when the tile does not divide so.
template <bool SUMSQ>
__device__ __forceinline__ bool epilogue_octets(const GemmK& p, const float* slab, int srow, int rows, const float* rs,
                                                int64_t row0, int tile_n, int tid) {
  const int bn = p.bn, q8 = bn >> 3;
  if ((bn & 7) != 0 || (q8 & 3) != 0 || 256 % q8 != 0 || rows % (256 / q8) != 0) return false;
  const int rstep = 256 / q8, np = rows / rstep, qw = q8 >> 2;
  const int wave = tid >> 6, lane = tid & 63;
  const int r_l = lane / qw, c8 = (wave * qw + lane - r_l * qw) << 3;
  const int64_t col0 = (int64_t)tile_n * bn;
  // this wave's strip (columns fit 32 bits, N < 2^31)
  const int s0 = (int)col0 + 8 * wave * qw, s1 = s0 + 8 * qw;
  for (int o = 0; o < p.n_out; ++o) {
    const EpiOutK& eo = p.out[o];
    // an fp32 copy right after its bf16 output is stored from the same values
    const int o2 = o + 1 < p.n_out && same_values(eo, p.out[o + 1]) ? o + 1 : -1;
    if (o2 >= 0) ++o;
    if (eo.ce <= s0 || eo.cb >= s1) continue;  // the window misses this wave's strip
    const int aoff = eo.a * bn, boff = eo.b * bn;
#define TH_EPI_CASE(OP_) \
  case OP_: epi_slice<OP_, SUMSQ>(p, eo, o2, slab, srow, aoff, boff, rs, row0, col0, r_l, c8, np, rstep); break
    switch (eo.op) {
      TH_EPI_CASE(TH_EPI_ACC);
      TH_EPI_CASE(TH_EPI_ROPE);
      TH_EPI_CASE(TH_EPI_ROPE_PAIR);
      TH_EPI_CASE(TH_EPI_SILU);
      TH_EPI_CASE(TH_EPI_SWIGLU);
      TH_EPI_CASE(TH_EPI_ADD);
      TH_EPI_CASE(TH_EPI_SOFTPLUS_ADD);
      default: epi_slice<TH_EPI_MUL, SUMSQ>(p, eo, o2, slab, srow, aoff, boff, rs, row0, col0, r_l, c8, np, rstep); break;
    }
#undef TH_EPI_CASE
  }
  return true;
}


// Evaluate every output op for the `rows` slab rows staged in LDS.
// slab[r * srow + i * bn + j] = acc_i(row0 + r, tile_n * bn + j).
__device__ __forceinline__ void epilogue_slab(const GemmK& p, const float* slab, int srow, int rows,
                              const float* rs, int64_t row0, int tile_n, int tid) {
  const int bn = p.bn;
  const int q4 = bn >> 2;
  const int units = rows * q4;
  const int64_t col0 = (int64_t)tile_n * bn;
  for (int o = 0; o < p.n_out; ++o) {
    const EpiOutK& eo = p.out[o];
    if (eo.ce <= col0 || eo.cb >= col0 + bn) continue;  // the output's window misses this tile
    const int op = eo.op;
    const int ia = eo.a, ib = eo.b;
    const float sa = 1.f, sb = 1.f;
    const bool scale_a = (p.rscale_mask >> ia) & 1u;
    const bool scale_b = ib >= 0 && ((p.rscale_mask >> ib) & 1u);
    for (int u = tid; u < units; u += 256) {
      const int r = u / q4;
      const int j = (u - r * q4) << 2;
      const int64_t gm = row0 + r;
      const int64_t gn = col0 + j;
      if (gm >= p.M || gn < eo.cb || gn >= eo.ce) continue;
      const int valid = (int)min((int64_t)4, (int64_t)eo.ce - gn);
      const int64_t gc = gn - eo.cb;  // output (and extra) column
      const float rr = p.sumsq ? rs[r] : 1.f;
      const float* srow_p = slab + r * srow;
      float4 a = *(const float4*)(srow_p + ia * bn + j);
      if (scale_a) { a.x *= rr; a.y *= rr; a.z *= rr; a.w *= rr; }
      float4 v;
      switch (op) {
        case TH_EPI_ACC:
          v = a;
          break;
        case TH_EPI_ROPE:
        case TH_EPI_ROPE_PAIR: {
          float4 rot;
          if (op == TH_EPI_ROPE) {
            const int hd = p.hd, half = hd >> 1;
            const int within = (int)(gn % hd);
            const int pj = within < half ? j + half : j - half;
            const float sg = within < half ? -1.f : 1.f;
            rot = *(const float4*)(srow_p + ia * bn + pj);
            const float s2 = scale_a ? sg * rr : sg;
            rot.x *= s2; rot.y *= s2; rot.z *= s2; rot.w *= s2;
          } else {
            rot = *(const float4*)(srow_p + ib * bn + j);
            if (scale_b) { rot.x *= rr; rot.y *= rr; rot.z *= rr; rot.w *= rr; }
          }
          const int64_t toff = (gm % p.period) * p.hd + (gn % p.hd);
          const float4 c = *(const float4*)(p.rcos + toff);
          const float4 s = *(const float4*)(p.rsin + toff);
          v.x = a.x * c.x + rot.x * s.x;
          v.y = a.y * c.y + rot.y * s.y;
          v.z = a.z * c.z + rot.z * s.z;
          v.w = a.w * c.w + rot.w * s.w;
          break;
        }
        case TH_EPI_SILU:
          v.x = a.x * sigmoidf_(a.x);
          v.y = a.y * sigmoidf_(a.y);
          v.z = a.z * sigmoidf_(a.z);
          v.w = a.w * sigmoidf_(a.w);
          break;
        case TH_EPI_SWIGLU: {
          float4 b = *(const float4*)(srow_p + ib * bn + j);
          if (scale_b) { b.x *= rr; b.y *= rr; b.z *= rr; b.w *= rr; }
          v.x = a.x * sigmoidf_(a.x) * b.x;
          v.y = a.y * sigmoidf_(a.y) * b.y;
          v.z = a.z * sigmoidf_(a.z) * b.z;
          v.w = a.w * sigmoidf_(a.w) * b.w;
          break;
        }
        case TH_EPI_ADD:
        case TH_EPI_SOFTPLUS_ADD:
        case TH_EPI_MUL: {
          const int e = eo.e;
          const float4 x = load4(p.extra[e], gm * p.ld_extra[e] + gc, p.extra_dtype[e],
                                 p.extra_vec[e] != 0, valid);
          if (op == TH_EPI_MUL) {
            v.x = a.x * x.x; v.y = a.y * x.y; v.z = a.z * x.z; v.w = a.w * x.w;
          } else {
            v.x = a.x + x.x; v.y = a.y + x.y; v.z = a.z + x.z; v.w = a.w + x.w;
            if (op == TH_EPI_SOFTPLUS_ADD) {
              v.x = softplusf_(v.x); v.y = softplusf_(v.y); v.z = softplusf_(v.z); v.w = softplusf_(v.w);
            }
          }
          break;
        }
        default:
          v = a;
          break;
      }
      (void)sa; (void)sb;
      store4(eo.ptr, gm * eo.ld + gc, eo.dtype, eo.vec != 0, valid, v);
    }
  }
}

__device__ __forceinline__ float sumsq8_bf16(uint4 w) {
  float s = 0.f;
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float lo = __uint_as_float(ws[q] << 16);
    const float hi = __uint_as_float(ws[q] & 0xffff0000u);
    s += lo * lo + hi * hi;
  }
  return s;
}

// Sum of squares of an MFMA operand fragment (8 bf16) with v_dot2_f32_bf16:
// each bf16 product is exact in fp32, accumulation is fp32.
__device__ __forceinline__ float sumsq8_dot(bf16x8_t v, float acc) {
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 0, 1), __builtin_shufflevector(v, v, 0, 1), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 2, 3), __builtin_shufflevector(v, v, 2, 3), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 4, 5), __builtin_shufflevector(v, v, 4, 5), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 6, 7), __builtin_shufflevector(v, v, 6, 7), acc, false);
  return acc;
}

// --------------------------------------------------------------- bf16 MFMA
template <int BM, int BNC>
__global__ void __launch_bounds__(256, 1) gemm_bf16_kernel(GemmK p) {
  constexpr int BK = 64;
  constexpr int WM = BM / 2, WN = BNC / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int AC = BM / 32, BC = BNC / 32;  // 16-byte chunks per thread
  constexpr int TILE_BYTES = (BM + BNC) * BK * 2;
  constexpr int SROW = BNC + 8;
  constexpr int EPI_BYTES = WM * SROW * 4;
  constexpr int MAIN_BYTES = 2 * TILE_BYTES;
  constexpr int BODY = MAIN_BYTES > EPI_BYTES ? MAIN_BYTES : EPI_BYTES;
  __shared__ __attribute__((aligned(16))) char smem[BODY + BM * 4];
  float* rs = (float*)(smem + BODY);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  int tmi, tni;
  map_tile(p.tiles_m, p.tiles_n, tmi, tni);
  const int64_t m0 = (int64_t)tmi * BM;
  const uint16_t* A = (const uint16_t*)p.A;
  const uint16_t* B = (const uint16_t*)p.B + (int64_t)tni * BNC * p.ldb;
  const int lrow = tid >> 3, lch = tid & 7;
  const int nk = (int)((p.K + BK - 1) / BK);

  uint4 ra[AC], rb[BC];
  float ss[AC];
  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < AC; ++i) ss[i] = 0.f;
#pragma unroll
  for (int t = 0; t < TM; ++t)
#pragma unroll
    for (int u = 0; u < TN; ++u)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[t][u][r] = 0.f;

  auto gload = [&](int kt) {
    const int64_t k = (int64_t)kt * BK + lch * 8;
    const bool kin = k < p.K;
#pragma unroll
    for (int i = 0; i < AC; ++i) {
      const int64_t r = m0 + lrow + 32 * i;
      ra[i] = (kin && r < p.M) ? *(const uint4*)(A + r * p.lda + k) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < BC; ++i)
      rb[i] = kin ? *(const uint4*)(B + (int64_t)(lrow + 32 * i) * p.ldb + k) : make_uint4(0, 0, 0, 0);
  };
  auto sstore = [&](int buf) {
    char* sa = smem + buf * TILE_BYTES;
    char* sb = sa + BM * BK * 2;
    const int sw = lch ^ (lrow & 7);
#pragma unroll
    for (int i = 0; i < AC; ++i) *(uint4*)(sa + (lrow + 32 * i) * 128 + (sw << 4)) = ra[i];
#pragma unroll
    for (int i = 0; i < BC; ++i) *(uint4*)(sb + (lrow + 32 * i) * 128 + (sw << 4)) = rb[i];
    if (p.sumsq) {
#pragma unroll
      for (int i = 0; i < AC; ++i) ss[i] += sumsq8_bf16(ra[i]);
    }
  };
  auto compute = [&](int buf) {
    const char* sa = smem + buf * TILE_BYTES;
    const char* sb = sa + BM * BK * 2;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int c = ((ks * 2 + (lane >> 5)) ^ (lane & 7)) << 4;
      bf16x8_t af[TM], bfv[TN];
#pragma unroll
      for (int t = 0; t < TM; ++t)
        af[t] = *(const bf16x8_t*)(sa + (wm * WM + t * 32 + (lane & 31)) * 128 + c);
#pragma unroll
      for (int u = 0; u < TN; ++u)
        bfv[u] = *(const bf16x8_t*)(sb + (wn * WN + u * 32 + (lane & 31)) * 128 + c);
#pragma unroll
      for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int u = 0; u < TN; ++u)
          acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[t], bfv[u], acc[t][u], 0, 0, 0);
    }
  };

  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) gload(kt + 1);
    compute(cur);
    if (kt + 1 < nk) sstore(cur ^ 1);
    __syncthreads();
  }

  if (p.sumsq) {
#pragma unroll
    for (int i = 0; i < AC; ++i) {
      float v = ss[i];
      v += __shfl_xor(v, 1);
      v += __shfl_xor(v, 2);
      v += __shfl_xor(v, 4);
      if (lch == 0) {
        const int r = lrow + 32 * i;
        const int64_t gr = m0 + r;
        v = row_sumsq(p, gr, v);
        rs[r] = rsqrtf(v * p.inv_k + p.eps);
        if (p.sumsq_out && tni == 0 && gr < p.M) p.sumsq_out[gr] = v;
      }
    }
  }

  float* slab = (float*)smem;
  // (not unrolled: the accumulator indices inside are constant either way, and the
  // epilogue calls in the body are too large for the unroller)
  for (int s = 0; s < 2; ++s) {
    if (wm == s) {
#pragma unroll
      for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int u = 0; u < TN; ++u)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = t * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            const int col = wn * WN + u * 32 + (lane & 31);
            slab[row * SROW + col] = acc[t][u][r];
          }
    }
    __syncthreads();
    epilogue_slab(p, slab, SROW, WM, rs + s * WM, m0 + s * WM, tni, tid);
    __syncthreads();
  }
}

// ------------------------------------------------- bf16 MFMA, direct-to-LDS
// Same tiling and epilogue as gemm_bf16_kernel, with the operand tiles
// streamed from HBM straight into LDS by global_load_lds_dwordx4 (gfx950):
// no staging VGPRs and no ds_write. Requires K % 64 == 0. (A wave issues the
// global form about 1.5x as fast as buffer_load ... lds, measured: one 1 KB
// load per ~80 cycles against ~120.)
//
// LDS layout: row R of a tile holds its 8 16-byte K chunks with chunk c in
// slot c ^ g(R), g(R) = (R & 7) ^ ((R >> 3) & 1). An MFMA fragment read (32
// consecutive rows, one chunk) then touches 16 distinct bank quads in every
// group of 16 lanes (64 banks x 4 bytes) and 8 distinct ones in every group of
// 8 lanes (32 banks): no bank conflicts under either service pattern.
// LDS fill: the wave's i-th load of a tile writes 1 KB = LDS rows
// 32*i + 8*wave .. +8 (128 bytes each); lane l lands in row +l/8, slot l%8, so
// it fetches global chunk (l%8) ^ g(row) = (l%8) ^ (l/8) ^ (wave&1). Rows of A
// past M re-read row M-1: in bounds, and the epilogue stores no row past M.
//
// Pipeline (2 stages): the loads of tile kt+1 are in flight during tile kt.
// Within a tile the fragments of step ks+1 are read from LDS while the MFMAs of
// step ks run; the barrier sits in the middle of the last step, after which the
// first fragments of tile kt+1 are read and the loads of tile kt+2 issued into
// the stage everyone has just finished reading.

// Wait until at most n tiles of PER loads each are still in flight (n < 8,
// n PER < 64).
template <int PER>
__device__ __forceinline__ void wait_tiles(int n) {
  switch (n) {
    case 0: wait_vmcnt<0>(); break;
    case 1: wait_vmcnt<PER>(); break;
    case 2: wait_vmcnt<(2 * PER < 64 ? 2 * PER : 63)>(); break;
    case 3: wait_vmcnt<(3 * PER < 64 ? 3 * PER : 63)>(); break;
    case 4: wait_vmcnt<(4 * PER < 64 ? 4 * PER : 63)>(); break;
    case 5: wait_vmcnt<(5 * PER < 64 ? 5 * PER : 63)>(); break;
    case 6: wait_vmcnt<(6 * PER < 64 ? 6 * PER : 63)>(); break;
    default: wait_vmcnt<(7 * PER < 64 ? 7 * PER : 63)>(); break;
  }
}

template <int BM, int BNC, bool SUMSQ, int STAGES>
__global__ void __launch_bounds__(256, 1) gemm_bf16_dl_kernel(GemmK p) {
#if defined(__HIP_DEVICE_COMPILE__)  // gfx950 LDS-load builtins exist only in the device pass
  constexpr int WM = BM / 2, WN = BNC / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int LA = BM / 32, LB = BNC / 32;  // 1 KB loads per wave per tile
  constexpr int STAGE = (BM + BNC) * 128;
  constexpr int SROW = BNC + 8;
  constexpr int EPI_BYTES = WM * SROW * 4;
  constexpr int MAIN_BYTES = STAGES * STAGE;
  static_assert(STAGES >= 2 && STAGES <= 8 && (STAGES - 1) * (LA + LB) < 64, "stage count");
  constexpr int BODY = MAIN_BYTES > EPI_BYTES ? MAIN_BYTES : EPI_BYTES;
  constexpr int NMF = TM * TN;
  // the row scales: at the end of the stages when that is clear of the
  // epilogue's slab (they are stored after the main loop's last reads, past a
  // barrier), so that a block within 80 KiB takes no extra LDS
  constexpr int RS_OFF = BODY - BM * 4 >= EPI_BYTES ? BODY - BM * 4 : BODY;
  __shared__ __attribute__((aligned(16))) char smem[RS_OFF + BM * 4];
  float* rs = (float*)(smem + RS_OFF);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  int tmi, tni;
  map_tile(p.tiles_m, p.tiles_n, tmi, tni);
  const int64_t m0 = (int64_t)tmi * BM;
  const int arows = (int)min((int64_t)BM, p.M - m0);
  // Uniform base pointers plus per-lane 32-bit byte offsets of each load's row;
  // lhs rows past M re-read row M-1 (in bounds; their results are never stored).
  const char* ga = (const char*)p.A + m0 * p.lda * 2;
  const char* gb = (const char*)p.B + (int64_t)tni * BNC * p.ldb * 2;
  const int lrow = lane >> 3;
  const uint32_t chunk = (uint32_t)(((lane & 7) ^ lrow ^ (wave & 1)) << 4);
  uint32_t voa[LA], vob[LB];
#pragma unroll
  for (int i = 0; i < LA; ++i) voa[i] = (uint32_t)(min(32 * i + 8 * wave + lrow, arows - 1) * p.lda * 2) + chunk;
#pragma unroll
  for (int i = 0; i < LB; ++i) vob[i] = (uint32_t)((32 * i + 8 * wave + lrow) * p.ldb * 2) + chunk;
  const int nk = (int)(p.K / 64);

  // (dma_load16: untracked by the compiler, covered by the wait_tiles below)
  const uint32_t lds0 = (uint32_t)(uintptr_t)smem;
  auto issue_tile = [&](int kt, int st) {
    const uint32_t sa = lds0 + st * STAGE;
    const uint32_t sb = sa + BM * 128;
    const int64_t kofs = (int64_t)kt * 128;
#pragma unroll
    for (int i = 0; i < LA; ++i) dma_load16(ga + kofs, voa[i], sa + (4 * i + wave) * 1024);
#pragma unroll
    for (int i = 0; i < LB; ++i) dma_load16(gb + kofs, vob[i], sb + (4 * i + wave) * 1024);
  };

  bf16x8_t fa[2][TM], fb[2][TN];
  f32x16_t acc[TM][TN];
  float ss[TM];
#pragma unroll
  for (int t = 0; t < TM; ++t) {
    ss[t] = 0.f;
#pragma unroll
    for (int u = 0; u < TN; ++u)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[t][u][r] = 0.f;
  }

  auto read_frags = [&](int st, int ks, int slot) {
    const char* sa = smem + st * STAGE;
    const char* sb = sa + BM * 128;
    const int c = ((ks * 2 + (lane >> 5)) ^ (lane & 7) ^ ((lane >> 3) & 1)) << 4;
#pragma unroll
    for (int t = 0; t < TM; ++t) fa[slot][t] = *(const bf16x8_t*)(sa + (wm * WM + t * 32 + (lane & 31)) * 128 + c);
#pragma unroll
    for (int u = 0; u < TN; ++u) fb[slot][u] = *(const bf16x8_t*)(sb + (wn * WN + u * 32 + (lane & 31)) * 128 + c);
  };
  auto mfmas = [&](int slot, int lo, int hi) {
#pragma unroll
    for (int i = 0; i < NMF; ++i) {
      if (i < lo || i >= hi) continue;
      const int t = i / TN, u = i % TN;
      acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[slot][t], fb[slot][u], acc[t][u], 0, 0, 0);
    }
  };
  // The two waves that share A rows (wn = 0, 1) split the row sums of squares:
  // wave wn accumulates the 32-row groups t with t % 2 == wn.
  auto sumsq_frags = [&](int slot) {
    if constexpr (SUMSQ) {
#pragma unroll
      for (int t = 0; t < TM; ++t)
        if ((t & 1) == wn) ss[t] = sumsq8_dot(fa[slot][t], ss[t]);
    }
  };

  // K tile j lives in stage j % STAGES; the first STAGES tiles start at once.
  const int pre = min(STAGES, nk);
  for (int j = 0; j < pre; ++j) issue_tile(j, j);
  wait_tiles<LA + LB>(pre - 1);
  __syncthreads();
  read_frags(0, 0, 0);

  // sched_barrier(0) fences keep the compiler from sinking a fragment read
  // next to the MFMA that consumes it: every read is issued one full step
  // (NMF MFMAs) ahead of its use.
  for (int kt = 0; kt < nk; ++kt) {
    const int st = kt % STAGES;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int slot = ks & 1;
      if (ks < 3) {
        read_frags(st, ks + 1, slot ^ 1);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(slot, 0, NMF);
        sumsq_frags(slot);
        __builtin_amdgcn_sched_barrier(0);
      } else {
        mfmas(slot, 0, NMF / 2);
        __builtin_amdgcn_sched_barrier(0);
        if (kt + 1 < nk) {
          // tile kt+1 must have landed; tiles kt+2 .. kt+STAGES-1 may still be in flight
          wait_tiles<LA + LB>(max(0, min(STAGES - 2, nk - 2 - kt)));
          __syncthreads();
          read_frags((kt + 1) % STAGES, 0, 0);
          // every wave has read all of stage st: refill it with tile kt+STAGES
          if (kt + STAGES < nk) issue_tile(kt + STAGES, st);
        }
        __builtin_amdgcn_sched_barrier(0);
        mfmas(slot, NMF / 2, NMF);
        sumsq_frags(slot);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

  float rsv[TM];
  if constexpr (SUMSQ) {
#pragma unroll
    for (int t = 0; t < TM; ++t) {
      const int64_t gr = m0 + wm * WM + t * 32 + (lane & 31);
      const float v = row_sumsq(p, gr, ss[t] + __shfl_xor(ss[t], 32));
      rsv[t] = rsqrtf(v * p.inv_k + p.eps);
      if ((t & 1) == wn && lane < 32) {
        if (p.sumsq_out && tni == 0 && gr < p.M) p.sumsq_out[gr] = v;
      }
    }
  }
  // (barriers for LDS reuse only: the global stores drain meanwhile)
  lds_barrier();
  if constexpr (SUMSQ) {
#pragma unroll
    for (int t = 0; t < TM; ++t)
      if ((t & 1) == wn && lane < 32) rs[wm * WM + t * 32 + lane] = rsv[t];
  }

  float* slab = (float*)smem;
  // (not unrolled: the accumulator indices inside are constant either way, and the
  // epilogue calls in the body are too large for the unroller)
  for (int s = 0; s < 2; ++s) {
    if (wm == s) {
#pragma unroll
      for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int u = 0; u < TN; ++u)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = t * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            const int col = wn * WN + u * 32 + (lane & 31);
            slab[row * SROW + col] = acc[t][u][r];
          }
    }
    lds_barrier();
    if (!epilogue_octets<SUMSQ>(p, slab, SROW, WM, rs + s * WM, m0 + s * WM, tni, tid))
      epilogue_slab(p, slab, SROW, WM, rs + s * WM, m0 + s * WM, tni, tid);
    if (s == 0) lds_barrier();
  }
#endif
}

// ------------------------- bf16 MFMA, persistent blocks + per-wave epilogue
// One block per CU walks the output tiles L = blockIdx.x, +gridDim.x, ... in
// map_tile order (each XCD keeps its contiguous tile range). Per tile the main
// loop is the direct-to-LDS loop above, except that wave (wm, wn) computes
// rows wm*WM .. of the wn-th column half of EVERY accumulator: subtile u holds
// accumulator u % n_acc, columns wn*bn/2 + (u / n_acc)*32 .. +32. An output op
// that combines accumulators (SWIGLU, ROPE_PAIR) or rotates within a head
// (ROPE with head_dim | bn/2) then finds every operand in its own wave, so the
// epilogue needs no block barrier: each wave transposes 16 rows at a time
// through a private slice of LDS stage 1 and writes 4 consecutive columns per
// lane. Before the epilogue starts, the next tile's first K tile is already
// streaming into stage 0, so its latency hides behind the epilogue.
//
// NW = 8 waves (two per SIMD, at most 256 registers each) split the rows in
// four: each wave holds 64 rows of its column half. A wave issues one global
// load per ~120 cycles whatever its width, and in order, so with one wave per
// SIMD the loads of a K tile hold back that SIMD's MFMAs; with two, one wave
// issues MFMAs while the other waits on its loads.
// NACC (the number of accumulators, p.n_acc) is a template argument so that
// every fragment's LDS row offset is a constant and the address registers of
// the main loop stay few.
// ASPLIT (two accumulators): wave column half wn holds all bn columns of
// accumulator wn instead, so a RoPE head as wide as bn stays in one wave; every
// output then reads one accumulator and is written by the waves that hold it.
template <int BM, int BNC, bool SUMSQ, int NW, int NACC, bool ASPLIT = false>
__global__ void __launch_bounds__(64 * NW, 1) gemm_bf16_pk_kernel(GemmK p) {
#if defined(__HIP_DEVICE_COMPILE__)  // gfx950 LDS-load builtins exist only in the device pass
  static_assert(NW == 4 || NW == 8, "4 or 8 waves");
  constexpr int WM = BM / (NW / 2), WN = BNC / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int LR = 8 * NW;                 // rows covered by one load of every wave
  constexpr int LA = BM / LR, LB = BNC / LR;  // 1 KB loads per wave per K tile
  static_assert(LA * LR == BM && LB * LR == BNC, "tile rows must be a multiple of 8 per wave");
  constexpr int STAGE = (BM + BNC) * 128;
  constexpr int NMF = TM * TN;
  constexpr int NLD = LA + LB, HLD = NLD / 2;  // loads per K tile; the first HLD go out with step 3
  constexpr int WS = WN + 8;                 // epilogue slice row stride (floats)
  constexpr int SLICE = 16 * WS * 4;         // bytes per wave: 16 rows
  // the slices start at stage 1 (free while the next tile's K tile 0 streams into stage 0)
  constexpr int BODY = STAGE + NW * SLICE > 2 * STAGE ? STAGE + NW * SLICE : 2 * STAGE;
  __shared__ __attribute__((aligned(16))) char smem[BODY + BM * 4];
  float* rsx = (float*)(smem + BODY);  // row scales of the current tile

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  constexpr int n_acc = NACC, bn = BNC / NACC, hbn = bn >> 1;
  static_assert(bn * NACC == BNC && hbn % 32 == 0, "column tile per accumulator");
  static_assert(!ASPLIT || NACC == 2, "the accumulator split needs two accumulators");
  constexpr int wcols = ASPLIT ? bn : hbn;  // columns of one accumulator held by a wave
  const int tiles = p.tiles_m * p.tiles_n;
  const int nk = (int)(p.K / 64);

  // subtile u: LDS row of its B fragment and its column in the epilogue slice
  int brow[TN], lcol[TN];
#pragma unroll
  for (int u = 0; u < TN; ++u) {
    if constexpr (ASPLIT) {
      brow[u] = wn * bn + u * 32 + (lane & 31);
      lcol[u] = u * 32;
    } else {
      const int a = u % n_acc, c32 = u / n_acc;
      brow[u] = a * bn + wn * hbn + c32 * 32 + (lane & 31);
      lcol[u] = a * hbn + c32 * 32;
    }
  }

  // Load i of a wave fills LDS rows LR*i + 8*wave .. +8 (1 KB); row R's chunk
  // slot is c ^ g(R) with g(R) = (R & 7) ^ ((R >> 3) & 1) = (lane >> 3) ^ (wave & 1).
  const int lrow = lane >> 3;
  const uint32_t chunk = (uint32_t)(((lane & 7) ^ lrow ^ (wave & 1)) << 4);
  // rhs load i reads rows LR i + 8 wave + lane / 8: a uniform step of LR rows
  // per load on top of one per-lane offset (the packed rhs is padded to whole
  // column tiles, so no row needs clamping)
  uint32_t voa[LA];
#pragma unroll
  for (int i = 0; i < LA; ++i) voa[i] = (uint32_t)((LR * i + 8 * wave + lrow) * p.lda * 2) + chunk;
  const uint32_t vob0 = (uint32_t)((8 * wave + lrow) * p.ldb * 2) + chunk;
  const int64_t bstep = (int64_t)LR * p.ldb * 2;

  // Operand rows of tile L: uniform base pointers (lhs rows m0.., rhs rows
  // tn*BNC..) plus the per-lane 32-bit offsets above. lhs rows past M re-read
  // row M-1, which is in bounds; their results are never stored. The offsets
  // of a new tile are set only after every load of the previous one landed.
  auto tile_rsrc = [&](int L, int& tm, int& tn, const char*& ga, const char*& gb) {
    map_tile_id(L, p.tiles_m, p.tiles_n, tm, tn);
    const int64_t m0 = (int64_t)tm * BM;
    const int arows = (int)min((int64_t)BM, p.M - m0);
    ga = (const char*)p.A + m0 * p.lda * 2;
    gb = (const char*)p.B + (int64_t)tn * BNC * p.ldb * 2;
#pragma unroll
    for (int i = 0; i < LA; ++i) voa[i] = (uint32_t)(min(LR * i + 8 * wave + lrow, arows - 1) * p.lda * 2) + chunk;
  };
  // Load i of K tile kt into stage st: i < LA fills lhs rows, the rest rhs
  // rows. global_load_lds: a wave issues these about 1.5x as fast as the
  // buffer-descriptor form.
  // Every address is a uniform base (tile, K tile and, for the rhs, the load's
  // row step; SGPRs) plus a 32-bit per-lane offset (dma_load16: the compiler
  // neither tracks these loads nor lets them turn its LDS-read waits into
  // waits for every read; the explicit waits below cover them).
  const uint32_t lds0 = (uint32_t)(uintptr_t)smem;
  auto issue_one = [&](const char* ga, const char* gb, int kt, int st, int i) {
    const uint32_t sa = lds0 + st * STAGE;
    const int64_t kofs = (int64_t)kt * 128;
    if (i < LA)
      dma_load16(ga + kofs, voa[i < LA ? i : 0], sa + (NW * i + wave) * 1024);
    else
      dma_load16(gb + kofs + (int64_t)(i >= LA ? i - LA : 0) * bstep, vob0, sa + BM * 128 + (NW * (i - LA) + wave) * 1024);
  };
  auto issue_tile = [&](const char* ga, const char* gb, int kt, int st) {
#pragma unroll
    for (int i = 0; i < NLD; ++i) issue_one(ga, gb, kt, st, i);
  };
  auto issue_half = [&](const char* ga, const char* gb, int kt, int st) {
#pragma unroll
    for (int i = 0; i < HLD; ++i) issue_one(ga, gb, kt, st, i);
  };

  bf16x8_t fa[2][TM], fb[2][TN];
  f32x16_t acc[TM][TN];
  static_assert(TM % 2 == 0, "the two column-half waves split the 32-row groups");
  float ss[TM / 2];  // ss[j]: row group t = 2j + wn
  auto read_frags = [&](int st, int ks, int slot) {
    const char* sa = smem + st * STAGE;
    const char* sb = sa + BM * 128;
    const int c = ((ks * 2 + (lane >> 5)) ^ (lane & 7) ^ ((lane >> 3) & 1)) << 4;
#pragma unroll
    for (int t = 0; t < TM; ++t) fa[slot][t] = *(const bf16x8_t*)(sa + (wm * WM + t * 32 + (lane & 31)) * 128 + c);
#pragma unroll
    for (int u = 0; u < TN; ++u) fb[slot][u] = *(const bf16x8_t*)(sb + brow[u] * 128 + c);
  };
  auto mfmas = [&](int slot, int lo, int hi) {
#pragma unroll
    for (int i = 0; i < NMF; ++i) {
      if (i < lo || i >= hi) continue;
      const int t = i / TN, u = i % TN;
      acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[slot][t], fb[slot][u], acc[t][u], 0, 0, 0);
    }
  };
  // MFMAs lo .. hi with loads l0 .. l1 of K tile kt (into stage st) spread
  // evenly between them, in this order: a wave issues in order, so a burst of
  // loads would hold back the MFMAs behind it until the load queue drains.
  auto mfmas_ld = [&](int slot, int lo, int hi, const char* ra, const char* rb, int kt, int st, int l0, int l1) {
#pragma unroll
    for (int i = 0; i < NMF; ++i) {
      if (i < lo || i >= hi) continue;
      const int t = i / TN, u = i % TN;
      acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[slot][t], fb[slot][u], acc[t][u], 0, 0, 0);
#pragma unroll
      for (int j = 0; j < NLD; ++j)
        if (j >= l0 && j < l1 && (j - l0) * (hi - lo) / (l1 - l0) == i - lo) issue_one(ra, rb, kt, st, j);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // wave wn accumulates the row sums of squares of the 32-row groups t % 2 == wn
  // (a select, not a branch, so the MFMA sequence stays one basic block)
  auto sumsq_frags = [&](int slot) {
    if constexpr (SUMSQ) {
#pragma unroll
      for (int j = 0; j < TM / 2; ++j) ss[j] = sumsq8_dot(wn ? fa[slot][2 * j + 1] : fa[slot][2 * j], ss[j]);
    }
  };

  int L = blockIdx.x;
  if (L >= tiles) return;
  int tmi, tni;
  const char *rsa, *rsb;
  tile_rsrc(L, tmi, tni, rsa, rsb);
  issue_tile(rsa, rsb, 0, 0);
  if (nk > 1) issue_half(rsa, rsb, 1, 1);

  char* slice = smem + STAGE + wave * SLICE;
  float* wsl = (float*)slice;

  for (;;) {
    // K tile 0 of tile L is in flight into stage 0 (and half of K tile 1 into stage 1)
    if (nk > 1)
      wait_vmcnt<HLD>();
    else
      wait_vmcnt<0>();
    // (LDS-only barrier: a __syncthreads would also wait for the half K tile
    // just issued; the previous tile's slice reads completed before the last one)
    barrier_keep_loads();
    read_frags(0, 0, 0);
#pragma unroll
    for (int j = 0; j < TM / 2; ++j) ss[j] = 0.f;
#pragma unroll
    for (int t = 0; t < TM; ++t) {
#pragma unroll
      for (int u = 0; u < TN; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][u][r] = 0.f;
    }

    // One K tile. K tile kt+2 goes into stage kt & 1 once every wave is past
    // the barrier of tile kt: loads 0 .. HLD with the last MFMAs of tile kt, the
    // rest with the first step of tile kt+1 (tile 1: its first half was issued
    // with tile 0). Past the last K tile the first-half loads fetch tile nk-1
    // again into the stage that is no longer read; the last tile issues nothing
    // and has no successor. STEADY is compile-time: two straight-line bodies.
    auto ktile = [&](int kt, auto steady) __attribute__((always_inline)) {
      constexpr bool STEADY = decltype(steady)::value;
      const int st = kt & 1;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int slot = ks & 1;
        if (ks < 3) {
          read_frags(st, ks + 1, slot ^ 1);
          __builtin_amdgcn_sched_barrier(0);
          if (STEADY && ks == 0)
            mfmas_ld(slot, 0, NMF, rsa, rsb, kt + 1, st ^ 1, HLD, NLD);
          else
            mfmas(slot, 0, NMF);
          sumsq_frags(slot);
          __builtin_amdgcn_sched_barrier(0);
        } else {
          mfmas(slot, 0, NMF / 2);
          __builtin_amdgcn_sched_barrier(0);
          if constexpr (STEADY) {
            wait_vmcnt<0>();
            lds_barrier();
            read_frags(st ^ 1, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            mfmas_ld(slot, NMF / 2, NMF, rsa, rsb, min(kt + 2, nk - 1), st, 0, HLD);
          } else {
            mfmas(slot, NMF / 2, NMF);
          }
          sumsq_frags(slot);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    };
    for (int kt = 0; kt < nk - 1; ++kt) ktile(kt, std::true_type{});
    ktile(nk - 1, std::false_type{});

    if constexpr (SUMSQ) {
#pragma unroll
      for (int j = 0; j < TM / 2; ++j) {
        float v = ss[j] + __shfl_xor(ss[j], 32);
        if (lane < 32) {
          const int r = wm * WM + (2 * j + wn) * 32 + lane;
          const int64_t gr = (int64_t)tmi * BM + r;
          if constexpr (!ASPLIT) v = row_sumsq(p, gr, v);
          rsx[r] = rsqrtf(v * p.inv_k + p.eps);
          if (p.sumsq_out && tni == 0 && gr < p.M) p.sumsq_out[gr] = v;
        }
      }
    }

    // Every wave is done with both stages (and its last loads, re-fetches into
    // the stage the epilogue slices overlay, have landed); start the next
    // tile's first K tile.
    wait_vmcnt<0>();
    lds_barrier();
    const int Ln = L + (int)gridDim.x;
    const bool more = Ln < tiles;
    int tmn = 0, tnn = 0;
    const char *rsan = rsa, *rsbn = rsb;
    if (more) {
      tile_rsrc(Ln, tmn, tnn, rsan, rsbn);
      issue_tile(rsan, rsbn, 0, 0);
    }

    // ---- epilogue of tile (tmi, tni), wave-private
    const int64_t row_w = (int64_t)tmi * BM + wm * WM;  // first row of this wave
    // Register epilogue: one bf16 SWIGLU output over a tile inside M and the
    // output's column window (the gate/up projection). The gate and up values of
    // an output element sit in the same lane and register of two subtiles, so
    // the product needs no transpose: it is formed from the accumulators and
    // stored in the MFMA C layout, where for a fixed register lanes 0..31 hold
    // 32 consecutive columns of one row (64 contiguous bytes) and lanes 32..63
    // the row 4 below. Same arithmetic, in the same order, as epi_pair.
    bool reg_epi = false;
    if constexpr (NACC == 2 && !ASPLIT) {
      const EpiOutK& e0 = p.out[0];
      const int64_t c0 = (int64_t)tni * bn;
      reg_epi = p.n_out == 1 && e0.op == TH_EPI_SWIGLU && e0.dtype == TH_BF16 && row_w - wm * WM + BM <= p.M &&
                e0.cb <= c0 && e0.ce >= c0 + bn;
      if (reg_epi) {
        const bool swap = e0.a != 0;  // the gate is accumulator slot 1
        const bool sa = SUMSQ && ((p.rscale_mask >> e0.a) & 1u);
        const bool sb = SUMSQ && ((p.rscale_mask >> e0.b) & 1u);
        // uniform base (row_w, the wave's first output column) + one 32-bit per-lane offset
        char* obase = (char*)e0.ptr + (row_w * e0.ld + (c0 + wn * hbn - e0.cb)) * 2;
        const uint32_t lofs = (uint32_t)(((lane >> 5) * 4 * e0.ld + (lane & 31)) * 2);
#pragma unroll
        for (int t = 0; t < TM; ++t) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            // row scales of rows 8q + 4 (lane / 32) + 0..3 of group t
            float4 rr = make_float4(1.f, 1.f, 1.f, 1.f);
            if constexpr (SUMSQ) rr = *(const float4*)(rsx + wm * WM + t * 32 + 8 * q + 4 * (lane >> 5));
            const float rrv[4] = {rr.x, rr.y, rr.z, rr.w};
#pragma unroll
            for (int c32 = 0; c32 < TN / 2; ++c32) {
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                const int r = 4 * q + j;
                const float x0 = acc[t][2 * c32][r], x1 = acc[t][2 * c32 + 1][r];
                float g = swap ? x1 : x0, u = swap ? x0 : x1;
                if (sa) g *= rrv[j];
                const float ub = sb ? u * rrv[j] : u;
                const float v = g * sigmoidf_(g) * ub;
                const int64_t rofs = ((int64_t)(t * 32 + 8 * q + j) * e0.ld + c32 * 32) * 2;
                *(uint16_t*)(obase + rofs + lofs) = f32_to_bf16(v);
              }
            }
          }
        }
      }
    }
    if (!reg_epi) {
    // first column of this wave (in every accumulator it holds)
    const int64_t col_w = (int64_t)tni * bn + (ASPLIT ? 0 : wn * hbn);
    const int qlog = __builtin_ctz((unsigned)(wcols >> 2));  // quads per row = wcols / 4
    // Rows 16*h .. +16 of the 32-row group t go through the slice. The copy out
    // of the accumulators is unrolled per (t, h) so every register index is a
    // constant; the read-back below is an ordinary loop.
    auto write_slice = [&](const f32x16_t(&at)[TN], auto hc) {
      constexpr int H = decltype(hc)::value;
#pragma unroll
      for (int u = 0; u < TN; ++u)
#pragma unroll
        for (int rr = 0; rr < 8; ++rr) {
          const int row16 = 8 * (rr >> 2) + 4 * (lane >> 5) + (rr & 3);
          wsl[row16 * WS + lcol[u] + (lane & 31)] = at[u][H * 8 + rr];
        }
    };
    using H0 = std::integral_constant<int, 0>;
    using H1 = std::integral_constant<int, 1>;
    for (int t = 0; t < TM; ++t) {
      for (int h = 0; h < 2; ++h) {
        switch (t * 2 + h) {
          case 0: write_slice(acc[0], H0{}); break;
          case 1: write_slice(acc[0], H1{}); break;
          case 2: if constexpr (TM > 1) write_slice(acc[1 % TM], H0{}); break;
          case 3: if constexpr (TM > 1) write_slice(acc[1 % TM], H1{}); break;
          case 4: if constexpr (TM > 2) write_slice(acc[2 % TM], H0{}); break;
          case 5: if constexpr (TM > 2) write_slice(acc[2 % TM], H1{}); break;
          case 6: if constexpr (TM > 3) write_slice(acc[3 % TM], H0{}); break;
          default: if constexpr (TM > 3) write_slice(acc[3 % TM], H1{}); break;
        }
        static_assert(TM <= 4, "write_slice cases cover four 32-row groups");
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        const int64_t row0 = row_w + t * 32 + h * 16;
        const float* rsrow = rsx + wm * WM + t * 32 + h * 16;
        const int q8log = qlog - 1;  // octets per row = wcols / 8 (4, 8 or 16)
        const int r_l = lane >> q8log, c8 = (lane & ((1 << q8log) - 1)) << 3;
        const int np = 1 << (q8log - 2), rp = 64 >> q8log;
        for (int o = 0; o < p.n_out; ++o) {
          const EpiOutK& eo = p.out[o];
          // an fp32 copy right after its bf16 output is stored from the same values
          const int o2 = o + 1 < p.n_out && same_values(eo, p.out[o + 1]) ? o + 1 : -1;
          if (o2 >= 0) ++o;
          if (ASPLIT && eo.a != wn) continue;
          if (eo.ce <= col_w || eo.cb >= col_w + wcols) continue;  // the window misses this wave's columns
          const int aoff = ASPLIT ? 0 : eo.a * hbn, boff = ASPLIT ? 0 : eo.b * hbn;
#define TH_EPI_CASE(OP_) \
  case OP_: epi_slice<OP_, SUMSQ>(p, eo, o2, wsl, WS, aoff, boff, rsrow, row0, col_w, r_l, c8, np, rp); break
          switch (eo.op) {
            TH_EPI_CASE(TH_EPI_ACC);
            TH_EPI_CASE(TH_EPI_ROPE);
            TH_EPI_CASE(TH_EPI_ROPE_PAIR);
            TH_EPI_CASE(TH_EPI_SILU);
            TH_EPI_CASE(TH_EPI_SWIGLU);
            TH_EPI_CASE(TH_EPI_ADD);
            TH_EPI_CASE(TH_EPI_SOFTPLUS_ADD);
            default: epi_slice<TH_EPI_MUL, SUMSQ>(p, eo, o2, wsl, WS, aoff, boff, rsrow, row0, col_w, r_l, c8, np, rp); break;
          }
#undef TH_EPI_CASE
        }
        // the next 16 rows overwrite this slice
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
    }

    lds_barrier();  // every wave is done with its stage-1 slice (its stores drain meanwhile)
    } else {
      // the register epilogue used no slice; rsx is rewritten only after the next
      // tile's K loop, past its barriers
    }
    if (!more) break;
    if (nk > 1) issue_half(rsan, rsbn, 1, 1);
    L = Ln;
    tmi = tmn;
    tni = tnn;
    rsa = rsan;
    rsb = rsbn;
  }
  wait_vmcnt<0>();  // no direct-to-LDS load may land after the workgroup ends
#endif
}

// --------------------------------------------------------------- fp32 MFMA
template <int BNC>
__global__ void __launch_bounds__(256, 1) gemm_f32_kernel(GemmK p) {
  constexpr int BM = 64, BK = 16, RSF = 20;  // LDS row stride in floats (80 B)
  constexpr int WM = 32, WN = BNC / 2, TN = WN / 32;
  constexpr int BC = BNC / 64;
  constexpr int TILE_FLOATS = (BM + BNC) * RSF;
  constexpr int SROW = BNC + 8;
  constexpr int EPI_FLOATS = WM * SROW;
  constexpr int MAIN_FLOATS = 2 * TILE_FLOATS;
  constexpr int BODY = MAIN_FLOATS > EPI_FLOATS ? MAIN_FLOATS : EPI_FLOATS;
  __shared__ __attribute__((aligned(16))) float smem[BODY + BM];
  float* rs = smem + BODY;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  int tmi, tni;
  map_tile(p.tiles_m, p.tiles_n, tmi, tni);
  const int64_t m0 = (int64_t)tmi * BM;
  const float* A = (const float*)p.A;
  const float* B = (const float*)p.B + (int64_t)tni * BNC * p.ldb;
  const int lrow = tid >> 2, lch = tid & 3;
  const int nk = (int)((p.K + BK - 1) / BK);

  float4 ra, rb[BC];
  float ss = 0.f;
  f32x16_t acc[TN];
#pragma unroll
  for (int u = 0; u < TN; ++u)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[u][r] = 0.f;

  auto gload = [&](int kt) {
    const int64_t k = (int64_t)kt * BK + lch * 4;
    const bool kin = k < p.K;
    const int64_t r = m0 + lrow;
    ra = (kin && r < p.M) ? *(const float4*)(A + r * p.lda + k) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < BC; ++i)
      rb[i] = kin ? *(const float4*)(B + (int64_t)(lrow + 64 * i) * p.ldb + k) : make_float4(0.f, 0.f, 0.f, 0.f);
  };
  auto sstore = [&](int buf) {
    float* sa = smem + buf * TILE_FLOATS;
    float* sb = sa + BM * RSF;
    *(float4*)(sa + lrow * RSF + lch * 4) = ra;
#pragma unroll
    for (int i = 0; i < BC; ++i) *(float4*)(sb + (lrow + 64 * i) * RSF + lch * 4) = rb[i];
    if (p.sumsq) ss += ra.x * ra.x + ra.y * ra.y + ra.z * ra.z + ra.w * ra.w;
  };
  auto compute = [&](int buf) {
    const float* sa = smem + buf * TILE_FLOATS;
    const float* sb = sa + BM * RSF;
#pragma unroll
    for (int ks = 0; ks < BK / 2; ++ks) {
      const int k = ks * 2 + (lane >> 5);
      const float a = sa[(wm * WM + (lane & 31)) * RSF + k];
#pragma unroll
      for (int u = 0; u < TN; ++u) {
        const float b = sb[(wn * WN + u * 32 + (lane & 31)) * RSF + k];
        acc[u] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[u], 0, 0, 0);
      }
    }
  };

  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) gload(kt + 1);
    compute(cur);
    if (kt + 1 < nk) sstore(cur ^ 1);
    __syncthreads();
  }

  if (p.sumsq) {
    float v = ss;
    v += __shfl_xor(v, 1);
    v += __shfl_xor(v, 2);
    if (lch == 0) {
      rs[lrow] = rsqrtf(v * p.inv_k + p.eps);
      const int64_t gr = m0 + lrow;
      if (p.sumsq_out && tni == 0 && gr < p.M) p.sumsq_out[gr] = v;
    }
  }

  float* slab = smem;
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    if (wm == s) {
#pragma unroll
      for (int u = 0; u < TN; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          const int col = wn * WN + u * 32 + (lane & 31);
          slab[row * SROW + col] = acc[u][r];
        }
    }
    __syncthreads();
    epilogue_slab(p, slab, SROW, WM, rs + s * WM, m0 + s * WM, tni, tid);
    __syncthreads();
  }
}

// ------------------------------------- fp32 MFMA, small grids (split-K in a workgroup)
// A workgroup computes 32 rows x BNC packed columns with NSUB = BNC / 32
// column slices times KS K slices of one wave each (NSUB * KS <= 16 waves), so
// a GEMM of a few hundred rows (the fp32 Llama block: 128 tokens) still runs
// on every SIMD. Each wave multiplies its 32 x 32 subtile over its K slice.
// Operands: per 8-wide K step, lane l takes row l % 32 and the float4 at
// k + 4 (l / 32) (its four components are four k = 2 steps of
// v_mfma_f32_32x32x2f32, the contraction index permuted the same way on both
// sides). They come through a wave-private LDS ring of PD steps filled by
// direct-to-LDS loads (lane l's 16 bytes land at slot + 16 l, which is also
// where it reads them back), so PD steps of loads are in flight with no
// workgroup barrier; explicit vmcnt waits cover the untracked loads. The KS
// partial tiles are then summed through LDS in slice order, and the ordinary
// slab epilogue runs on the first 256 threads.
template <int BNC>
__global__ void __launch_bounds__(1024, 1) gemm_f32_sk_kernel(GemmK p) {
#if defined(__HIP_DEVICE_COMPILE__)  // gfx950 LDS-load instructions exist only in the device pass
  constexpr int NSUB = BNC / 32;
  constexpr int KS = 16 / NSUB > 0 ? 16 / NSUB : 1;
  constexpr int NWV = NSUB * KS, NT = 64 * NWV;
  constexpr int SROW = BNC + 8;
  constexpr int SLAB = 32 * SROW * 4;            // epilogue slab bytes
  constexpr int PART = KS * 32 * BNC * 4;        // partial tiles (after the K loop)
  constexpr int STEP = 2048;                     // one K step of a wave: A then B, 1 KB each
  constexpr int PD = (160 * 1024 - SLAB - 2048) / (NWV * STEP) >= 4 ? 4 : 3;
  constexpr int RING = NWV * PD * STEP;
  constexpr int BODY = RING > PART ? RING : PART;
  __shared__ __attribute__((aligned(16))) char smem[BODY + SLAB];
  __shared__ float ssp[KS * 32];
  __shared__ float rs[32];
  float* part = (float*)smem;
  float* slab = (float*)(smem + BODY);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ns = wave % NSUB, ks = wave / NSUB;
  int tmi, tni;
  map_tile(p.tiles_m, p.tiles_n, tmi, tni);
  const int64_t m0 = (int64_t)tmi * 32;
  const int row = (int)min(m0 + (lane & 31), p.M - 1);  // rows past M re-read row M-1 (never stored)
  const int h4 = 4 * (lane >> 5);
  // K slice of this wave: whole 8-wide steps
  const int64_t kq = (p.K + 8 * KS - 1) / (8 * KS) * 8;
  const int64_t k0 = ks * kq, k1 = min(p.K, k0 + kq);
  const int nsteps = k1 > k0 ? (int)((k1 - k0 + 7) / 8) : 0;
  // per-lane byte offsets from uniform bases (the host keeps both operands under 2^31 bytes);
  // a float4 past the slice re-reads the slice's last one (K % 4 == 0), zeroed where used
  const char* Ab = (const char*)p.A;
  const char* Bb = (const char*)p.B;
  const uint32_t arow = (uint32_t)((int64_t)row * p.lda * 4);
  const uint32_t brow = (uint32_t)(((int64_t)tni * BNC + ns * 32 + (lane & 31)) * p.ldb * 4);
  const int64_t klast = k1 > k0 ? k1 - 4 : 0;
  const uint32_t ring = (uint32_t)(uintptr_t)smem + (uint32_t)(wave * PD * STEP);
  auto issue = [&](int st) {  // step st into ring slot st % PD
    const int64_t k = k0 + 8 * (int64_t)st + h4;
    const uint32_t kb = (uint32_t)(min(k, klast) * 4);
    const uint32_t dst = ring + (uint32_t)((st % PD) * STEP);
    dma_load16(Ab, arow + kb, dst);
    dma_load16(Bb, brow + kb, dst + 1024);
  };
  f32x16_t acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.f;
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < PD; ++j) issue(j);
  for (int st = 0; st < nsteps; ++st) {
    // step st has landed when at most the PD - 1 later steps' loads are in flight
    wait_vmcnt<2 * (PD - 1)>();
    asm volatile("" ::: "memory");
    const char* slotp = smem + wave * PD * STEP + (st % PD) * STEP;
    float4 a = *(const float4*)(slotp + 16 * lane);
    float4 b = *(const float4*)(slotp + 1024 + 16 * lane);
    if (!(k0 + 8 * (int64_t)st + h4 < k1)) a = b = make_float4(0.f, 0.f, 0.f, 0.f);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, b.x, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, b.y, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, b.z, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, b.w, acc, 0, 0, 0);
    ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;  // (used only with sumsq)
    // the slot's reads are consumed (the MFMAs above used them): refill it;
    // past the last step the loads re-read the slice end, so every wait keeps its count
    asm volatile("" ::: "memory");
    issue(st + PD);
  }
  wait_vmcnt<0>();   // no direct-to-LDS load lands after this point
  __syncthreads();   // every wave is done with the rings before they hold the partial tiles
  // partial tile of slice ks: part[ks][row][col], rows 8(r/4) + 4(l/32) + r%4, column l%32
#pragma unroll
  for (int r = 0; r < 16; ++r)
    part[(ks * 32 + 8 * (r >> 2) + h4 + (r & 3)) * BNC + ns * 32 + (lane & 31)] = acc[r];
  if (p.sumsq && ns == 0) {
    const float v = ss + __shfl_xor(ss, 32);
    if (lane < 32) ssp[ks * 32 + lane] = v;
  }
  __syncthreads();
  for (int e = tid; e < 32 * BNC; e += NT) {
    const int r = e / BNC, c = e - r * BNC;
    float v = part[e];
#pragma unroll
    for (int q = 1; q < KS; ++q) v += part[q * 32 * BNC + e];
    slab[r * SROW + c] = v;
  }
  if (p.sumsq && tid < 32) {
    float v = 0.f;
#pragma unroll
    for (int q = 0; q < KS; ++q) v += ssp[q * 32 + tid];
    rs[tid] = rsqrtf(v * p.inv_k + p.eps);
    const int64_t gr = m0 + tid;
    if (p.sumsq_out && tni == 0 && gr < p.M) p.sumsq_out[gr] = v;
  }
  __syncthreads();
  if (tid < 256) epilogue_slab(p, slab, SROW, 32, rs, m0, tni, tid);
#endif
}

// ------------------------- fp32 MFMA, small grids with a workspace (split-K over workgroups)
// Pass 1 (gemm_f32_ksp_kernel): workgroup (tile, g) multiplies 32 rows x BNC
// packed columns over K slice g, one wave per 32 x 32 subtile, with the same
// operand layout and wave-private LDS ring as gemm_f32_sk_kernel, and stores its
// partial tile to part[g][row][column] (rows of the padded row count Mp); the
// column-0 workgroups also store the slice's row sums of squares ssq[g][row].
// Pass 2 (gemm_f32_ksr_kernel): one workgroup per 8 (or 2) rows x BNC columns sums the
// KSG partials in slice order (deterministic) into an LDS slab and runs the
// slab epilogue. Enough pass-1 workgroups to cover the GPU (about one per CU)
// for the fp32 block's GEMMs of 128 rows, which one workgroup per tile cannot.
struct F32Ksp {
  GemmK k;
  float* part;  // [KSG][Mp][Npk]
  float* ssq;   // [KSG][Mp]
  int64_t Mp, Npk, kq;
  int ksg;
};

template <int BNC>
__global__ void __launch_bounds__(BNC * 2) gemm_f32_ksp_kernel(F32Ksp q) {
#if defined(__HIP_DEVICE_COMPILE__)  // gfx950 LDS-load instructions exist only in the device pass
  constexpr int NSUB = BNC / 32, STEP = 2048, PD = 4;
  __shared__ __attribute__((aligned(16))) char smem[NSUB * PD * STEP];
  const GemmK& p = q.k;
  const int lane = threadIdx.x & 63;
  const int ns = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int tmi, tni;
  map_tile(p.tiles_m, p.tiles_n, tmi, tni);
  const int g = blockIdx.y;
  const int64_t m0 = (int64_t)tmi * 32;
  const int row = (int)min(m0 + (lane & 31), p.M - 1);  // rows past M re-read row M-1 (never stored)
  const int h4 = 4 * (lane >> 5);
  const int64_t k0 = g * q.kq, k1 = min(p.K, k0 + q.kq);
  const int nsteps = k1 > k0 ? (int)((k1 - k0 + 7) / 8) : 0;
  const char* Ab = (const char*)p.A;
  const char* Bb = (const char*)p.B;
  const uint32_t arow = (uint32_t)((int64_t)row * p.lda * 4);
  const uint32_t brow = (uint32_t)(((int64_t)tni * BNC + ns * 32 + (lane & 31)) * p.ldb * 4);
  const int64_t klast = k1 > k0 ? k1 - 4 : 0;
  const uint32_t ring = (uint32_t)(uintptr_t)smem + (uint32_t)(ns * PD * STEP);
  auto issue = [&](int st) {  // step st into ring slot st % PD (past the slice: the slice end again)
    const int64_t k = k0 + 8 * (int64_t)st + h4;
    const uint32_t kb = (uint32_t)(min(k, klast) * 4);
    const uint32_t dst = ring + (uint32_t)((st % PD) * STEP);
    dma_load16(Ab, arow + kb, dst);
    dma_load16(Bb, brow + kb, dst + 1024);
  };
  f32x16_t acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.f;
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < PD; ++j) issue(j);
  for (int st = 0; st < nsteps; ++st) {
    wait_vmcnt<2 * (PD - 1)>();  // step st landed; the PD - 1 later steps may be in flight
    asm volatile("" ::: "memory");
    const char* slotp = smem + ns * PD * STEP + (st % PD) * STEP;
    float4 a = *(const float4*)(slotp + 16 * lane);
    float4 b = *(const float4*)(slotp + 1024 + 16 * lane);
    if (!(k0 + 8 * (int64_t)st + h4 < k1)) a = b = make_float4(0.f, 0.f, 0.f, 0.f);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, b.x, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, b.y, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, b.z, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, b.w, acc, 0, 0, 0);
    ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;  // (used only with sumsq)
    asm volatile("" ::: "memory");
    issue(st + PD);
  }
  wait_vmcnt<0>();  // no direct-to-LDS load lands after the workgroup ends
  // partial subtile: rows 8(r/4) + 4(l/32) + r%4, column l%32 (32 lanes store 128 contiguous bytes)
  float* dst = q.part + ((int64_t)g * q.Mp + m0 + h4) * q.Npk + (int64_t)tni * BNC + ns * 32 + (lane & 31);
#pragma unroll
  for (int r = 0; r < 16; ++r) dst[(int64_t)(8 * (r >> 2) + (r & 3)) * q.Npk] = acc[r];
  if (p.sumsq && ns == 0 && tni == 0) {
    const float v = ss + __shfl_xor(ss, 32);
    if (lane < 32) q.ssq[(int64_t)g * q.Mp + m0 + lane] = v;
  }
#endif
}

template <int BNC, int RB>
__global__ void __launch_bounds__(256) gemm_f32_ksr_kernel(F32Ksp q) {
  constexpr int SROW = BNC + 8, V4 = RB * BNC / 4;  // float4s of the RB-row slab
  __shared__ __attribute__((aligned(16))) float slab[RB * SROW];
  __shared__ float rs[RB];
  const GemmK& p = q.k;
  const int tid = threadIdx.x;
  const int tn = (int)blockIdx.x % p.tiles_n, tr = (int)blockIdx.x / p.tiles_n;
  const int64_t r0 = (int64_t)tr * RB;
  for (int v = tid; v < V4; v += 256) {
    const int r = v / (BNC / 4), c4 = (v - r * (BNC / 4)) * 4;
    const float* src = q.part + (r0 + r) * q.Npk + (int64_t)tn * BNC + c4;
    const int64_t plane = q.Mp * q.Npk;
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
    // slices in order, eight loads in flight at a time
    for (int g0 = 0; g0 < q.ksg; g0 += 8) {
      float4 x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (g0 + u < q.ksg) x[u] = *(const float4*)(src + (int64_t)(g0 + u) * plane);
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (g0 + u < q.ksg) {
          a.x += x[u].x; a.y += x[u].y; a.z += x[u].z; a.w += x[u].w;
        }
    }
    *(float4*)(slab + r * SROW + c4) = a;
  }
  if (p.sumsq && tid < RB) {
    // the slices' row sums in order, eight loads in flight at a time (indices
    // clamped and additions past the end selected away: no branch between the
    // loads for the compiler to wait in)
    const float* sq = q.ssq + r0 + tid;
    float v = 0.f;
    for (int g0 = 0; g0 < q.ksg; g0 += 8) {
      float x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) x[u] = sq[(int64_t)min(g0 + u, q.ksg - 1) * q.Mp];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float t = v + x[u];
        v = g0 + u < q.ksg ? t : v;
      }
    }
    rs[tid] = rsqrtf(v * p.inv_k + p.eps);
    const int64_t gr = r0 + tid;
    if (p.sumsq_out && tn == 0 && gr < p.M) p.sumsq_out[gr] = v;
  }
  __syncthreads();
  epilogue_slab(p, slab, SROW, RB, rs, r0, tn, tid);
}

// K slices of the split-K fp32 path for tiles 32-row x BNC tiles: about one
// workgroup per CU, each slice at least two 8-wide steps. (Two per CU measured
// 15% slower on the fp32 block: twice the partial sums to write and re-read,
// each workgroup's K slice little more than its load pipeline's depth.)
static int f32_ksp_slices(int64_t tiles, int64_t K) {
  const int64_t cus = device_cus() > 0 ? device_cus() : 256;
  const int64_t want = cdiv(cus, tiles);
  return (int)std::max((int64_t)1, std::min({want, cdiv(K, 16), (int64_t)64}));
}

static int64_t f32_ksp_bytes(int64_t M, int64_t Npk, int64_t K, int bnc) {
  const int64_t Mp = cdiv(M, 32) * 32;
  const int ksg = f32_ksp_slices(cdiv(M, 32) * (Npk / bnc), K);
  return (int64_t)ksg * Mp * (Npk + 1) * 4;
}

// ------------------------------------------------------------------ packing
struct PackK {
  const void* src[TH_MAX_ACC];
  int64_t ld[TH_MAX_ACC];
  int src_dtype, out_dtype;
  int64_t N, K, Kp, rows;
  int bn, bnc;
  void* out;
};

// out[r][k] = src_i[k][t*bn + j] with r = t*bnc + i*bn + j; zero outside N, K.
__global__ void __launch_bounds__(256) pack_rhs_kernel(PackK p) {
  __shared__ float tile[32][33];
  const int64_t k0 = (int64_t)blockIdx.x * 32, r0 = (int64_t)blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  {
    const int64_t r = r0 + tx;
    const int64_t t = r / p.bnc, rem = r - t * p.bnc;
    const int i = (int)(rem / p.bn);
    const int64_t n = t * p.bn + (rem - (int64_t)i * p.bn);
    for (int yy = ty; yy < 32; yy += 8) {
      const int64_t k = k0 + yy;
      float v = 0.f;
      if (r < p.rows && k < p.K && n < p.N) v = load_elem(p.src[i], k * p.ld[i] + n, p.src_dtype);
      tile[yy][tx] = v;
    }
  }
  __syncthreads();
  for (int yy = ty; yy < 32; yy += 8) {
    const int64_t r = r0 + yy, k = k0 + tx;
    if (r < p.rows && k < p.Kp) store_elem(p.out, r * p.Kp + k, p.out_dtype, tile[tx][yy]);
  }
}

// e4m3 operands, bytes copied unchanged, in fragment-major order: for each
// group g of 32 packed rows and each 32-wide K chunk c, one 1 KiB block at
// (g * Kp/32 + c) * 1024 whose 16-byte slot l (l = 0..63) holds row
// 32g + l%32, k = 32c + 16*(l/32) .. +16. A wave loading 16 bytes per lane
// then reads one contiguous KiB: exactly the MFMA operands of that chunk.
// One thread per 16-byte slot.
__global__ void __launch_bounds__(256) pack_rhs_fp8_kernel(PackK p) {
  const int64_t slot = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t nch = p.Kp / 32;
  const int64_t total = (p.rows / 32) * nch * 64;
  if (slot >= total) return;
  const int l = (int)(slot & 63);
  const int64_t blk = slot >> 6;
  const int64_t g = blk / nch, c = blk - g * nch;
  const int64_t r = g * 32 + (l & 31);
  const int64_t t = r / p.bnc, rem = r - t * p.bnc;
  const int i = (int)(rem / p.bn);
  const int64_t n = t * p.bn + (rem - (int64_t)i * p.bn);
  const int64_t k0 = c * 32 + 16 * (l >> 5);
  uint32_t w[4] = {0, 0, 0, 0};
  const uint8_t* src = (const uint8_t*)p.src[i];
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int64_t k = k0 + q;
    const uint32_t v = (n < p.N && k < p.K) ? src[k * p.ld[i] + n] : 0u;
    w[q >> 2] |= v << (8 * (q & 3));
  }
  *(uint4*)((uint8_t*)p.out + slot * 16) = make_uint4(w[0], w[1], w[2], w[3]);
}

// Per-accumulator column tile bn; the block tile is n_acc * bn columns.
static int choose_bn(int64_t N, int n_acc, int in_dtype) {
  // e4m3 weights: 128-column packed tiles, the shared-activation kernel's
  // workgroup (both SwiGLU halves of a column stay inside one workgroup)
  if (in_dtype == TH_F8E4M3 && (n_acc == 1 || n_acc == 2) && N >= 128) return 128 / n_acc;
  if (in_dtype == TH_F32) {
    switch (n_acc) {
      case 1: return N > 64 ? 128 : 64;
      case 2: return N > 32 ? 64 : 32;
      case 3: return 64;
      default: return N > 32 ? 64 : 32;
    }
  }
  switch (n_acc) {
    case 1: return N >= 2048 ? 256 : (N >= 768 ? 128 : 64);
    case 2: return N >= 128 ? 128 : (N > 32 ? 64 : 32);
    case 3: return 64;
    default: return N > 32 ? 64 : 32;
  }
}

static int64_t packed_kp(int64_t K, int in_dtype) {
  const int64_t a = in_dtype == TH_F32 ? 4 : in_dtype == TH_F8E4M3 ? 32 : 8;  // whole 16-byte loads / 32-K chunks
  return (K + a - 1) / a * a;
}

static int elem_bytes(int dtype) { return dtype == TH_F32 ? 4 : dtype == TH_F8E4M3 ? 1 : 2; }
static bool gemm_in_ok(int d) { return d == TH_BF16 || d == TH_F32 || d == TH_F8E4M3; }

static bool aligned(const void* p, int bytes) { return ((uintptr_t)p % bytes) == 0; }

}  // namespace th

using namespace th;

extern "C" int th_gemm_acc_tile(int64_t N, int32_t n_acc, int32_t in_dtype) {
  if (N <= 0 || n_acc < 1 || n_acc > TH_MAX_ACC) return 0;
  return choose_bn(N, n_acc, in_dtype);
}

extern "C" int64_t th_gemm_packed_bytes(int64_t N, int64_t K, int32_t n_acc, int32_t in_dtype) {
  if (N <= 0 || K <= 0 || n_acc < 1 || n_acc > TH_MAX_ACC) return -1;
  if (!gemm_in_ok(in_dtype)) return -1;
  const int bn = choose_bn(N, n_acc, in_dtype);
  const int64_t rows = cdiv(N, bn) * bn * n_acc;
  return rows * packed_kp(K, in_dtype) * elem_bytes(in_dtype);
}

extern "C" int64_t th_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t n_acc, int32_t in_dtype) {
  if (M <= 0 || N <= 0 || K <= 0 || n_acc < 1 || n_acc > TH_MAX_ACC || !gemm_in_ok(in_dtype)) return -1;
  const int bn = choose_bn(N, n_acc, in_dtype);
  if (in_dtype == TH_F32) {
    // the split-K pass of small grids (too few 64-row tiles to occupy the GPU); optional:
    // without it th_gemm splits K inside each workgroup instead
    const int64_t cus = device_cus() > 0 ? device_cus() : 256;
    if (cdiv(M, 64) * cdiv(N, bn) >= cus) return 0;
    return f32_ksp_bytes(M, cdiv(N, bn) * bn * n_acc, K, bn * n_acc);
  }
  if (in_dtype != TH_F8E4M3) return 0;
  return fp8_workspace_bytes(M, cdiv(N, bn) * bn * n_acc, K, bn, n_acc);
}

extern "C" int th_gemm_pack_rhs(const void* const* src, const int64_t* ld_src, int32_t src_dtype,
                                int64_t N, int64_t K, int32_t n_acc, int32_t in_dtype, void* packed,
                                void* stream) {
  TH_CHECK_ARG(src && ld_src && packed, "th_gemm_pack_rhs: null pointer argument");
  TH_CHECK_ARG(N > 0 && K > 0, "th_gemm_pack_rhs: N=%lld K=%lld must be positive", (long long)N, (long long)K);
  TH_CHECK_ARG(n_acc >= 1 && n_acc <= TH_MAX_ACC, "th_gemm_pack_rhs: n_acc=%d out of range", n_acc);
  TH_CHECK_ARG(gemm_in_ok(in_dtype), "th_gemm_pack_rhs: in_dtype %d unsupported", in_dtype);
  TH_CHECK_ARG(in_dtype == TH_F8E4M3 ? src_dtype == TH_F8E4M3 : (src_dtype == TH_BF16 || src_dtype == TH_F32),
               "th_gemm_pack_rhs: src_dtype %d does not fit in_dtype %d", src_dtype, in_dtype);
  PackK p{};
  for (int i = 0; i < n_acc; ++i) {
    TH_CHECK_ARG(src[i] != nullptr, "th_gemm_pack_rhs: src[%d] is null", i);
    TH_CHECK_ARG(ld_src[i] >= N, "th_gemm_pack_rhs: ld_src[%d]=%lld < N", i, (long long)ld_src[i]);
    p.src[i] = src[i];
    p.ld[i] = ld_src[i];
  }
  if (!device_ready()) {
    set_error("th_gemm_pack_rhs: th_init was not called for the current device");
    return TH_ERR_NOT_INIT;
  }
  p.src_dtype = src_dtype;
  p.out_dtype = in_dtype;
  p.N = N;
  p.K = K;
  p.Kp = packed_kp(K, in_dtype);
  p.bn = choose_bn(N, n_acc, in_dtype);
  p.bnc = p.bn * n_acc;
  p.rows = cdiv(N, p.bn) * p.bnc;
  p.out = packed;
  dim3 grid((unsigned)cdiv(p.Kp, 32), (unsigned)cdiv(p.rows, 32));
  if (in_dtype == TH_F8E4M3)
    hipLaunchKernelGGL(pack_rhs_fp8_kernel, dim3((unsigned)cdiv((p.rows / 32) * (p.Kp / 32) * 64, 256)), dim3(256), 0,
                       (hipStream_t)stream, p);
  else
    hipLaunchKernelGGL(pack_rhs_kernel, grid, dim3(256), 0, (hipStream_t)stream, p);
  TH_CHECK_LAUNCH();
  return TH_OK;
}

template <int BM, int BNC>
static void launch_bf16(const GemmK& k, hipStream_t s) {
  hipLaunchKernelGGL((gemm_bf16_kernel<BM, BNC>), dim3(k.tiles_m * k.tiles_n), dim3(256), 0, s, k);
}

// 64-row tiles are for small problems: deeper pipelines there hide the
// global-load latency that a short K loop cannot amortise. Up to 144 KiB of
// stages (eight for 64 x 64 tiles: a K of 512 is then in flight at once).
template <int BM, int BNC>
constexpr int dl_stages() {
  constexpr int s = 147456 / ((BM + BNC) * 128);
  return BM > 64 ? 2 : (s > 8 ? 8 : s);
}

// Two workgroups per CU: stages within 80 KiB each (the row scales share them).
template <int BM, int BNC>
constexpr int dl_stages2() {
  constexpr int s = 81920 / ((BM + BNC) * 128);
  return s > 8 ? 8 : s;
}

template <int BM, int BNC>
static void launch_bf16_dl(const GemmK& k, hipStream_t s) {
  const int tiles = k.tiles_m * k.tiles_n, cus = device_cus();
  auto go = [&](auto st) {
    constexpr int S = decltype(st)::value;
    if (k.sumsq)
      hipLaunchKernelGGL((gemm_bf16_dl_kernel<BM, BNC, true, S>), dim3(tiles), dim3(256), 0, s, k);
    else
      hipLaunchKernelGGL((gemm_bf16_dl_kernel<BM, BNC, false, S>), dim3(tiles), dim3(256), 0, s, k);
  };
  // More tiles than CUs but no more than two per CU: shallower stages let two
  // workgroups share a CU, so the tiles run as one round (each workgroup's
  // load latency and epilogue under the other's work) instead of two.
  if constexpr (BM == 64 && dl_stages2<BM, BNC>() >= 2) {
    if (cus > 0 && tiles > cus && tiles <= 2 * cus) {
      go(std::integral_constant<int, dl_stages2<BM, BNC>()>());
      return;
    }
  }
  go(std::integral_constant<int, dl_stages<BM, BNC>()>());
}

template <int BM, int BNC>
static void launch_bf16_pk(const GemmK& k, hipStream_t s) {
  const int tiles = k.tiles_m * k.tiles_n;
  const int cus = device_cus();
  const int grid = cus > 0 && tiles > cus ? cus : tiles;
  auto go = [&](auto nacc) {
    constexpr int NA = decltype(nacc)::value;
    if constexpr (BNC % NA == 0 && (BNC / NA / 2) % 32 == 0) {
      constexpr int NW = BM == 256 ? 8 : 4;  // eight waves (two per SIMD) only for 256-row tiles
      if constexpr (NA == 2) {
        if (k.asplit) {
          if (k.sumsq)
            hipLaunchKernelGGL((gemm_bf16_pk_kernel<BM, BNC, true, NW, 2, true>), dim3(grid), dim3(64 * NW), 0, s, k);
          else
            hipLaunchKernelGGL((gemm_bf16_pk_kernel<BM, BNC, false, NW, 2, true>), dim3(grid), dim3(64 * NW), 0, s, k);
          return;
        }
      }
      if (k.sumsq)
        hipLaunchKernelGGL((gemm_bf16_pk_kernel<BM, BNC, true, NW, NA>), dim3(grid), dim3(64 * NW), 0, s, k);
      else
        hipLaunchKernelGGL((gemm_bf16_pk_kernel<BM, BNC, false, NW, NA>), dim3(grid), dim3(64 * NW), 0, s, k);
    } else {
      launch_bf16_dl<BM, BNC>(k, s);  // no per-wave split of this column tile (the host selects none such)
    }
  };
  switch (k.n_acc) {
    case 1: go(std::integral_constant<int, 1>{}); break;
    case 2: go(std::integral_constant<int, 2>{}); break;
    case 3: go(std::integral_constant<int, 3>{}); break;
    default: go(std::integral_constant<int, 4>{}); break;
  }
}

enum class MainLoop { staged, direct, persistent };

template <int BM, int BNC>
static void launch_bf16_any(const GemmK& k, MainLoop m, hipStream_t s) {
  if constexpr (BM == 64) {  // 64-row tiles exist for the direct loop only
    launch_bf16_dl<BM, BNC>(k, s);
  } else {
    switch (m) {
      case MainLoop::persistent: launch_bf16_pk<BM, BNC>(k, s); break;
      case MainLoop::direct: launch_bf16_dl<BM, BNC>(k, s); break;
      default: launch_bf16<BM, BNC>(k, s); break;
    }
  }
}

template <int BNC>
static void launch_f32(const GemmK& k, hipStream_t s) {
  hipLaunchKernelGGL((gemm_f32_kernel<BNC>), dim3(k.tiles_m * k.tiles_n), dim3(256), 0, s, k);
}

// 32-row tiles, K split over the waves of a workgroup (tiles_m counts 32-row tiles)
template <int BNC>
static void launch_f32_sk(const GemmK& k, hipStream_t s) {
  constexpr int NSUB = BNC / 32, KS = 16 / NSUB > 0 ? 16 / NSUB : 1;
  hipLaunchKernelGGL((gemm_f32_sk_kernel<BNC>), dim3(k.tiles_m * k.tiles_n), dim3(64 * NSUB * KS), 0, s, k);
}

// 32-row tiles, K split over workgroups through the workspace, then the reduce / epilogue pass
template <int BNC>
static void launch_f32_ksp(const F32Ksp& q, hipStream_t s) {
  hipLaunchKernelGGL((gemm_f32_ksp_kernel<BNC>), dim3(q.k.tiles_m * q.k.tiles_n, q.ksg), dim3(2 * BNC), 0, s, q);
  // 8-row slabs, or 2-row ones when 8-row ones would leave CUs without a
  // workgroup (the partials are then fetched by every CU)
  const int64_t cus = device_cus() > 0 ? device_cus() : 256;
  if (q.Mp / 8 * q.k.tiles_n < cus)
    hipLaunchKernelGGL((gemm_f32_ksr_kernel<BNC, 2>), dim3((unsigned)(q.Mp / 2 * q.k.tiles_n)), dim3(256), 0, s, q);
  else
    hipLaunchKernelGGL((gemm_f32_ksr_kernel<BNC, 8>), dim3((unsigned)(q.Mp / 8 * q.k.tiles_n)), dim3(256), 0, s, q);
}

extern "C" int th_gemm(const th_gemm_desc* d, void* stream) {
  TH_CHECK_ARG(d != nullptr, "th_gemm: null descriptor");
  TH_CHECK_ARG(d->M > 0 && d->N > 0 && d->K > 0, "th_gemm: M=%lld N=%lld K=%lld must be positive",
               (long long)d->M, (long long)d->N, (long long)d->K);
  TH_CHECK_ARG(d->n_acc >= 1 && d->n_acc <= TH_MAX_ACC, "th_gemm: n_acc=%d out of range 1..%d", d->n_acc, TH_MAX_ACC);
  TH_CHECK_ARG(gemm_in_ok(d->in_dtype), "th_gemm: in_dtype %d unsupported", d->in_dtype);
  TH_CHECK_ARG(d->lhs && d->rhs_packed, "th_gemm: null lhs or rhs_packed");
  const bool fp8 = d->in_dtype == TH_F8E4M3;
  if (fp8) {
    TH_CHECK_ARG(d->M <= 128, "th_gemm: fp8 weights are for at most 128 rows (got M=%lld)", (long long)d->M);
    TH_CHECK_ARG(d->K % 32 == 0, "th_gemm: fp8 weights need K %% 32 == 0 (K=%lld)", (long long)d->K);
    TH_CHECK_ARG(d->rhs_scale != nullptr, "th_gemm: fp8 weights need rhs_scale");
  }
  const int align = d->in_dtype == TH_F32 ? 4 : 8;
  TH_CHECK_ARG(d->K % align == 0, "th_gemm: K=%lld must be a multiple of %d", (long long)d->K, align);
  TH_CHECK_ARG(d->ld_lhs >= d->K && d->ld_lhs % align == 0, "th_gemm: ld_lhs=%lld invalid", (long long)d->ld_lhs);
  TH_CHECK_ARG(aligned(d->lhs, 16) && aligned(d->rhs_packed, 16), "th_gemm: lhs/rhs_packed must be 16-byte aligned");
  TH_CHECK_ARG(d->n_out >= 1 && d->n_out <= TH_MAX_OUT, "th_gemm: n_out=%d out of range", d->n_out);
  TH_CHECK_ARG(d->n_extra >= 0 && d->n_extra <= TH_MAX_EXTRA, "th_gemm: n_extra=%d out of range", d->n_extra);
  TH_CHECK_ARG(d->rscale_mask == 0 || d->sumsq, "th_gemm: rscale_mask set without sumsq");
  if (d->lhs_gain != nullptr && !fp8) {
    set_error("th_gemm: lhs_gain is implemented for TH_F8E4M3 weights only");
    return TH_ERR_UNSUPPORTED;
  }
  TH_CHECK_ARG(d->lhs_gain == nullptr || aligned(d->lhs_gain, 16), "th_gemm: lhs_gain must be 16-byte aligned");
  if (d->rs_parts != nullptr) {
    TH_CHECK_ARG(d->in_dtype == TH_BF16 || (fp8 && d->lhs_gain == nullptr),
                 "th_gemm: rs_parts is implemented for TH_BF16, and TH_F8E4M3 without lhs_gain");
    TH_CHECK_ARG(d->sumsq, "th_gemm: rs_parts set without sumsq");
    TH_CHECK_ARG(d->n_rs_parts > 0 && d->n_rs_parts % 4 == 0 && d->ld_rs_parts >= d->n_rs_parts &&
                     d->ld_rs_parts % 4 == 0 && aligned(d->rs_parts, 16),
                 "th_gemm: rs_parts needs a positive multiple of 4 parts per row, 16-byte aligned rows");
  }
  if (d->gain_out != nullptr) {
    if (!fp8) {
      set_error("th_gemm: gain_out is implemented for TH_F8E4M3 weights only");
      return TH_ERR_UNSUPPORTED;
    }
    TH_CHECK_ARG(d->gain_out_index >= 0 && d->gain_out_index < d->n_out, "th_gemm: gain_out_index out of range");
    const th_epi_out& go = d->out[d->gain_out_index];
    TH_CHECK_ARG(go.dtype == TH_BF16 && go.col_begin == 0 && (go.col_end == 0 || go.col_end == d->N),
                 "th_gemm: the gain_out output must be bf16 over all N columns");
    TH_CHECK_ARG(d->N % 1024 == 0, "th_gemm: gain_out needs N a multiple of 1024 (N=%lld)", (long long)d->N);
    TH_CHECK_ARG(d->ss_parts_out != nullptr && d->ld_ss_parts_out >= d->N / 256 && d->ld_ss_parts_out % 4 == 0 &&
                     aligned(d->ss_parts_out, 16) && aligned(d->gain_out, 16),
                 "th_gemm: gain_out needs ss_parts_out [M, N/256] fp32 (16-byte aligned rows) and an aligned gain");
  }
  int bn = choose_bn(d->N, d->n_acc, d->in_dtype);
  // One accumulator over 1024 <= N < 2048 columns: 256 x 256 tiles, one per CU
  // per wave, when they make whole waves, instead of twice as many 256 x 128
  // tiles: the same MFMA work per CU for a third less operand traffic per FLOP
  // (16384 x 1024 x 2048: 87.6 -> 75.1 us). N a multiple of 256 keeps the
  // packed rhs exactly as packed for 128-column tiles (one accumulator's
  // packed rows are its columns in order, padded to the tile width).
  bool wide = false;
  if (d->in_dtype == TH_BF16 && d->n_acc == 1 && bn == 128 && d->N % 256 == 0 && d->K % 64 == 0) {
    bool rope = false;
    for (int o = 0; o < d->n_out; ++o) rope |= d->out[o].op == TH_EPI_ROPE || d->out[o].op == TH_EPI_ROPE_PAIR;
    const int64_t cus = device_cus() > 0 ? device_cus() : 256;
    const int64_t t256 = cdiv(d->M, 256) * (d->N / 256);
    wide = !rope && t256 >= cus && t256 % cus == 0;
    if (wide) bn = 256;
  }
  GemmK k{};
  k.A = d->lhs;
  k.lda = d->ld_lhs;
  k.B = d->rhs_packed;
  k.ldb = packed_kp(d->K, d->in_dtype);
  k.M = d->M;
  k.N = d->N;
  k.K = d->K;
  k.bn = bn;
  k.n_acc = d->n_acc;
  k.sumsq = d->sumsq ? 1 : 0;
  k.rscale_mask = d->rscale_mask;
  k.inv_k = d->inv_k;
  k.eps = d->eps;
  for (int e = 0; e < d->n_extra; ++e) {
    TH_CHECK_ARG(d->extra[e] != nullptr, "th_gemm: extra[%d] is null", e);
    TH_CHECK_ARG(d->extra_dtype[e] == TH_BF16 || d->extra_dtype[e] == TH_F32, "th_gemm: extra_dtype[%d] unsupported", e);
    k.extra[e] = d->extra[e];
    k.ld_extra[e] = d->ld_extra[e];
    k.extra_dtype[e] = d->extra_dtype[e];
    const int eb = d->extra_dtype[e] == TH_F32 ? 16 : 8;
    k.extra_vec[e] = aligned(d->extra[e], eb) && d->ld_extra[e] % 4 == 0;
    k.extra_vec8[e] = aligned(d->extra[e], 16) && d->ld_extra[e] % (d->extra_dtype[e] == TH_F32 ? 4 : 8) == 0;
  }
  bool need_rope = false;
  for (int o = 0; o < d->n_out; ++o) {
    const th_epi_out& eo = d->out[o];
    TH_CHECK_ARG(eo.op >= TH_EPI_ACC && eo.op <= TH_EPI_MUL, "th_gemm: out[%d].op=%d unknown", o, eo.op);
    TH_CHECK_ARG(eo.a >= 0 && eo.a < d->n_acc, "th_gemm: out[%d].a=%d out of range", o, eo.a);
    const bool uses_b = eo.op == TH_EPI_ROPE_PAIR || eo.op == TH_EPI_SWIGLU;
    TH_CHECK_ARG(!uses_b || (eo.b >= 0 && eo.b < d->n_acc), "th_gemm: out[%d].b=%d out of range", o, eo.b);
    const bool uses_e = eo.op == TH_EPI_ADD || eo.op == TH_EPI_SOFTPLUS_ADD || eo.op == TH_EPI_MUL;
    TH_CHECK_ARG(!uses_e || (eo.e >= 0 && eo.e < d->n_extra), "th_gemm: out[%d].e=%d out of range", o, eo.e);
    const int64_t cb = eo.col_begin, ce = eo.col_end ? eo.col_end : d->N;
    TH_CHECK_ARG(cb >= 0 && cb < ce && ce <= d->N && cb % 8 == 0 && (ce % 8 == 0 || ce == d->N),
                 "th_gemm: out[%d] column window [%lld, %lld) must lie in [0, N=%lld) on multiples of 8", o,
                 (long long)cb, (long long)ce, (long long)d->N);
    TH_CHECK_ARG(eo.ptr != nullptr && eo.ld >= ce - cb, "th_gemm: out[%d] null or ld < its width", o);
    TH_CHECK_ARG(!uses_e || d->ld_extra[eo.e] >= ce - cb, "th_gemm: out[%d] extra row stride < its width", o);
    TH_CHECK_ARG(eo.dtype == TH_BF16 || eo.dtype == TH_F32, "th_gemm: out[%d].dtype unsupported", o);
    need_rope |= eo.op == TH_EPI_ROPE || eo.op == TH_EPI_ROPE_PAIR;
    k.out[o].op = eo.op;
    k.out[o].a = eo.a;
    k.out[o].b = uses_b ? eo.b : -1;
    k.out[o].e = uses_e ? eo.e : -1;
    k.out[o].ptr = eo.ptr;
    k.out[o].ld = eo.ld;
    k.out[o].dtype = eo.dtype;
    const int ob = eo.dtype == TH_F32 ? 16 : 8;
    k.out[o].vec = aligned(eo.ptr, ob) && eo.ld % 4 == 0;
    k.out[o].vec8 = aligned(eo.ptr, 16) && eo.ld % (eo.dtype == TH_F32 ? 4 : 8) == 0;
    k.out[o].cb = (int)cb;
    k.out[o].ce = (int)ce;
    if (eo.op == TH_EPI_ROPE || eo.op == TH_EPI_ROPE_PAIR) {
      TH_CHECK_ARG(d->rope_head_dim > 0 && cb % d->rope_head_dim == 0,
                   "th_gemm: out[%d] RoPE window must start on a head (head_dim %d)", o, d->rope_head_dim);
    }
    if (eo.op == TH_EPI_ROPE) {
      // (e4m3 weights: the reduce pass reads rotation partners from any tile)
      TH_CHECK_ARG(d->rope_head_dim > 0 && d->rope_head_dim % 2 == 0 && (fp8 || bn % d->rope_head_dim == 0),
                   "th_gemm: fused RoPE needs the column tile (%d) to hold whole heads (head_dim %d)", bn,
                   d->rope_head_dim);
    }
  }
  k.n_out = d->n_out;
  if (need_rope) {
    TH_CHECK_ARG(d->rope_cos && d->rope_sin, "th_gemm: RoPE output without cos/sin tables");
    TH_CHECK_ARG(d->rope_head_dim >= 4 && d->rope_head_dim % 8 == 0 && d->N % d->rope_head_dim == 0,
                 "th_gemm: rope_head_dim=%d invalid for N=%lld", d->rope_head_dim, (long long)d->N);
    TH_CHECK_ARG(d->rope_period > 0, "th_gemm: rope_period must be positive");
    TH_CHECK_ARG(aligned(d->rope_cos, 16) && aligned(d->rope_sin, 16), "th_gemm: RoPE tables must be 16-byte aligned");
  }
  k.rcos = d->rope_cos;
  k.rsin = d->rope_sin;
  k.hd = d->rope_head_dim > 0 ? d->rope_head_dim : 1;
  k.period = d->rope_period > 0 ? d->rope_period : 1;
  k.sumsq_out = d->sumsq_out;
  k.gain = d->lhs_gain;
  k.rs_parts = d->rs_parts;
  k.ld_rs_parts = d->ld_rs_parts;
  k.n_rs_parts = d->n_rs_parts;
  k.gain_out = d->gain_out;
  k.ss_parts_out = d->ss_parts_out;
  k.ld_ss_parts_out = d->ld_ss_parts_out;
  k.gain_index = d->gain_out_index;
  if (!device_ready()) {
    set_error("th_gemm: th_init was not called for the current device");
    return TH_ERR_NOT_INIT;
  }

  hipStream_t s = (hipStream_t)stream;
  const int bnc = bn * d->n_acc;
  k.tiles_n = (int)cdiv(d->N, bn);
  if (fp8) {
    k.tiles_m = 1;
    return launch_gemm_fp8(k, cdiv(d->N, bn) * bnc, d->rhs_scale, d->workspace, d->workspace_bytes, s);
  }
  if (d->in_dtype == TH_F32) {
    const int64_t cus = device_cus() > 0 ? device_cus() : 256;
    // (32-bit per-lane byte offsets into both operands)
    const bool small_ok = d->M * d->ld_lhs * 4 < ((int64_t)1 << 31) && (int64_t)cdiv(d->N, bn) * bnc * k.ldb * 4 <
                                                                             ((int64_t)1 << 31);
    if (small_ok && cdiv(d->M, 64) * k.tiles_n < cus) {
      k.tiles_m = (int)cdiv(d->M, 32);
      const int64_t npk = (int64_t)k.tiles_n * bnc;
      if (d->workspace && d->workspace_bytes >= f32_ksp_bytes(d->M, npk, d->K, bnc) &&
          ((uintptr_t)d->workspace & 15) == 0) {
        // too few 64-row tiles to occupy the GPU: K split over workgroups through the workspace
        F32Ksp q{};
        q.k = k;
        q.Mp = (int64_t)k.tiles_m * 32;
        q.Npk = npk;
        q.ksg = f32_ksp_slices((int64_t)k.tiles_m * k.tiles_n, d->K);
        q.kq = cdiv(cdiv(d->K, q.ksg), 8) * 8;
        q.ksg = (int)cdiv(d->K, q.kq);
        q.part = d->workspace;
        q.ssq = d->workspace + q.ksg * q.Mp * q.Npk;
        switch (bnc) {
          case 64: launch_f32_ksp<64>(q, s); break;
          case 128: launch_f32_ksp<128>(q, s); break;
          case 192: launch_f32_ksp<192>(q, s); break;
          case 256: launch_f32_ksp<256>(q, s); break;
          default: set_error("th_gemm: no fp32 kernel for tile %d", bnc); return TH_ERR_UNSUPPORTED;
        }
        TH_CHECK_LAUNCH();
        return TH_OK;
      }
      // without a workspace: 32-row tiles with the K loop split over the waves of a workgroup
      switch (bnc) {
        case 64: launch_f32_sk<64>(k, s); break;
        case 128: launch_f32_sk<128>(k, s); break;
        case 192: launch_f32_sk<192>(k, s); break;
        case 256: launch_f32_sk<256>(k, s); break;
        default: set_error("th_gemm: no fp32 kernel for tile %d", bnc); return TH_ERR_UNSUPPORTED;
      }
      TH_CHECK_LAUNCH();
      return TH_OK;
    }
    k.tiles_m = (int)cdiv(d->M, 64);
    switch (bnc) {
      case 64: launch_f32<64>(k, s); break;
      case 128: launch_f32<128>(k, s); break;
      case 192: launch_f32<192>(k, s); break;
      case 256: launch_f32<256>(k, s); break;
      default: set_error("th_gemm: no fp32 kernel for tile %d", bnc); return TH_ERR_UNSUPPORTED;
    }
  } else {
    // Row tile: 256 when that still gives two blocks per CU (or for the whole
    // waves of 256 x 256 tiles above), 128 when it gives one, else 64 (small
    // problems need the parallelism more than the reuse).
    const int64_t cus = device_cus() > 0 ? device_cus() : 256;
    int bm = wide || cdiv(d->M, 256) * k.tiles_n >= 2 * cus ? 256 : cdiv(d->M, 128) * k.tiles_n >= cus ? 128 : 64;
    const bool big = bm == 256;
    k.tiles_m = (int)cdiv(d->M, bm);
    // Direct-to-LDS main loop: whole 64-wide K tiles, and 32-bit buffer offsets
    // (one block's rows of lhs and of the packed rhs under 2 GiB).
    const bool direct = d->K % 64 == 0 && (int64_t)256 * d->ld_lhs * 2 < ((int64_t)1 << 31) &&
                        (int64_t)bnc * k.ldb * 2 < ((int64_t)1 << 31);
    // Persistent blocks with the per-wave epilogue: each wave holds half of
    // every accumulator's columns (bn/2, a multiple of 32), so a fused RoPE
    // head must fit in that half.
    bool wave_epi = bn >= 64 && d->M < ((int64_t)1 << 31) && d->N < ((int64_t)1 << 31);
    bool rope_in_half = true;
    for (int o = 0; o < d->n_out; ++o)
      if (d->out[o].op == TH_EPI_ROPE) rope_in_half &= (bn / 2) % k.hd == 0;
    if (!rope_in_half) {
      // two accumulators, each output reading one: a wave can hold a whole
      // accumulator tile (bn columns) instead, and with it whole heads
      bool split = d->n_acc == 2 && bn % k.hd == 0;
      for (int o = 0; o < d->n_out; ++o) split &= d->out[o].b < 0;
      k.asplit = split ? 1 : 0;
      wave_epi &= split;
    }
    // (the whole-accumulator-per-wave instances leave the row-sum parts out: registers)
    if (k.asplit && d->rs_parts != nullptr) {
      set_error("th_gemm: rs_parts is not implemented with whole-head RoPE on two accumulators");
      return TH_ERR_UNSUPPORTED;
    }
    MainLoop ml = MainLoop::staged;
    if (direct) ml = wave_epi ? MainLoop::persistent : MainLoop::direct;
    if (bm == 64 && ml == MainLoop::persistent) ml = MainLoop::direct;  // 64-row tiles: direct loop only
    if (bm == 64 && ml == MainLoop::staged) {  // the staged loop has no 64-row tile
      k.tiles_m = (int)cdiv(d->M, 128);
      bm = 128;
    }
    switch (bnc) {
      case 64: bm == 64 ? launch_bf16_any<64, 64>(k, ml, s) : big ? launch_bf16_any<256, 64>(k, ml, s) : launch_bf16_any<128, 64>(k, ml, s); break;
      case 128: bm == 64 ? launch_bf16_any<64, 128>(k, ml, s) : big ? launch_bf16_any<256, 128>(k, ml, s) : launch_bf16_any<128, 128>(k, ml, s); break;
      case 192: bm == 64 ? launch_bf16_any<64, 192>(k, ml, s) : big ? launch_bf16_any<256, 192>(k, ml, s) : launch_bf16_any<128, 192>(k, ml, s); break;
      case 256: bm == 64 ? launch_bf16_any<64, 256>(k, ml, s) : big ? launch_bf16_any<256, 256>(k, ml, s) : launch_bf16_any<128, 256>(k, ml, s); break;
      default: set_error("th_gemm: no bf16 kernel for tile %d", bnc); return TH_ERR_UNSUPPORTED;
    }
  }
  TH_CHECK_LAUNCH();
  return TH_OK;
}
