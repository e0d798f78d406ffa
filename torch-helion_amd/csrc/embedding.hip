// th_embedding: the token-embedding row gather (the `embedding` op of the
// OpGraph, made from aten.embedding by the capture handler; the reference's
// MambaModel takes float hidden states and has no table, models/mamba.py:343-359).
//
// HBM bound: per token it reads one id and one table row and writes one row
// (plus an optional fp32 copy). One lane moves one 16-byte chunk, so a wave
// covers 1 KiB of consecutive bytes of one or more rows and every access is
// a full 16-byte vector load or store. Rows whose width or stride is not a
// multiple of 16 bytes take the element-wise kernel.
#include "common.h"

namespace th {

struct EmbK {
  const void* table;
  int64_t ldt;
  const void* ids;
  void* out;
  int64_t ldo;
  float* out32;
  int64_t ldo32;
  int32_t* n_invalid;
  int64_t tokens;
  int64_t vocab;
  int dim;
  int cpr;    // 16-byte chunks per row (vector kernel) or elements per row
  int shift;  // log2(cpr) when cpr is a power of two, else -1
};

__device__ __forceinline__ int64_t row_of(const EmbK& p, int64_t i) {
  return p.shift >= 0 ? i >> p.shift : i / p.cpr;
}

template <typename IdT>
__device__ __forceinline__ bool lookup(const EmbK& p, int64_t t, int64_t& id) {
  id = (int64_t)((const IdT*)p.ids)[t];
  return id >= 0 && id < p.vocab;
}

// EB = element bytes (2 bf16, 4 fp32).
template <typename IdT, int EB>
__global__ void __launch_bounds__(256) embedding_vec_kernel(EmbK p) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= p.tokens * p.cpr) return;
  const int64_t t = row_of(p, i);
  const int c = (int)(i - t * p.cpr);
  int64_t id;
  const bool ok = lookup<IdT>(p, t, id);
  uint4 v = make_uint4(0, 0, 0, 0);
  if (ok)
    v = *(const uint4*)((const char*)p.table + id * p.ldt * EB + (int64_t)c * 16);
  else if (c == 0 && p.n_invalid)
    atomicAdd(p.n_invalid, 1);
  *(uint4*)((char*)p.out + t * p.ldo * EB + (int64_t)c * 16) = v;
  if (p.out32) {
    float* o = p.out32 + t * p.ldo32 + (int64_t)c * (16 / EB);
    if constexpr (EB == 2) {
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
      float f[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f[2 * q] = __uint_as_float(w[q] << 16);
        f[2 * q + 1] = __uint_as_float(w[q] & 0xffff0000u);
      }
      *(float4*)o = make_float4(f[0], f[1], f[2], f[3]);
      *(float4*)(o + 4) = make_float4(f[4], f[5], f[6], f[7]);
    } else {
      *(uint4*)o = v;
    }
  }
}

template <typename IdT>
__global__ void __launch_bounds__(256) embedding_elem_kernel(EmbK p, int dtype) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= p.tokens * p.cpr) return;
  const int64_t t = row_of(p, i);
  const int c = (int)(i - t * p.cpr);
  int64_t id;
  const bool ok = lookup<IdT>(p, t, id);
  float v = 0.f;
  if (ok)
    v = load_elem(p.table, id * p.ldt + c, dtype);
  else if (c == 0 && p.n_invalid)
    atomicAdd(p.n_invalid, 1);
  store_elem(p.out, t * p.ldo + c, dtype, v);
  if (p.out32) p.out32[t * p.ldo32 + c] = v;
}

}  // namespace th

using namespace th;

namespace {
bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }
}  // namespace

extern "C" int th_embedding(const th_embedding_desc* d, void* stream) {
  TH_CHECK_ARG(d != nullptr, "th_embedding: null descriptor");
  TH_CHECK_ARG(d->tokens >= 0 && d->dim > 0 && d->vocab > 0, "th_embedding: bad sizes");
  TH_CHECK_ARG(d->dtype == TH_BF16 || d->dtype == TH_F32, "th_embedding: dtype %d unsupported", d->dtype);
  TH_CHECK_ARG(d->ids_dtype == TH_I64 || d->ids_dtype == TH_I32, "th_embedding: ids dtype %d unsupported",
               d->ids_dtype);
  TH_CHECK_ARG(d->ld_table >= d->dim && d->ld_out >= d->dim, "th_embedding: row stride < dim");
  TH_CHECK_ARG(!d->out32 || d->ld_out32 >= d->dim, "th_embedding: out32 row stride < dim");
  if (d->tokens == 0) return TH_OK;
  TH_CHECK_ARG(d->table && d->ids && d->out, "th_embedding: null operand");
  if (!device_ready()) {
    set_error("th_embedding: th_init was not called for the current device");
    return TH_ERR_NOT_INIT;
  }
  const int eb = d->dtype == TH_BF16 ? 2 : 4;
  const int per = 16 / eb;
  const bool vec = d->dim % per == 0 && d->ld_table % per == 0 && d->ld_out % per == 0 && aligned16(d->table) &&
                   aligned16(d->out) && (!d->out32 || (d->ld_out32 % 4 == 0 && aligned16(d->out32)));
  EmbK k{};
  k.table = d->table; k.ldt = d->ld_table; k.ids = d->ids; k.out = d->out; k.ldo = d->ld_out;
  k.out32 = d->out32; k.ldo32 = d->ld_out32; k.n_invalid = d->n_invalid;
  k.tokens = d->tokens; k.vocab = d->vocab; k.dim = d->dim;
  k.cpr = vec ? d->dim / per : d->dim;
  k.shift = (k.cpr & (k.cpr - 1)) == 0 ? __builtin_ctz((unsigned)k.cpr) : -1;
  const int64_t work = d->tokens * k.cpr;
  TH_CHECK_ARG(cdiv(work, 256) < (int64_t)1 << 31, "th_embedding: %lld tokens exceed one launch",
               (long long)d->tokens);
  const dim3 grid((unsigned)cdiv(work, 256));
  hipStream_t s = (hipStream_t)stream;
  const bool i64 = d->ids_dtype == TH_I64;
  if (vec && eb == 2) {
    if (i64) hipLaunchKernelGGL((embedding_vec_kernel<int64_t, 2>), grid, dim3(256), 0, s, k);
    else hipLaunchKernelGGL((embedding_vec_kernel<int32_t, 2>), grid, dim3(256), 0, s, k);
  } else if (vec) {
    if (i64) hipLaunchKernelGGL((embedding_vec_kernel<int64_t, 4>), grid, dim3(256), 0, s, k);
    else hipLaunchKernelGGL((embedding_vec_kernel<int32_t, 4>), grid, dim3(256), 0, s, k);
  } else {
    if (i64) hipLaunchKernelGGL(embedding_elem_kernel<int64_t>, grid, dim3(256), 0, s, k, (int)d->dtype);
    else hipLaunchKernelGGL(embedding_elem_kernel<int32_t>, grid, dim3(256), 0, s, k, (int)d->dtype);
  }
  TH_CHECK_LAUNCH();
  return TH_OK;
}
