// Row-wise kernels: the stand-alone RMSNorm and the epilogue VM fallback.
//
// th_rmsnorm (reference: the GEMM-less norm kernel of optimizer/partition.py:165-177
// whose epilogue is `x * (sumsq/K + eps)^-1/2 * g_full`, optimizer/passes.py:357-370):
// HBM bound, one wave per row, the row held in registers between the
// sum-of-squares pass and the scaling pass so it is read from HBM once.
//
// th_epilogue_vm (reference: the epilogue SSA interpreter loop of
// codegen/interpret.py:27-34 over the registered ops of capture/ops.py:34-37):
// one pass per op over fp32 slots in a caller workspace. It exists so that any
// epilogue the fused catalogue of th_gemm does not cover still runs on the GPU.
#include "common.h"

namespace th {

struct NormK {
  const void* x;
  int64_t ldx;
  void* out;
  int64_t ldo;
  const float* gain;
  int64_t M, K;
  int xdt, odt;
  float inv_k, eps;
  float* out32;
  int64_t ldo32;
  int ovec, o32vec;  // fp32 out / out32 rows are 16-byte aligned
};

// NCH = 16-byte chunks per lane held in registers (0 = stream the row twice);
// XB = bf16 input (8 values per chunk) or fp32 (4). Every load and store is a
// 16-byte vector access except fp32 outputs whose rows are not 16-byte aligned.
template <int NCH, bool XB>
__global__ void __launch_bounds__(256) rmsnorm_kernel(NormK p) {
  constexpr int PER = XB ? 8 : 4;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= p.M) return;
  const int64_t nch = p.K / PER;  // K is a multiple of PER
  const uint4* xr = (const uint4*)((const char*)p.x + row * p.ldx * (XB ? 2 : 4));
  auto vals = [&](uint4 w, float* v) {
    if constexpr (XB) {
      const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        v[2 * q] = __uint_as_float(ws[q] << 16);
        v[2 * q + 1] = __uint_as_float(ws[q] & 0xffff0000u);
      }
    } else {
      v[0] = __uint_as_float(w.x); v[1] = __uint_as_float(w.y);
      v[2] = __uint_as_float(w.z); v[3] = __uint_as_float(w.w);
    }
  };
  float ss = 0.f;
  uint4 keep[NCH > 0 ? NCH : 1];
  if constexpr (NCH > 0) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int64_t c = lane + 64 * i;
      keep[i] = c < nch ? xr[c] : make_uint4(0, 0, 0, 0);
      float v[PER];
      vals(keep[i], v);
#pragma unroll
      for (int q = 0; q < PER; ++q) ss += v[q] * v[q];
    }
  } else {
    for (int64_t c = lane; c < nch; c += 64) {
      float v[PER];
      vals(xr[c], v);
#pragma unroll
      for (int q = 0; q < PER; ++q) ss += v[q] * v[q];
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  const float r = rsqrtf(ss * p.inv_k + p.eps);
  auto store_f32 = [&](float* dst, bool vec, const float* v) {
    if (vec) {
#pragma unroll
      for (int q = 0; q < PER; q += 4) *(float4*)(dst + q) = make_float4(v[q], v[q + 1], v[q + 2], v[q + 3]);
    } else {
#pragma unroll
      for (int q = 0; q < PER; ++q) dst[q] = v[q];
    }
  };
  auto emit = [&](int64_t c, uint4 w) {
    float v[PER];
    vals(w, v);
    const int64_t base = c * PER;
#pragma unroll
    for (int q = 0; q < PER; q += 4) {
      const float4 g = *(const float4*)(p.gain + base + q);
      v[q] *= r * g.x; v[q + 1] *= r * g.y; v[q + 2] *= r * g.z; v[q + 3] *= r * g.w;
    }
    if (p.out32) store_f32(p.out32 + row * p.ldo32 + base, p.o32vec, v);
    if (p.odt == TH_BF16) {
      uint16_t* orow = (uint16_t*)p.out + row * p.ldo + base;
      if constexpr (XB) {
        uint4 o;
        o.x = pk_bf16x2(v[0], v[1]);
        o.y = pk_bf16x2(v[2], v[3]);
        o.z = pk_bf16x2(v[4], v[5]);
        o.w = pk_bf16x2(v[6], v[7]);
        *(uint4*)orow = o;
      } else {
#pragma unroll
        for (int q = 0; q < PER; ++q) orow[q] = f32_to_bf16(v[q]);
      }
    } else {
      store_f32((float*)p.out + row * p.ldo + base, p.ovec, v);
    }
  };
  if constexpr (NCH > 0) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int64_t c = lane + 64 * i;
      if (c < nch) emit(c, keep[i]);
    }
  } else {
    for (int64_t c = lane; c < nch; c += 64) emit(c, xr[c]);
  }
}

// ------------------------------------------------------------- epilogue VM
struct VmElemK {
  int code, mode;
  float scalar;
  const float* a;
  const float* b;
  float* dst;
  th_vm_operand src;  // LOAD
  int64_t M, N;
};

__global__ void __launch_bounds__(256) vm_elem_kernel(VmElemK p) {
  const int64_t total = p.M * p.N;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t m = i / p.N, n = i - m * p.N;
    float r;
    if (p.code == TH_VM_LOAD) {
      const int64_t off = p.src.column ? m * p.src.ld : m * p.src.ld + n;
      r = load_elem(p.src.ptr, off, p.src.dtype);
    } else if (p.code == TH_VM_COPY) {
      r = p.a[i];
    } else if (p.code == TH_VM_EXP) {
      r = expf(p.a[i]);
    } else if (p.code == TH_VM_LOG) {
      r = logf(p.a[i]);
    } else {
      float x, y;
      if (p.mode == 0) { x = p.a[i]; y = p.b[i]; }
      else if (p.mode == 1) { x = p.a[i]; y = p.scalar; }
      else { x = p.scalar; y = p.a[i]; }
      switch (p.code) {
        case TH_VM_ADD: r = x + y; break;
        case TH_VM_SUB: r = x - y; break;
        case TH_VM_MUL: r = x * y; break;
        case TH_VM_DIV: r = x / y; break;
        case TH_VM_MAX: r = fmaxf(x, y); break;
        default: r = powf(x, y); break;
      }
    }
    p.dst[i] = r;
  }
}

__global__ void __launch_bounds__(256) vm_rowred_kernel(const float* a, float* dst, int64_t N, int is_max) {
  __shared__ float red[4];
  const int64_t m = blockIdx.x;
  const float* ar = a + m * N;
  float acc = is_max ? -INFINITY : 0.f;
  for (int64_t n = threadIdx.x; n < N; n += 256) acc = is_max ? fmaxf(acc, ar[n]) : acc + ar[n];
  for (int o = 32; o > 0; o >>= 1) {
    const float t = __shfl_xor(acc, o);
    acc = is_max ? fmaxf(acc, t) : acc + t;
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  float tot = red[0];
  for (int w = 1; w < 4; ++w) tot = is_max ? fmaxf(tot, red[w]) : tot + red[w];
  float* dr = dst + m * N;
  for (int64_t n = threadIdx.x; n < N; n += 256) dr[n] = tot;
}

__global__ void __launch_bounds__(256) vm_store_kernel(const float* s, void* out, int64_t ld, int dtype, int64_t M, int64_t N) {
  const int64_t total = M * N;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t m = i / N, n = i - m * N;
    store_elem(out, m * ld + n, dtype, s[i]);
  }
}

}  // namespace th

using namespace th;

extern "C" int th_rmsnorm(const th_rmsnorm_desc* d, void* stream) {
  TH_CHECK_ARG(d != nullptr, "th_rmsnorm: null descriptor");
  TH_CHECK_ARG(d->M > 0 && d->K > 0, "th_rmsnorm: M=%lld K=%lld must be positive", (long long)d->M, (long long)d->K);
  TH_CHECK_ARG(d->x && d->out && d->gain, "th_rmsnorm: null pointer");
  TH_CHECK_ARG(d->x_dtype == TH_BF16 || d->x_dtype == TH_F32, "th_rmsnorm: x_dtype unsupported");
  TH_CHECK_ARG(d->out_dtype == TH_BF16 || d->out_dtype == TH_F32, "th_rmsnorm: out_dtype unsupported");
  const int per = d->x_dtype == TH_BF16 ? 8 : 4;
  TH_CHECK_ARG(d->K % per == 0 && d->ld_x % per == 0 && d->ld_x >= d->K, "th_rmsnorm: K and ld_x must be multiples of %d", per);
  TH_CHECK_ARG(d->ld_out >= d->K, "th_rmsnorm: ld_out < K");
  TH_CHECK_ARG((uintptr_t)d->x % 16 == 0, "th_rmsnorm: x must be 16-byte aligned");
  if (d->out_dtype == TH_BF16 && per == 8)
    TH_CHECK_ARG((uintptr_t)d->out % 16 == 0 && d->ld_out % 8 == 0, "th_rmsnorm: bf16 out must be 16-byte aligned with ld %% 8 == 0");
  if (!device_ready()) {
    set_error("th_rmsnorm: th_init was not called for the current device");
    return TH_ERR_NOT_INIT;
  }
  NormK k{};
  k.x = d->x; k.ldx = d->ld_x; k.out = d->out; k.ldo = d->ld_out; k.gain = d->gain;
  k.M = d->M; k.K = d->K; k.xdt = d->x_dtype; k.odt = d->out_dtype; k.inv_k = d->inv_k; k.eps = d->eps;
  k.out32 = d->out32; k.ldo32 = d->ld_out32;
  TH_CHECK_ARG(!d->out32 || d->ld_out32 >= d->K, "th_rmsnorm: ld_out32 < K");
  const int64_t nch = d->K / per;
  auto al16 = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
  k.ovec = d->out_dtype == TH_F32 && al16(d->out) && d->ld_out % 4 == 0;
  k.o32vec = d->out32 && al16(d->out32) && d->ld_out32 % 4 == 0;
  TH_CHECK_ARG(al16(d->gain), "th_rmsnorm: gain must be 16-byte aligned");
  const dim3 grid((unsigned)cdiv(d->M, 4));
  hipStream_t s = (hipStream_t)stream;
  const int nsel = nch <= 64 ? 1 : nch <= 128 ? 2 : nch <= 256 ? 4 : nch <= 512 ? 8 : nch <= 1024 ? 16 : 0;
  const bool xb = d->x_dtype == TH_BF16;
#define TH_NORM_LAUNCH(N_)                                                     \
  do {                                                                         \
    if (xb)                                                                    \
      hipLaunchKernelGGL((rmsnorm_kernel<N_, true>), grid, dim3(256), 0, s, k);  \
    else                                                                       \
      hipLaunchKernelGGL((rmsnorm_kernel<N_, false>), grid, dim3(256), 0, s, k); \
  } while (0)
  switch (nsel) {
    case 1: TH_NORM_LAUNCH(1); break;
    case 2: TH_NORM_LAUNCH(2); break;
    case 4: TH_NORM_LAUNCH(4); break;
    case 8: TH_NORM_LAUNCH(8); break;
    case 16: TH_NORM_LAUNCH(16); break;
    default: TH_NORM_LAUNCH(0); break;
  }
#undef TH_NORM_LAUNCH
  TH_CHECK_LAUNCH();
  return TH_OK;
}

extern "C" int th_epilogue_vm(const th_vm_desc* d, void* stream) {
  TH_CHECK_ARG(d != nullptr, "th_epilogue_vm: null descriptor");
  TH_CHECK_ARG(d->M > 0 && d->N > 0, "th_epilogue_vm: M, N must be positive");
  TH_CHECK_ARG(d->n_in >= 0 && d->n_in <= TH_VM_MAX_IN, "th_epilogue_vm: n_in out of range");
  TH_CHECK_ARG(d->n_ops >= 0 && d->n_ops <= TH_VM_MAX_OPS, "th_epilogue_vm: n_ops out of range");
  TH_CHECK_ARG(d->n_out >= 1 && d->n_out <= TH_VM_MAX_OUT, "th_epilogue_vm: n_out out of range");
  TH_CHECK_ARG(d->n_slots >= 1 && d->workspace, "th_epilogue_vm: no workspace");
  for (int i = 0; i < d->n_in; ++i) {
    TH_CHECK_ARG(d->in[i].ptr != nullptr, "th_epilogue_vm: operand %d is null", i);
    TH_CHECK_ARG(d->in[i].dtype == TH_BF16 || d->in[i].dtype == TH_F32, "th_epilogue_vm: operand %d dtype", i);
    TH_CHECK_ARG(d->in[i].ld >= (d->in[i].column ? 1 : d->N), "th_epilogue_vm: operand %d row stride too small", i);
  }
  for (int i = 0; i < d->n_ops; ++i) {
    const th_vm_op& op = d->ops[i];
    TH_CHECK_ARG(op.code >= TH_VM_LOAD && op.code <= TH_VM_COPY, "th_epilogue_vm: op %d code %d", i, op.code);
    TH_CHECK_ARG(op.dst >= 0 && op.dst < d->n_slots, "th_epilogue_vm: op %d dst slot", i);
    if (op.code == TH_VM_LOAD) {
      TH_CHECK_ARG(op.a >= 0 && op.a < d->n_in, "th_epilogue_vm: op %d loads operand %d", i, op.a);
    } else {
      TH_CHECK_ARG(op.a >= 0 && op.a < d->n_slots, "th_epilogue_vm: op %d slot a", i);
      const bool binary = op.code >= TH_VM_ADD && op.code <= TH_VM_POW;
      TH_CHECK_ARG(!binary || op.mode != 0 || (op.b >= 0 && op.b < d->n_slots), "th_epilogue_vm: op %d slot b", i);
    }
  }
  for (int i = 0; i < d->n_out; ++i)
    TH_CHECK_ARG(d->out[i].ptr && d->out[i].slot >= 0 && d->out[i].slot < d->n_slots && d->out[i].ld >= d->N,
                 "th_epilogue_vm: output %d invalid", i);
  if (!device_ready()) {
    set_error("th_epilogue_vm: th_init was not called for the current device");
    return TH_ERR_NOT_INIT;
  }
  hipStream_t s = (hipStream_t)stream;
  const int64_t MN = d->M * d->N;
  const unsigned blocks = (unsigned)std::min<int64_t>(cdiv(MN, 256), 8192);
  auto slot = [&](int i) { return d->workspace + (int64_t)i * MN; };
  for (int i = 0; i < d->n_ops; ++i) {
    const th_vm_op& op = d->ops[i];
    if (op.code == TH_VM_ROW_SUM || op.code == TH_VM_ROW_MAX) {
      hipLaunchKernelGGL(vm_rowred_kernel, dim3((unsigned)d->M), dim3(256), 0, s, (const float*)slot(op.a),
                         slot(op.dst), d->N, op.code == TH_VM_ROW_MAX ? 1 : 0);
    } else {
      VmElemK k{};
      k.code = op.code; k.mode = op.mode; k.scalar = op.scalar; k.M = d->M; k.N = d->N;
      k.dst = slot(op.dst);
      if (op.code == TH_VM_LOAD) {
        k.src = d->in[op.a];
      } else {
        k.a = slot(op.a);
        k.b = (op.mode == 0 && op.b >= 0) ? slot(op.b) : nullptr;
      }
      hipLaunchKernelGGL(vm_elem_kernel, dim3(blocks), dim3(256), 0, s, k);
    }
    TH_CHECK_LAUNCH();
  }
  for (int i = 0; i < d->n_out; ++i) {
    hipLaunchKernelGGL(vm_store_kernel, dim3(blocks), dim3(256), 0, s, (const float*)slot(d->out[i].slot),
                       d->out[i].ptr, d->out[i].ld, d->out[i].dtype, d->M, d->N);
    TH_CHECK_LAUNCH();
  }
  return TH_OK;
}
