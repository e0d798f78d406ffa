// Shared device/host helpers for the gfx950 kernels of libth_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "th_hip.h"

namespace th {

// MFMA operand / accumulator vector types (CDNA4 v_mfma_*_bf16 take 8 bf16
// per lane; the 32x32 variants return 16 fp32 per lane).
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Wait until at most N of this wave's vector-memory operations (loads, stores,
// direct-to-LDS loads; they retire in issue order) are outstanding.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  // s_waitcnt fields (gfx9): vmcnt[3:0], expcnt[6:4], lgkmcnt[11:8], vmcnt_hi[15:14]
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Wait until this wave's LDS accesses have completed (ds_write results are
// visible to the other waves once they pass the next barrier).
__device__ __forceinline__ void wait_lgkmcnt0() {
  // vmcnt and expcnt at their maxima (no wait), lgkmcnt 0
  __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));
}

// Direct-to-LDS load of 16 bytes per lane (global_load_lds_dwordx4): lane l's
// 16 bytes at base + voff land at LDS byte address lds + 16 l; base and lds
// are wave-uniform. Inline assembly rather than __builtin_amdgcn_global_load_lds:
// the compiler counts the builtin's LDS write among the LDS operations its own
// waits cover, so each wait it inserts for an ordinary LDS read turns into a
// wait for all of them (lgkmcnt(0)), exposing the latency of fragment reads
// issued a step ahead of their MFMAs. The compiler does not track this load:
// the caller waits for it (wait_vmcnt) before anything reads its destination
// and before the workgroup ends. The LDS address goes in through an "{m0}"
// operand, so the compiler itself writes M0 (and knows it is in use) rather
// than relying on a clobber of a reserved register.
__device__ __forceinline__ void dma_load16(const void* base, uint32_t voff, uint32_t lds) {
  // s_nop: one wait state between the compiler's M0 write, which it cannot
  // see is read by the load inside the statement, and the load.
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "{m0}"(lds) : "memory");
}

// Workgroup barrier that leaves global loads in flight (__syncthreads, and
// even an LDS-only workgroup fence once direct-to-LDS loads are pending,
// drain all of them). The wavefront-scope fences only keep the compiler from
// moving memory accesses across the barrier; the caller provides what the
// hardware needs: each wave has consumed its earlier LDS reads (their values
// were used before the barrier) and has waited, with wait_vmcnt, for its own
// direct-to-LDS loads whose data other waves read after the barrier.
__device__ __forceinline__ void barrier_keep_loads() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Workgroup barrier for reuse of LDS only: this wave's LDS accesses complete,
// then the barrier. Unlike __syncthreads it does not wait for the wave's
// global stores (on gfx9 a store counts in vmcnt until the memory system
// acknowledges it, microseconds under load): an epilogue that stages tiles
// through LDS keeps its stores draining while it moves on.
__device__ __forceinline__ void lds_barrier() {
  wait_lgkmcnt0();
  barrier_keep_loads();
}

// ------------------------------------------------------------ bf16 helpers
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}

// Round-to-nearest-even fp32 -> bf16 (what torch's .to(bfloat16) does; NaN
// stays a quiet NaN). The cast compiles to gfx950's v_cvt_pk_bf16_f32 (see
// pk_bf16x2 for a pair in one instruction): epilogues are VALU-bound, and the
// bit arithmetic this replaces took about six instructions per value.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// Two fp32 -> one packed bf16 pair (a in the low half), round to nearest even,
// in one v_cvt_pk_bf16_f32 (two single casts cost a shift and an OR besides).
__device__ __forceinline__ uint32_t pk_bf16x2(float a, float b) {
  typedef float f2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 b2_t __attribute__((ext_vector_type(2)));
  const f2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, b2_t));
}

__device__ __forceinline__ float load_elem(const void* p, int64_t i, int dtype) {
  if (dtype == TH_BF16) return bf16_to_f32(((const uint16_t*)p)[i]);
  return ((const float*)p)[i];
}

__device__ __forceinline__ void store_elem(void* p, int64_t i, int dtype, float v) {
  if (dtype == TH_BF16)
    ((uint16_t*)p)[i] = f32_to_bf16(v);
  else
    ((float*)p)[i] = v;
}

// 1 / (1 + e^-x) with the hardware reciprocal (v_rcp_f32, 1 ulp) instead of an
// IEEE division sequence: these run once per output element of GEMM epilogues
__device__ __forceinline__ float sigmoidf_(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }
// log(1 + exp(x)) without a large-x guard: the OpIR softplus rewrite drops
// torch's threshold, so this is the value the program defines.
__device__ __forceinline__ float softplusf_(float x) { return __logf(1.f + __expf(x)); }

// --------------------------------------------------------------- host side
void set_error(const char* fmt, ...);
bool device_ready();  // th_init was called for the current device
int device_cus();     // compute units of the current device (0 before th_init)
int ssd_init_device();  // per-device set-up of the scan kernels (called by th_init)
int fp8_scratch_init_device(int device);  // per-device address of th_gemm_noalloc's scratch (th_init)

#define TH_CHECK_ARG(cond, ...)            \
  do {                                     \
    if (!(cond)) {                         \
      ::th::set_error(__VA_ARGS__);        \
      return TH_ERR_INVALID;               \
    }                                      \
  } while (0)

#define TH_CHECK_HIP(expr)                                                     \
  do {                                                                         \
    hipError_t e_ = (expr);                                                    \
    if (e_ != hipSuccess) {                                                    \
      ::th::set_error("%s failed: %s", #expr, hipGetErrorString(e_));          \
      return TH_ERR_HIP;                                                       \
    }                                                                          \
  } while (0)

#define TH_CHECK_LAUNCH()                                                      \
  do {                                                                         \
    hipError_t e_ = hipGetLastError();                                         \
    if (e_ != hipSuccess) {                                                    \
      ::th::set_error("kernel launch failed: %s", hipGetErrorString(e_));      \
      return TH_ERR_HIP;                                                       \
    }                                                                          \
  } while (0)

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace th
