// Peak probes of the current device for the hardware spec's "measured" block:
// the dense MFMA rate of the instructions the kernels issue
// (v_mfma_f32_32x32x16_bf16, v_mfma_f32_16x16x32_bf16, v_mfma_f32_32x32x2f32)
// and the HBM stream bandwidth (read only, and copy). Prints one JSON object.
//
// MFMA: every wave runs independent accumulator chains of one instruction
// on register operands (no memory traffic in the loop); the grid is 8
// workgroups of 256 threads per CU, so each SIMD holds several waves and the
// issue rate, not a dependency chain, is what is timed.
// HBM: a 4 GiB buffer (16x the 256 MB Infinity Cache) read with 16-byte loads
// in a grid-stride loop; copy reads one 2 GiB buffer and writes another.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

#define CHECK(x)                                                                   \
  do {                                                                             \
    hipError_t e_ = (x);                                                           \
    if (e_ != hipSuccess) {                                                        \
      fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));             \
      exit(1);                                                                     \
    }                                                                              \
  } while (0)

// independent accumulator chains per wave: 4 for the 32x32 forms, 8 for the
// shorter 16x16 one (whose result is ready sooner)
constexpr int NCH = 4, NCH16 = 8;

template <int KIND>
__global__ void __launch_bounds__(256) mfma_rate(float* out, int iters) {
  const int lane = threadIdx.x & 63;
  float seed = 1e-3f * (float)(lane & 7);
  if constexpr (KIND == 0 || KIND == 1) {
    bf16x8_t a, b;
    for (int i = 0; i < 8; ++i) {
      a[i] = (__bf16)(seed + 1e-4f * i);
      b[i] = (__bf16)(seed - 1e-4f * i);
    }
    if constexpr (KIND == 0) {
      f32x16_t acc[NCH] = {};
      for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int c = 0; c < NCH; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
      }
      float s = 0.f;
      for (int c = 0; c < NCH; ++c)
        for (int r = 0; r < 16; ++r) s += acc[c][r];
      out[blockIdx.x * blockDim.x + threadIdx.x] = s;
    } else {
      f32x4_t acc[NCH16] = {};
      for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int c = 0; c < NCH16; ++c) acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[c], 0, 0, 0);
      }
      float s = 0.f;
      for (int c = 0; c < NCH16; ++c)
        for (int r = 0; r < 4; ++r) s += acc[c][r];
      out[blockIdx.x * blockDim.x + threadIdx.x] = s;
    }
  } else {
    f32x16_t acc[NCH] = {};
    const float a = seed, b = seed * 0.5f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int c = 0; c < NCH; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[c], 0, 0, 0);
    }
    float s = 0.f;
    for (int c = 0; c < NCH; ++c)
      for (int r = 0; r < 16; ++r) s += acc[c][r];
    out[blockIdx.x * blockDim.x + threadIdx.x] = s;
  }
}

// Grid-stride 16-byte reads; one XOR per workgroup thread is stored so the
// loads stay live.
__global__ void __launch_bounds__(256) stream_read(const uint4* __restrict__ src, int64_t n, uint32_t* out) {
  uint32_t x = 0;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint4 v = src[i];
    x ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  out[blockIdx.x * blockDim.x + threadIdx.x] = x;
}

__global__ void __launch_bounds__(256) stream_copy(const uint4* __restrict__ src, uint4* __restrict__ dst, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

__global__ void fill(uint4* p, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    p[i] = make_uint4((uint32_t)i, (uint32_t)(i >> 7), 3u, 5u);
}

// Best of `reps` timed launches of f (after one untimed), in milliseconds.
template <class F>
static float best_ms(F f, int reps) {
  hipEvent_t a, b;
  CHECK(hipEventCreate(&a));
  CHECK(hipEventCreate(&b));
  f();
  CHECK(hipDeviceSynchronize());
  float best = 1e30f;
  for (int r = 0; r < reps; ++r) {
    CHECK(hipEventRecord(a, 0));
    f();
    CHECK(hipEventRecord(b, 0));
    CHECK(hipEventSynchronize(b));
    float ms = 0.f;
    CHECK(hipEventElapsedTime(&ms, a, b));
    best = std::min(best, ms);
  }
  CHECK(hipEventDestroy(a));
  CHECK(hipEventDestroy(b));
  return best;
}

int main() {
  hipDeviceProp_t prop;
  CHECK(hipGetDeviceProperties(&prop, 0));
  const int cus = prop.multiProcessorCount;
  const int blocks = cus * 8, threads = 256, iters = 20000;
  float* out;
  CHECK(hipMalloc(&out, (size_t)blocks * threads * sizeof(float)));
  const double waves = (double)blocks * threads / 64;
  // flops per instruction: 2 M N K
  const double f32x32x16 = 2.0 * 32 * 32 * 16, f16x16x32 = 2.0 * 16 * 16 * 32, f32x32x2 = 2.0 * 32 * 32 * 2;
  const float t0 = best_ms([&] { mfma_rate<0><<<blocks, threads>>>(out, iters); }, 3);
  const float t1 = best_ms([&] { mfma_rate<1><<<blocks, threads>>>(out, iters / 2); }, 3);
  const float t2 = best_ms([&] { mfma_rate<2><<<blocks, threads>>>(out, iters / 4); }, 3);
  const double bf16_32 = waves * iters * NCH * f32x32x16 / (t0 * 1e-3) / 1e12;
  const double bf16_16 = waves * (iters / 2) * NCH16 * f16x16x32 / (t1 * 1e-3) / 1e12;
  const double f32_32 = waves * (iters / 4) * NCH * f32x32x2 / (t2 * 1e-3) / 1e12;

  const int64_t read_bytes = (int64_t)4 << 30, copy_bytes = (int64_t)2 << 30;
  uint4 *src, *dst;
  uint32_t* sink;
  CHECK(hipMalloc(&src, read_bytes));
  CHECK(hipMalloc(&dst, copy_bytes));
  const int sblocks = cus * 16;
  CHECK(hipMalloc(&sink, (size_t)sblocks * threads * sizeof(uint32_t)));
  fill<<<sblocks, threads>>>(src, read_bytes / 16);
  CHECK(hipGetLastError());
  const float tr = best_ms([&] { stream_read<<<sblocks, threads>>>(src, read_bytes / 16, sink); }, 10);
  const float tc = best_ms([&] { stream_copy<<<sblocks, threads>>>(src, dst, copy_bytes / 16); }, 10);
  CHECK(hipGetLastError());
  CHECK(hipDeviceSynchronize());
  printf("{\"device\": \"%s\", \"compute_units\": %d, \"clock_mhz\": %d, "
         "\"mfma_tflops\": {\"bfloat16_32x32x16\": %.1f, \"bfloat16_16x16x32\": %.1f, \"float32_32x32x2\": %.1f}, "
         "\"hbm_read_gbs\": %.0f, \"hbm_copy_gbs\": %.0f, "
         "\"method\": \"MFMA: %d workgroups x 256 threads, %d (32x32) or %d (16x16) independent accumulators per wave, register "
         "operands, best of 3; HBM: 16-byte grid-stride loads over a 4 GiB buffer (read) and a 2 GiB to 2 GiB "
         "copy (read + write bytes), %d workgroups, best of 10\"}\n",
         prop.gcnArchName, cus, prop.clockRate / 1000, bf16_32, bf16_16, f32_32, read_bytes / (tr * 1e-3) / 1e9,
         2.0 * copy_bytes / (tc * 1e-3) / 1e9, blocks, NCH, NCH16, sblocks);
  CHECK(hipFree(src));
  CHECK(hipFree(dst));
  CHECK(hipFree(sink));
  CHECK(hipFree(out));
  return 0;
}
