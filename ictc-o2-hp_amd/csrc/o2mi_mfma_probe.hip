// fp32 matrix-core issue probe: how much MFMA time VALU instructions cost on
// the running GPU, the figure that bounds the radial kernels (their affine
// map runs on v_mfma_f32_16x16x4_f32, their uvu products on the VALU).
//
// One block of 8 waves per CU (two waves per SIMD), everything in registers,
// one store per lane.  Each wave that issues MFMAs runs iterations of 32
// independent v_mfma_f32_16x16x4_f32 (32 accumulators).  Patterns:
//   mfma              every wave issues MFMAs only;
//   clustered K       every wave issues K VALU FMAs, then its 32 MFMAs;
//   interleaved K     every wave issues K/32 VALU FMAs after each MFMA;
//   other-wave K      waves 0-3 (one per SIMD) issue MFMAs only, waves 4-7
//                     (the SIMD's other wave) K VALU FMAs per iteration.
// The VALU FMAs run on 8 independent registers and never touch the MFMA
// operands.  Prints TFLOP/s of the MFMA waves and the share of the 157.3
// TFLOP/s fp32 matrix peak for each pattern.
//
// Usage: o2mi_mfma_probe [iterations]
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

namespace {

using f4 = float __attribute__((ext_vector_type(4)));

constexpr int kBlocks = 256;
constexpr int kThreads = 512;
constexpr double kPeak = 157.3;  // TFLOP/s, MI355X fp32 matrix

enum Pattern { kMfmaOnly, kClustered, kInterleaved, kOtherWave };

__device__ __forceinline__ void valu_fma(float& x, float y) {
  asm volatile("v_fma_f32 %0, %1, %0, %1" : "+v"(x) : "v"(y));
}

template <int kPattern, int K>
__global__ __launch_bounds__(kThreads, 1) void probe_kernel(float* out, int iters) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool mfma_wave = kPattern != kOtherWave || wave < 4;
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = 0.5f * i;
  const float a = threadIdx.x * 1e-3f, b = 1.0f - threadIdx.x * 1e-4f;
  float s = 0.f;
  if (mfma_wave) {
    f4 acc[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) acc[i] = f4{0.f, 0.f, 0.f, 0.f};
    for (int it = 0; it < iters; ++it) {
      if constexpr (kPattern == kClustered) {
#pragma unroll
        for (int i = 0; i < K; ++i) valu_fma(v[i & 7], b);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[i], 0, 0, 0);
        if constexpr (kPattern == kInterleaved) {
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int q = 0; q < K / 32; ++q) valu_fma(v[(i + q) & 7], b);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) s += acc[i].x + acc[i].y + acc[i].z + acc[i].w;
  } else {
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int i = 0; i < K; ++i) valu_fma(v[i & 7], b);
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) s += v[i];
  out[blockIdx.x * kThreads + threadIdx.x] = s;
}

#define PROBE_CHECK(x)                                                          \
  do {                                                                          \
    hipError_t e_ = (x);                                                        \
    if (e_ != hipSuccess) {                                                     \
      std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));              \
      std::exit(2);                                                             \
    }                                                                           \
  } while (0)

template <int kPattern, int K>
void run(float* out, int iters, const char* name) {
  hipEvent_t e0, e1;
  PROBE_CHECK(hipEventCreate(&e0));
  PROBE_CHECK(hipEventCreate(&e1));
  hipLaunchKernelGGL((probe_kernel<kPattern, K>), dim3(kBlocks), dim3(kThreads), 0, 0, out, 10);
  PROBE_CHECK(hipGetLastError());
  PROBE_CHECK(hipEventRecord(e0));
  hipLaunchKernelGGL((probe_kernel<kPattern, K>), dim3(kBlocks), dim3(kThreads), 0, 0, out, iters);
  PROBE_CHECK(hipGetLastError());
  PROBE_CHECK(hipEventRecord(e1));
  PROBE_CHECK(hipEventSynchronize(e1));
  float ms = 0.f;
  PROBE_CHECK(hipEventElapsedTime(&ms, e0, e1));
  const int mfma_waves = kPattern == kOtherWave ? 4 : 8;
  const double flop = (double)kBlocks * mfma_waves * iters * 32 * 2048.0;
  const double tf = flop / ms / 1e9;
  std::printf("{\"pattern\": \"%s\", \"valu_per_32_mfma\": %d, \"ms\": %.4f, \"tflops\": %.1f, "
              "\"frac\": %.3f}\n", name, K, ms, tf, tf / kPeak);
  PROBE_CHECK(hipEventDestroy(e0));
  PROBE_CHECK(hipEventDestroy(e1));
}

}  // namespace

int main(int argc, char** argv) {
  const int iters = argc > 1 ? std::atoi(argv[1]) : 2000;
  if (iters <= 0) {
    std::fprintf(stderr, "iterations must be positive\n");
    return 1;
  }
  float* out = nullptr;
  PROBE_CHECK(hipMalloc(&out, sizeof(float) * kBlocks * kThreads));
  run<kMfmaOnly, 0>(out, iters, "mfma");
  run<kClustered, 32>(out, iters, "clustered");
  run<kClustered, 64>(out, iters, "clustered");
  run<kClustered, 128>(out, iters, "clustered");
  run<kInterleaved, 32>(out, iters, "interleaved");
  run<kInterleaved, 64>(out, iters, "interleaved");
  run<kInterleaved, 128>(out, iters, "interleaved");
  run<kOtherWave, 32>(out, iters, "other-wave");
  run<kOtherWave, 64>(out, iters, "other-wave");
  run<kOtherWave, 128>(out, iters, "other-wave");
  PROBE_CHECK(hipDeviceSynchronize());
  PROBE_CHECK(hipFree(out));
  return 0;
}
