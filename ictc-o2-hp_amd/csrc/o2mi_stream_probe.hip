// HBM streaming ceilings of the running GPU for the TP kernels' traffic mixes.
//
// The fused backward reads three [N, W] f32 tensors and writes two; the
// forward reads two and writes one.  This probe streams exactly those mixes
// with plain kernels -- rows of W floats, block b taking rows b, b + G, ...,
// non-temporal loads and stores, each thread loading its share of a row with
// 4- or 8-byte accesses -- over 1..8 blocks of 256 threads per CU, and prints
// one JSON object with the best GB/s of each mix (min of 5 timed launches per
// configuration).  It measures what the memory system delivers for these
// mixes; the kernels are judged against it next to the 8 TB/s nominal peak.
//
// Usage: o2mi_stream_probe [rows] [width]   (defaults 131072, 3328)
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <string>

namespace {

using f2 = float __attribute__((ext_vector_type(2)));

#define PROBE_CHECK(x)                                                          \
  do {                                                                          \
    hipError_t e_ = (x);                                                        \
    if (e_ != hipSuccess) {                                                     \
      std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));              \
      std::exit(1);                                                             \
    }                                                                           \
  } while (0)

// T elements per access; the row has `vecs` of them; PER covers a row with 256
// threads (guarded).  Rows of the same index in every tensor, like the TP kernels.
template <class T, int PER>
__global__ __launch_bounds__(256) void r3w2(const T* __restrict__ x, const T* __restrict__ y,
                                            const T* __restrict__ g, T* __restrict__ o1,
                                            T* __restrict__ o2, int n_rows, int vecs) {
  for (int r = blockIdx.x; r < n_rows; r += gridDim.x) {
    const size_t base = (size_t)r * vecs;
    T a[PER], b[PER], c[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int e = k * 256 + threadIdx.x;
      if (e < vecs) {
        a[k] = __builtin_nontemporal_load(x + base + e);
        b[k] = __builtin_nontemporal_load(y + base + e);
        c[k] = __builtin_nontemporal_load(g + base + e);
      }
    }
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int e = k * 256 + threadIdx.x;
      if (e < vecs) {
        __builtin_nontemporal_store(a[k] * c[k] + b[k], o1 + base + e);
        __builtin_nontemporal_store(b[k] * c[k] + a[k], o2 + base + e);
      }
    }
  }
}

template <class T, int PER>
__global__ __launch_bounds__(256) void r2w1(const T* __restrict__ x, const T* __restrict__ y,
                                            T* __restrict__ o1, int n_rows, int vecs) {
  for (int r = blockIdx.x; r < n_rows; r += gridDim.x) {
    const size_t base = (size_t)r * vecs;
    T a[PER], b[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int e = k * 256 + threadIdx.x;
      if (e < vecs) {
        a[k] = __builtin_nontemporal_load(x + base + e);
        b[k] = __builtin_nontemporal_load(y + base + e);
      }
    }
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int e = k * 256 + threadIdx.x;
      if (e < vecs) __builtin_nontemporal_store(a[k] * b[k], o1 + base + e);
    }
  }
}

template <class F>
float best_ms(F&& launch) {
  hipEvent_t e0, e1;
  PROBE_CHECK(hipEventCreate(&e0));
  PROBE_CHECK(hipEventCreate(&e1));
  launch();
  float best = 1e30f;
  for (int rep = 0; rep < 5; ++rep) {
    PROBE_CHECK(hipEventRecord(e0));
    launch();
    PROBE_CHECK(hipEventRecord(e1));
    PROBE_CHECK(hipEventSynchronize(e1));
    float ms = 0.f;
    PROBE_CHECK(hipEventElapsedTime(&ms, e0, e1));
    if (ms < best) best = ms;
  }
  PROBE_CHECK(hipEventDestroy(e0));
  PROBE_CHECK(hipEventDestroy(e1));
  return best;
}

struct Best {
  double gbs = 0.0;
  int width_bytes = 0, blocks_per_cu = 0;
};

template <class T, int PER>
void sweep(float* const* buf, int n_rows, int width, int cus, Best* b3, Best* b2) {
  const int vecs = width * 4 / (int)sizeof(T);
  const double tensor_gb = (double)n_rows * width * 4 / 1e9;
  const T* const* in = reinterpret_cast<const T* const*>(buf);
  T* const* out = reinterpret_cast<T* const*>(buf);
  for (int per_cu : {1, 2, 3, 4, 6, 8}) {
    const int grid = per_cu * cus;
    const float t3 = best_ms([&] {
      hipLaunchKernelGGL((r3w2<T, PER>), dim3(grid), dim3(256), 0, 0, in[0], in[1], in[2], out[3],
                         out[4], n_rows, vecs);
    });
    const float t2 = best_ms([&] {
      hipLaunchKernelGGL((r2w1<T, PER>), dim3(grid), dim3(256), 0, 0, in[0], in[1], out[3],
                         n_rows, vecs);
    });
    PROBE_CHECK(hipGetLastError());
    const double g3 = 5 * tensor_gb / (t3 * 1e-3), g2 = 3 * tensor_gb / (t2 * 1e-3);
    if (g3 > b3->gbs) *b3 = {g3, (int)sizeof(T), per_cu};
    if (g2 > b2->gbs) *b2 = {g2, (int)sizeof(T), per_cu};
  }
}

}  // namespace

int main(int argc, char** argv) {
  const int n_rows = argc > 1 ? std::atoi(argv[1]) : 131072;
  const int width = argc > 2 ? std::atoi(argv[2]) : 3328;
  // Each thread covers up to 16 floats (4-byte) or 8 float pairs of a row.
  if (n_rows <= 0 || width <= 0 || width % 2 != 0 || width > 16 * 256) {
    std::fprintf(stderr, "need rows > 0 and an even width <= 4096\n");
    return 2;
  }
  hipDeviceProp_t prop;
  PROBE_CHECK(hipGetDeviceProperties(&prop, 0));
  float* buf[5];
  const size_t bytes = (size_t)n_rows * width * 4;
  for (auto& p : buf) {
    PROBE_CHECK(hipMalloc(&p, bytes));
    PROBE_CHECK(hipMemset(p, 0, bytes));
  }
  Best b3, b2;
  sweep<float, 16>(buf, n_rows, width, prop.multiProcessorCount, &b3, &b2);
  sweep<f2, 8>(buf, n_rows, width, prop.multiProcessorCount, &b3, &b2);
  for (auto p : buf) PROBE_CHECK(hipFree(p));
  std::printf(
      "{\"device\": \"%s\", \"cus\": %d, \"rows\": %d, \"width\": %d, "
      "\"read3_write2_GBps\": %.1f, \"read3_write2_access_bytes\": %d, "
      "\"read3_write2_blocks_per_cu\": %d, \"read2_write1_GBps\": %.1f, "
      "\"read2_write1_access_bytes\": %d, \"read2_write1_blocks_per_cu\": %d}\n",
      prop.gcnArchName, prop.multiProcessorCount, n_rows, width, b3.gbs, b3.width_bytes,
      b3.blocks_per_cu, b2.gbs, b2.width_bytes, b2.blocks_per_cu);
  return 0;
}
