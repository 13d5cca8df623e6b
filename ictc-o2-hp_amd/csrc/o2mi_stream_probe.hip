// HBM streaming ceilings of the running GPU for the TP kernels' traffic mixes.
//
// The fused backward reads three [N, W] f32 tensors and writes two; the
// forward reads two and writes one.  This probe streams exactly those mixes
// with plain kernels: block b takes row chunks b, b + G, b + 2G, ... (R rows
// of W floats per chunk, the same chunk in every tensor, like the TP kernels),
// each thread loading its share of a chunk with 4-, 8- or 16-byte
// non-temporal accesses, all loads of a chunk before its stores.  It sweeps
// access width x rows per chunk (R = 1, 2, 4) x 1..8 blocks of 256 threads per
// CU and reports the best configuration's GB/s for each mix, each
// configuration timed as the median of 7 launches (a minimum let one launch
// timed short set a ceiling 10% above every other reading).  It measures what the memory system delivers for these
// mixes; the kernels are judged against it next to the 8 TB/s nominal peak.
//
// Usage: o2mi_stream_probe [rows] [width] [--table]
//   --table  also prints one JSON line per configuration before the summary.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>

namespace {

using f2 = float __attribute__((ext_vector_type(2)));
using f4 = float __attribute__((ext_vector_type(4)));

#define PROBE_CHECK(x)                                                          \
  do {                                                                          \
    hipError_t e_ = (x);                                                        \
    if (e_ != hipSuccess) {                                                     \
      std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));              \
      std::exit(1);                                                             \
    }                                                                           \
  } while (0)

constexpr int kThreads = 256;

// One chunk holds `vecs` elements of type T per tensor (R rows; the last chunk
// may hold fewer rows: `last_vecs`).  Thread t covers elements t, t + 256, ...
// (PER of them, guarded).
template <class T, int PER>
__global__ __launch_bounds__(kThreads) void r3w2(const T* __restrict__ x,
                                                 const T* __restrict__ y,
                                                 const T* __restrict__ g, T* __restrict__ o1,
                                                 T* __restrict__ o2, int chunks, int vecs,
                                                 int last_vecs) {
  for (int r = blockIdx.x; r < chunks; r += gridDim.x) {
    const size_t base = (size_t)r * vecs;
    const int n = r == chunks - 1 ? last_vecs : vecs;
    T a[PER], b[PER], c[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int e = k * kThreads + threadIdx.x;
      if (e < n) {
        a[k] = __builtin_nontemporal_load(x + base + e);
        b[k] = __builtin_nontemporal_load(y + base + e);
        c[k] = __builtin_nontemporal_load(g + base + e);
      }
    }
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int e = k * kThreads + threadIdx.x;
      if (e < n) {
        __builtin_nontemporal_store(a[k] * c[k] + b[k], o1 + base + e);
        __builtin_nontemporal_store(b[k] * c[k] + a[k], o2 + base + e);
      }
    }
  }
}

template <class T, int PER>
__global__ __launch_bounds__(kThreads) void r2w1(const T* __restrict__ x,
                                                 const T* __restrict__ y, T* __restrict__ o1,
                                                 int chunks, int vecs, int last_vecs) {
  for (int r = blockIdx.x; r < chunks; r += gridDim.x) {
    const size_t base = (size_t)r * vecs;
    const int n = r == chunks - 1 ? last_vecs : vecs;
    T a[PER], b[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int e = k * kThreads + threadIdx.x;
      if (e < n) {
        a[k] = __builtin_nontemporal_load(x + base + e);
        b[k] = __builtin_nontemporal_load(y + base + e);
      }
    }
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int e = k * kThreads + threadIdx.x;
      if (e < n) __builtin_nontemporal_store(a[k] * b[k], o1 + base + e);
    }
  }
}

template <class F>
float median_ms(F&& launch) {
  constexpr int kReps = 7;
  hipEvent_t e0, e1;
  PROBE_CHECK(hipEventCreate(&e0));
  PROBE_CHECK(hipEventCreate(&e1));
  launch();
  float ms[kReps];
  for (int rep = 0; rep < kReps; ++rep) {
    PROBE_CHECK(hipEventRecord(e0));
    launch();
    PROBE_CHECK(hipEventRecord(e1));
    PROBE_CHECK(hipEventSynchronize(e1));
    PROBE_CHECK(hipEventElapsedTime(&ms[rep], e0, e1));
  }
  PROBE_CHECK(hipEventDestroy(e0));
  PROBE_CHECK(hipEventDestroy(e1));
  for (int i = 1; i < kReps; ++i)  // insertion sort of 7 values
    for (int j = i; j > 0 && ms[j] < ms[j - 1]; --j) {
      const float t = ms[j];
      ms[j] = ms[j - 1];
      ms[j - 1] = t;
    }
  return ms[kReps / 2];
}

struct Best {
  double gbs = 0.0;
  int width_bytes = 0, rows_per_chunk = 0, blocks_per_cu = 0;
};

struct Sweep {
  float* buf[5];
  int n_rows, width, cus;
  bool table;
  Best b3, b2;
};

// One (access type, rows per chunk) combination over 1..8 blocks per CU.
// The caller guarantees PER * 256 >= rows_per_chunk * width * 4 / sizeof(T).
template <class T, int PER>
void sweep(Sweep& s, int rows_per_chunk) {
  const int row_vecs = s.width * 4 / (int)sizeof(T);
  const int vecs = rows_per_chunk * row_vecs;
  const int chunks = (s.n_rows + rows_per_chunk - 1) / rows_per_chunk;
  const int last_vecs = (s.n_rows - (chunks - 1) * rows_per_chunk) * row_vecs;
  const double tensor_gb = (double)s.n_rows * s.width * 4 / 1e9;
  const T* const* in = reinterpret_cast<const T* const*>(s.buf);
  T* const* out = reinterpret_cast<T* const*>(s.buf);
  for (int per_cu : {1, 2, 3, 4, 6, 8}) {
    const int grid = per_cu * s.cus;
    const float t3 = median_ms([&] {
      hipLaunchKernelGGL((r3w2<T, PER>), dim3(grid), dim3(kThreads), 0, 0, in[0], in[1], in[2],
                         out[3], out[4], chunks, vecs, last_vecs);
    });
    const float t2 = median_ms([&] {
      hipLaunchKernelGGL((r2w1<T, PER>), dim3(grid), dim3(kThreads), 0, 0, in[0], in[1],
                         out[3], chunks, vecs, last_vecs);
    });
    PROBE_CHECK(hipGetLastError());
    const double g3 = 5 * tensor_gb / (t3 * 1e-3), g2 = 3 * tensor_gb / (t2 * 1e-3);
    if (s.table)
      std::printf("{\"access_bytes\": %d, \"rows_per_chunk\": %d, \"blocks_per_cu\": %d, "
                  "\"read3_write2_GBps\": %.1f, \"read2_write1_GBps\": %.1f}\n",
                  (int)sizeof(T), rows_per_chunk, per_cu, g3, g2);
    if (g3 > s.b3.gbs) s.b3 = {g3, (int)sizeof(T), rows_per_chunk, per_cu};
    if (g2 > s.b2.gbs) s.b2 = {g2, (int)sizeof(T), rows_per_chunk, per_cu};
  }
}

// Smallest compiled PER that covers a chunk of `vecs` elements (0: none).
template <class T>
void sweep_any(Sweep& s, int rows_per_chunk) {
  const int vecs = rows_per_chunk * (s.width * 4 / (int)sizeof(T));
  const int per = (vecs + kThreads - 1) / kThreads;
  if (per <= 4)
    sweep<T, 4>(s, rows_per_chunk);
  else if (per <= 8)
    sweep<T, 8>(s, rows_per_chunk);
  else if (per <= 13)
    sweep<T, 13>(s, rows_per_chunk);
  else if (per <= 16)
    sweep<T, 16>(s, rows_per_chunk);
}

}  // namespace

int main(int argc, char** argv) {
  int positional[2] = {131072, 3328};
  int npos = 0;
  bool table = false;
  for (int i = 1; i < argc; ++i) {
    if (std::strcmp(argv[i], "--table") == 0)
      table = true;
    else if (npos < 2)
      positional[npos++] = std::atoi(argv[i]);
  }
  const int n_rows = positional[0], width = positional[1];
  // Every access type must divide a row: width a multiple of 4 floats.
  if (n_rows <= 0 || width <= 0 || width % 4 != 0 || width > 16 * kThreads) {
    std::fprintf(stderr, "need rows > 0 and a width that is a multiple of 4, <= 4096\n");
    return 2;
  }
  hipDeviceProp_t prop;
  PROBE_CHECK(hipGetDeviceProperties(&prop, 0));
  Sweep s;
  s.n_rows = n_rows;
  s.width = width;
  s.cus = prop.multiProcessorCount;
  s.table = table;
  const size_t bytes = (size_t)n_rows * width * 4;
  for (auto& p : s.buf) {
    PROBE_CHECK(hipMalloc(&p, bytes));
    PROBE_CHECK(hipMemset(p, 0, bytes));
  }
  for (int rows_per_chunk : {1, 2, 4}) {
    sweep_any<float>(s, rows_per_chunk);
    sweep_any<f2>(s, rows_per_chunk);
    sweep_any<f4>(s, rows_per_chunk);
  }
  for (auto p : s.buf) PROBE_CHECK(hipFree(p));
  std::printf(
      "{\"device\": \"%s\", \"cus\": %d, \"rows\": %d, \"width\": %d, "
      "\"read3_write2_GBps\": %.1f, \"read3_write2_access_bytes\": %d, "
      "\"read3_write2_rows_per_chunk\": %d, \"read3_write2_blocks_per_cu\": %d, "
      "\"read2_write1_GBps\": %.1f, \"read2_write1_access_bytes\": %d, "
      "\"read2_write1_rows_per_chunk\": %d, \"read2_write1_blocks_per_cu\": %d}\n",
      prop.gcnArchName, s.cus, n_rows, width, s.b3.gbs, s.b3.width_bytes, s.b3.rows_per_chunk,
      s.b3.blocks_per_cu, s.b2.gbs, s.b2.width_bytes, s.b2.rows_per_chunk, s.b2.blocks_per_cu);
  return 0;
}
