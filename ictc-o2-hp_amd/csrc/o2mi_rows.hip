// Row gather and deterministic row segment sums for gfx950: the node <-> edge
// data movement around the radial product of a message-passing layer.
//
//   gather:      dst[e, :] = src[index[e], :]        (an index outside the
//                                                      table gives a zero row)
//   segment sum: dst[s, :] = sum over k in [offsets[s], offsets[s+1]) of
//                rows[order[k], :], added in increasing k
//
// The segment sum is the adjoint of the gather when `order` sorts the edges by
// index (stably) and `offsets` delimits each table row's run: it replaces an
// atomic scatter-add with a fixed summation order, so the result is bitwise
// reproducible.  Both are HBM-bound: each row is read once and written once.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include <string>
#include <type_traits>

#include "ictc_o2_hp_amd.h"
#include "o2mi_error.hpp"

namespace o2mi {
namespace rows {
namespace {

using f4 = float __attribute__((ext_vector_type(4)));

int fail(int status, const std::string& message) {
  o2mi_error_slot() = message;
  return status;
}

// One thread per (row, vector column); V floats per vector (1 or 4).
template <int V>
__global__ __launch_bounds__(256) void gather_kernel(const float* __restrict__ src,
                                                     int64_t src_rows,
                                                     const int64_t* __restrict__ index,
                                                     int64_t n_rows, int64_t vecs,
                                                     float* __restrict__ dst) {
  using T = std::conditional_t<V == 4, f4, float>;
  const int64_t items = n_rows * vecs;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < items;
       i += (int64_t)gridDim.x * 256) {
    const int64_t row = i / vecs, c = i - row * vecs;
    const int64_t id = index[row];
    T v{};
    if (id >= 0 && id < src_rows) v = reinterpret_cast<const T*>(src)[id * vecs + c];
    __builtin_nontemporal_store(v, reinterpret_cast<T*>(dst) + i);
  }
}

// One block per segment; the block's threads cover the row in vectors of V
// floats (a loop when a row has more than 256 vectors).  Four source rows are
// loaded before they are added, in order, so four rows are in flight.
template <int V>
__global__ __launch_bounds__(256) void segment_sum_kernel(const float* __restrict__ rows,
                                                          int64_t n_rows, int64_t vecs,
                                                          const int64_t* __restrict__ order,
                                                          const int64_t* __restrict__ offsets,
                                                          int64_t n_segments,
                                                          float* __restrict__ dst) {
  using T = std::conditional_t<V == 4, f4, float>;
  const T* src = reinterpret_cast<const T*>(rows);
  for (int64_t s = blockIdx.x; s < n_segments; s += gridDim.x) {
    // Runs are clamped to [0, n_rows): any offsets stay inside `order`.
    const int64_t lo = offsets[s] < 0 ? 0 : offsets[s];
    const int64_t hi = offsets[s + 1] < n_rows ? offsets[s + 1] : n_rows;
    for (int64_t c = threadIdx.x; c < vecs; c += 256) {
      T acc{};
      int64_t k = lo;
      for (; k + 4 <= hi; k += 4) {
        T v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int64_t r = order[k + u];
          v[u] = T{};
          if (r >= 0 && r < n_rows) v[u] = __builtin_nontemporal_load(src + r * vecs + c);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) acc += v[u];
      }
      for (; k < hi; ++k) {
        const int64_t r = order[k];
        if (r >= 0 && r < n_rows) acc += __builtin_nontemporal_load(src + r * vecs + c);
      }
      reinterpret_cast<T*>(dst)[s * vecs + c] = acc;
    }
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

unsigned grid_for(int64_t items) {
  const int64_t blocks = (items + 255) / 256;
  return (unsigned)(blocks < 65536 ? (blocks > 0 ? blocks : 1) : 65536);
}

}  // namespace
}  // namespace rows
}  // namespace o2mi

using namespace o2mi::rows;

extern "C" {

int o2mi_rows_gather_f32(const float* src, int64_t src_rows, const int64_t* index,
                         int64_t n_rows, int64_t width, float* dst, void* stream) {
  if (n_rows < 0 || src_rows < 0 || width < 0)
    return fail(O2MI_ERR_INVALID_ARGUMENT, "negative size");
  if (n_rows == 0 || width == 0) return O2MI_OK;
  if (!index || !dst || (!src && src_rows > 0))
    return fail(O2MI_ERR_INVALID_ARGUMENT, "NULL pointer");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const bool vec = width % 4 == 0 && aligned16(src) && aligned16(dst);
  const int64_t vecs = vec ? width / 4 : width;
  if (vec)
    hipLaunchKernelGGL(gather_kernel<4>, dim3(grid_for(n_rows * vecs)), dim3(256), 0, s, src,
                       src_rows, index, n_rows, vecs, dst);
  else
    hipLaunchKernelGGL(gather_kernel<1>, dim3(grid_for(n_rows * vecs)), dim3(256), 0, s, src,
                       src_rows, index, n_rows, vecs, dst);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(O2MI_ERR_HIP, std::string("gather launch: ") + hipGetErrorString(err));
  return O2MI_OK;
}

int o2mi_rows_segment_sum_f32(const float* rows, int64_t n_rows, int64_t width,
                              const int64_t* order, const int64_t* offsets, int64_t n_segments,
                              float* dst, void* stream) {
  if (n_rows < 0 || width < 0 || n_segments < 0)
    return fail(O2MI_ERR_INVALID_ARGUMENT, "negative size");
  if (n_segments == 0 || width == 0) return O2MI_OK;
  if (!offsets || !dst || (n_rows > 0 && (!rows || !order)))
    return fail(O2MI_ERR_INVALID_ARGUMENT, "NULL pointer");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const bool vec = width % 4 == 0 && (n_rows == 0 || aligned16(rows)) && aligned16(dst);
  const int64_t vecs = vec ? width / 4 : width;
  const unsigned grid = (unsigned)(n_segments < 1048576 ? n_segments : 1048576);
  if (vec)
    hipLaunchKernelGGL(segment_sum_kernel<4>, dim3(grid), dim3(256), 0, s, rows, n_rows, vecs,
                       order, offsets, n_segments, dst);
  else
    hipLaunchKernelGGL(segment_sum_kernel<1>, dim3(grid), dim3(256), 0, s, rows, n_rows, vecs,
                       order, offsets, n_segments, dst);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return fail(O2MI_ERR_HIP, std::string("segment sum launch: ") + hipGetErrorString(err));
  return O2MI_OK;
}

}  // extern "C"
