// Host-side launchers for one generated plan: the per-plan kernel set that
// the C ABI dispatches to.  Included by each generated tp_<plan>.hip file.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>

#include "o2mi_tp.hpp"

namespace o2mi {

// Kernel variants of one plan.
enum TPVariant : int {
  kVariantChannelMajorVec2 = 0,  // layout 0, 8-byte aligned rows: float2 accesses
  kVariantChannelMajor = 1,      // layout 0, any alignment
  kVariantComponentMajor = 2,    // layouts 1 and 2
  kNumVariants = 3,
};

struct TPTableView {
  int m_max, full, normalization;
  int n_keys, n_paths, n_terms, n_units;
  const KeySpec* keys;
  const PathSpec* paths;
  const TermSpec* terms;
};

using TPForwardFn = hipError_t (*)(int variant, const float* x, const float* y, const float* w,
                                   float* out, const TPGeom& g, int grid, hipStream_t stream);
using TPBackwardFn = hipError_t (*)(int variant, const float* x, const float* y, const float* w,
                                    const float* gout, float* dx, float* dy, float* partial,
                                    const TPGeom& g, int grid, int needed, hipStream_t stream);
using TPOccupancyFn = int (*)(int variant, bool backward);

struct TPKernelSet {
  TPTableView table;
  TPForwardFn forward;
  TPBackwardFn backward;
  TPOccupancyFn blocks_per_cu;
  int backward_tile;  // lanes of a row per backward block (backward_tile<P>())
  int forward_block;  // threads per forward block (forward_block<P>())
  int forward_tile;   // lanes of a row per forward block (forward_tile<P>())
};

// Sets the dynamic-LDS limit of `kernel` once per device (the backward uses
// more than the 64 KiB default).
inline hipError_t allow_lds(const void* kernel, size_t bytes, std::atomic<uint64_t>& done) {
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return err;
  const uint64_t bit = 1ull << (device & 63);
  if (done.load(std::memory_order_acquire) & bit) return hipSuccess;
  err = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (err == hipSuccess) done.fetch_or(bit, std::memory_order_acq_rel);
  return err;
}

template <class P, int kLayout, bool kVec2>
hipError_t launch_forward(const float* x, const float* y, const float* w, float* out,
                          const TPGeom& g, int grid, hipStream_t stream) {
  static std::atomic<uint64_t> done{0};
  const void* kernel = reinterpret_cast<const void*>(&tp_forward_kernel<P, kLayout, kVec2>);
  const size_t lds = forward_lds<P>() ? lds_bytes<P, forward_tile<P>()>() : 0;
  if (lds > 0) {
    const hipError_t err = allow_lds(kernel, lds, done);
    if (err != hipSuccess) return err;
  }
  hipLaunchKernelGGL((tp_forward_kernel<P, kLayout, kVec2>), dim3(grid), dim3(forward_block<P>()),
                     lds, stream, x, y, w, out, g);
  return hipGetLastError();
}

template <class P, int kLayout, bool kVec2>
hipError_t launch_backward(const float* x, const float* y, const float* w, const float* gout,
                           float* dx, float* dy, float* partial, const TPGeom& g, int grid,
                           int needed, hipStream_t stream) {
  static std::atomic<uint64_t> done{0};
  const void* kernel = reinterpret_cast<const void*>(&tp_backward_kernel<P, kLayout, kVec2>);
  const size_t lds = lds_bytes<P, backward_tile<P>()>();
  hipError_t err = allow_lds(kernel, lds, done);
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL((tp_backward_kernel<P, kLayout, kVec2>), dim3(grid), dim3(kBackwardBlock), lds,
                     stream, x, y, w, gout, dx, dy, partial, g, needed);
  return hipGetLastError();
}

template <class P>
hipError_t forward_dispatch(int variant, const float* x, const float* y, const float* w,
                            float* out, const TPGeom& g, int grid, hipStream_t stream) {
  switch (variant) {
    case kVariantChannelMajorVec2:
      return launch_forward<P, 0, true>(x, y, w, out, g, grid, stream);
    case kVariantChannelMajor:
      return launch_forward<P, 0, false>(x, y, w, out, g, grid, stream);
    default:
      return launch_forward<P, 1, false>(x, y, w, out, g, grid, stream);
  }
}

template <class P>
hipError_t backward_dispatch(int variant, const float* x, const float* y, const float* w,
                             const float* gout, float* dx, float* dy, float* partial,
                             const TPGeom& g, int grid, int needed, hipStream_t stream) {
  switch (variant) {
    case kVariantChannelMajorVec2:
      return launch_backward<P, 0, true>(x, y, w, gout, dx, dy, partial, g, grid, needed, stream);
    case kVariantChannelMajor:
      return launch_backward<P, 0, false>(x, y, w, gout, dx, dy, partial, g, grid, needed, stream);
    default:
      return launch_backward<P, 1, false>(x, y, w, gout, dx, dy, partial, g, grid, needed, stream);
  }
}

template <class P, int kLayout, bool kVec2>
int occupancy_of(bool backward) {
  int blocks = 0;
  static std::atomic<uint64_t> done_f{0}, done_b{0};
  if (backward) {
    const void* kernel = reinterpret_cast<const void*>(&tp_backward_kernel<P, kLayout, kVec2>);
    const size_t lds = lds_bytes<P, backward_tile<P>()>();
    if (allow_lds(kernel, lds, done_b) != hipSuccess) return 1;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &blocks, tp_backward_kernel<P, kLayout, kVec2>, kBackwardBlock, lds) != hipSuccess)
      return 1;
  } else {
    const void* kernel = reinterpret_cast<const void*>(&tp_forward_kernel<P, kLayout, kVec2>);
    const size_t lds = forward_lds<P>() ? lds_bytes<P, forward_tile<P>()>() : 0;
    if (lds > 0 && allow_lds(kernel, lds, done_f) != hipSuccess) return 1;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &blocks, tp_forward_kernel<P, kLayout, kVec2>, forward_block<P>(), lds) != hipSuccess)
      return 1;
  }
  return blocks > 0 ? blocks : 1;
}

template <class P>
int occupancy_dispatch(int variant, bool backward) {
  switch (variant) {
    case kVariantChannelMajorVec2:
      return occupancy_of<P, 0, true>(backward);
    case kVariantChannelMajor:
      return occupancy_of<P, 0, false>(backward);
    default:
      return occupancy_of<P, 1, false>(backward);
  }
}

template <class P>
const TPKernelSet* tp_kernel_set() {
  static const TPKernelSet set = {
      {P::kM, P::kFull ? 1 : 0, P::kNorm, P::kKeys, P::kPaths, P::kTerms, P::kUnits, P::keys,
       P::paths, P::terms},
      &forward_dispatch<P>,
      &backward_dispatch<P>,
      &occupancy_dispatch<P>,
      backward_tile<P>(),
      forward_block<P>(),
      forward_tile<P>(),
  };
  return &set;
}

}  // namespace o2mi

#define O2MI_DEFINE_TP_SET(NAME) \
  const o2mi::TPKernelSet* o2mi_tp_set_##NAME() { return o2mi::tp_kernel_set<o2mi::plans::NAME>(); }
