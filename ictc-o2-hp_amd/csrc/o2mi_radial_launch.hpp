// Host launchers of the fused radial kernels, one kernel set per plan.
#pragma once

#include <hip/hip_runtime.h>

#include "o2mi_radial.hpp"
#include "o2mi_radial_streamed.hpp"
#include "o2mi_radial_weight.hpp"
#include "o2mi_uvu_vshared.hpp"

namespace o2mi {
namespace radial {

// The uvu product with shared weights and 2 <= V <= 8 (Args::alpha = weights
// [P][C][V], Args::V = V).
struct VSharedLaunchers {
  int dw_edges;   // edges per staged tile of the weight-gradient kernel
  int dw_groups;  // path groups (grid z) of the weight-gradient kernel
  hipError_t (*forward)(const Args&, float* out, hipStream_t);
  hipError_t (*backward)(const Args&, const float* gout, float* gx, float* gy, int needed,
                         hipStream_t);
  hipError_t (*dw)(const Args&, const float* gout, int64_t edges_per_slice, int slices,
                   float* part, hipStream_t);
};

struct KernelSet {
  int paths;
  int comps1;   // components per channel of the first input
  int comps2;   // width of the second input (V = 1)
  int kh;       // hidden width supported: <= 4 * kh
  int weight_edges;   // edges per staged tile of the affine-adjoint kernel
  int weight_groups;  // path groups (grid z) of the affine-adjoint kernel
  int stream_edges;   // edges per block of the forward / input-adjoint kernels
  hipError_t (*forward)(const Args&, float* out, hipStream_t);
  hipError_t (*backward)(const Args&, const float* gout, float* gx, float* gy, float* ghid,
                         int needed, hipStream_t);
  hipError_t (*weight)(const Args&, const float* gout, int64_t edges_per_slice, int slices,
                       float* part_alpha, float* part_bias, hipStream_t);
  // The V = 1 uvu product with shared weights (Args::alpha = weights [P][C]).
  int dw_edges;       // edges per staged tile of the shared-weight gradient kernel
  hipError_t (*shared_forward)(const Args&, float* out, hipStream_t);
  hipError_t (*shared_backward)(const Args&, const float* gout, float* gx, float* gy,
                                int needed, hipStream_t);
  hipError_t (*shared_dw)(const Args&, const float* gout, int64_t edges_per_slice, int slices,
                          float* part, hipStream_t);
  const VSharedLaunchers* vshared;
  // The V = 1 uvu product with per-row weights (Args::alpha = weights [n][P*C]).
  hipError_t (*row_forward)(const Args&, float* out, hipStream_t);
  hipError_t (*row_backward)(const Args&, const float* gout, float* gx, float* gy, float* gw,
                             int needed, hipStream_t);
};

static_assert(kSFwdWaves == kSBwdWaves, "forward and input adjoints share one edge blocking");
constexpr int kStreamEdges = kEdgesPerWave * kSFwdWaves;

// Grid: edge blocks x channel splits (Args::tile_span).
inline dim3 stream_grid(const Args& a) {
  return dim3((unsigned)((a.n + kStreamEdges - 1) / kStreamEdges),
              (unsigned)((a.C + a.tile_span - 1) / a.tile_span));
}

template <class Plan, int KH>
hipError_t launch_forward(const Args& a, float* out, hipStream_t s) {
  hipLaunchKernelGGL((radial_forward_streamed_kernel<Plan, KH>), stream_grid(a),
                     dim3(64 * kSFwdWaves), 0, s, a, out);
  return hipGetLastError();
}

template <class Plan, int KH>
hipError_t launch_backward(const Args& a, const float* gout, float* gx, float* gy, float* ghid,
                           int needed, hipStream_t s) {
  hipLaunchKernelGGL((radial_backward_streamed_kernel<Plan, KH>), stream_grid(a),
                     dim3(64 * kSBwdWaves), 0, s, a, gout, gx, gy, ghid, needed);
  return hipGetLastError();
}

template <class Plan, int KH>
hipError_t launch_weight(const Args& a, const float* gout, int64_t edges_per_slice, int slices,
                         float* part_alpha, float* part_bias, hipStream_t s) {
  if constexpr (Plan::kWgtTwoPhase)
    hipLaunchKernelGGL((radial_weight_gw_kernel<Plan, KH>),
                       dim3((unsigned)slices, (unsigned)(a.C / 16)), dim3(kGwThreads), 0, s, a,
                       gout, edges_per_slice, part_alpha, part_bias);
  else if constexpr (Plan::kWgtStreamed)
    hipLaunchKernelGGL((radial_weight_streamed_kernel<Plan, KH>),
                       dim3((unsigned)slices, (unsigned)(a.C / 16), wgt_groups<Plan>()),
                       dim3(64 * kSWgtWaves), 0, s, a, gout, edges_per_slice, part_alpha,
                       part_bias);
  else
    hipLaunchKernelGGL((radial_weight_kernel<Plan, KH>),
                       dim3((unsigned)slices, (unsigned)(a.C / 16)), dim3(kThreads), 0, s, a,
                       gout, edges_per_slice, part_alpha, part_bias);
  return hipGetLastError();
}

template <class Plan, int KH>
hipError_t launch_shared_forward(const Args& a, float* out, hipStream_t s) {
  hipLaunchKernelGGL((radial_forward_streamed_kernel<Plan, KH, kSharedW>), stream_grid(a),
                     dim3(64 * kSFwdWaves), 0, s, a, out);
  return hipGetLastError();
}

template <class Plan, int KH>
hipError_t launch_shared_backward(const Args& a, const float* gout, float* gx, float* gy,
                                  int needed, hipStream_t s) {
  hipLaunchKernelGGL((radial_backward_streamed_kernel<Plan, KH, kSharedW>), stream_grid(a),
                     dim3(64 * kSBwdWaves), 0, s, a, gout, gx, gy, nullptr, needed & 3);
  return hipGetLastError();
}

// Per-row weights: waves in pairs over 32-channel tiles, 16 edges per group
// of row_pairs(C) pairs (16 edges per block at C >= 128, 64 below C = 64).
inline int row_stream_edges(int C) { return kStreamEdges / 2 / row_pairs(C); }

inline dim3 row_grid(const Args& a) {
  const int per_block = row_stream_edges(a.C);
  return dim3((unsigned)((a.n + per_block - 1) / per_block),
              (unsigned)((a.C + a.tile_span - 1) / a.tile_span));
}

template <class Plan, int KH>
hipError_t launch_row_forward(const Args& a, float* out, hipStream_t s) {
  hipLaunchKernelGGL((radial_forward_streamed_kernel<Plan, KH, kRowW>), row_grid(a),
                     dim3(64 * kSFwdWaves), 0, s, a, out);
  return hipGetLastError();
}

// gw: per-row weight adjoint [n][P*C] (bit 4 of needed).
template <class Plan, int KH>
hipError_t launch_row_backward(const Args& a, const float* gout, float* gx, float* gy, float* gw,
                               int needed, hipStream_t s) {
  hipLaunchKernelGGL((radial_backward_streamed_kernel<Plan, KH, kRowW>), row_grid(a),
                     dim3(64 * kSBwdWaves), 0, s, a, gout, gx, gy, gw, needed & 7);
  return hipGetLastError();
}

template <class Plan, int KH>
hipError_t launch_shared_dw(const Args& a, const float* gout, int64_t edges_per_slice,
                            int slices, float* part, hipStream_t s) {
  hipLaunchKernelGGL((uvu_shared_dw_kernel<Plan, KH>),
                     dim3((unsigned)slices, (unsigned)(a.C / 16)), dim3(kThreads), 0, s, a, gout,
                     edges_per_slice, part);
  return hipGetLastError();
}

template <class Plan>
hipError_t launch_vshared_forward(const Args& a, float* out, hipStream_t s) {
  hipLaunchKernelGGL((uvu_vshared_forward_kernel<Plan>), stream_grid(a), dim3(64 * kSFwdWaves), 0,
                     s, a, out);
  return hipGetLastError();
}

template <class Plan>
hipError_t launch_vshared_backward(const Args& a, const float* gout, float* gx, float* gy,
                                   int needed, hipStream_t s) {
  hipLaunchKernelGGL((uvu_vshared_backward_kernel<Plan>), stream_grid(a), dim3(64 * kSBwdWaves),
                     0, s, a, gout, gx, gy, needed & 3);
  return hipGetLastError();
}

template <class Plan>
hipError_t launch_vshared_dw(const Args& a, const float* gout, int64_t edges_per_slice,
                             int slices, float* part, hipStream_t s) {
  hipLaunchKernelGGL((uvu_vshared_dw_kernel<Plan>),
                     dim3((unsigned)slices, (unsigned)(a.C / 16), (unsigned)vdw_groups<Plan>()),
                     dim3(kThreads), 0, s, a, gout, edges_per_slice, part);
  return hipGetLastError();
}

template <class Plan>
const VSharedLaunchers* vshared_launchers() {
  static const VSharedLaunchers l = {vdw_edges<Plan>(), vdw_groups<Plan>(),
                                     &launch_vshared_forward<Plan>,
                                     &launch_vshared_backward<Plan>, &launch_vshared_dw<Plan>};
  return &l;
}

template <class Plan>
constexpr int weight_groups() {
  if constexpr (Plan::kWgtStreamed && !Plan::kWgtTwoPhase) return wgt_groups<Plan>();
  else return 1;
}

// The shared-weight uvu launchers of a plan live in a translation unit of
// their own (O2MI_DEFINE_UVU_SHARED): both halves of a large structure then
// compile in parallel.
struct SharedLaunchers {
  hipError_t (*forward)(const Args&, float* out, hipStream_t);
  hipError_t (*backward)(const Args&, const float* gout, float* gx, float* gy, int needed,
                         hipStream_t);
  hipError_t (*dw)(const Args&, const float* gout, int64_t edges_per_slice, int slices,
                   float* part, hipStream_t);
  // The same product with per-row weights [n][P*C] (Args::alpha).
  hipError_t (*row_forward)(const Args&, float* out, hipStream_t);
  hipError_t (*row_backward)(const Args&, const float* gout, float* gx, float* gy, float* gw,
                             int needed, hipStream_t);
};

template <class Plan, int KH>
const SharedLaunchers* shared_launchers() {
  static const SharedLaunchers l = {&launch_shared_forward<Plan, KH>,
                                    &launch_shared_backward<Plan, KH>,
                                    &launch_shared_dw<Plan, KH>, &launch_row_forward<Plan, KH>,
                                    &launch_row_backward<Plan, KH>};
  return &l;
}

template <class Plan, int KH>
const KernelSet* kernel_set(const SharedLaunchers* shared, const VSharedLaunchers* vshared) {
  static const KernelSet set = {Plan::kPaths, Plan::kComps1, Plan::kComps2, KH,
                                Plan::kWeightEdges, weight_groups<Plan>(), kStreamEdges,
                                &launch_forward<Plan, KH>, &launch_backward<Plan, KH>,
                                &launch_weight<Plan, KH>, dw_edges<Plan, KH>(),
                                shared->forward, shared->backward, shared->dw, vshared,
                                shared->row_forward, shared->row_backward};
  return &set;
}

}  // namespace radial
}  // namespace o2mi

#define O2MI_DEFINE_RADIAL_SET(NAME, KH)                                                \
  const o2mi::radial::SharedLaunchers* o2mi_uvu_shared_##NAME##_##KH();                  \
  const o2mi::radial::VSharedLaunchers* o2mi_uvu_vshared_##NAME##_##KH();                \
  const o2mi::radial::KernelSet* o2mi_radial_set_##NAME##_##KH() {                      \
    return o2mi::radial::kernel_set<o2mi::radial::plans::NAME, KH>(                     \
        o2mi_uvu_shared_##NAME##_##KH(), o2mi_uvu_vshared_##NAME##_##KH());             \
  }

#define O2MI_DEFINE_UVU_SHARED(NAME, KH)                                                \
  const o2mi::radial::SharedLaunchers* o2mi_uvu_shared_##NAME##_##KH() {                \
    return o2mi::radial::shared_launchers<o2mi::radial::plans::NAME, KH>();              \
  }

#define O2MI_DEFINE_UVU_VSHARED(NAME, KH)                                               \
  const o2mi::radial::VSharedLaunchers* o2mi_uvu_vshared_##NAME##_##KH() {              \
    return o2mi::radial::vshared_launchers<o2mi::radial::plans::NAME>();                 \
  }
