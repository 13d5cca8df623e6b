// Host interface of the table-driven TP kernels (o2mi_tp_generic.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace o2mi {
namespace generic {

struct Geom {
  int64_t n_rows;
  int64_t weight_numel;  // P_w
  int channels;          // C
  int width;             // W
  int lanes;             // 2C (full) or C (canonical)
  int full;              // 1 for full parity
  int layout;            // 0 channel-major, 1 / 2 component-major
  int n_keys;            // 0e, [0o], 1..M
  int n_paths;           // rows of the path table
};

struct WeightShape {
  int threads, tiles, chunks;
  int64_t groups;  // row groups = partial rows of dw
};

// Largest key count the kernels' LDS holds (m_max <= max_keys() - 2 in full
// parity, - 1 in canonical).
int max_keys();

hipError_t forward(const float* x, const float* y, const float* w, float* out,
                   const int32_t* info, const float* coef, const Geom& g, int cus,
                   hipStream_t stream);
hipError_t input_adjoint(const float* x, const float* y, const float* w, const float* gout,
                         float* dx, float* dy, const int32_t* info, const float* coef,
                         const Geom& g, int needed, int cus, hipStream_t stream);
WeightShape weight_shape(const Geom& g, int cus);
// Writes groups x P_w partial sums of dw into `partial`.
hipError_t weight_adjoint(const float* x, const float* y, const float* gout, float* partial,
                          const int32_t* info, const float* coef, const Geom& g,
                          const WeightShape& ws, hipStream_t stream);

}  // namespace generic
}  // namespace o2mi
