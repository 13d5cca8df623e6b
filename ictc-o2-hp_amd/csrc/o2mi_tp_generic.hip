// Table-driven O(2) tensor-product kernels: any m_max, run when no plan is
// compiled for the representation (the compiled plans cover m_max <= 8).
//
// The path table is the op's own device metadata (triton_o2.py:786-794,
// built as in runtime_weight.py:14-29): path_info int32 [P, 25] =
// (start, mul, dim, is_freq) of the first, second and output key, the first
// packed weight, then (i, j, k) of up to four terms; path_coefficients f32
// [P, 4] = the terms' signed coefficients (0 for an absent term).  The path
// loop is uniform across a block, so the table is read with scalar loads.
//
// Work mapping.  One thread = one (row, lane); a lane is one output channel
// o of the widest multiplicity (2C in full parity, ordered 2c + q like the
// compiled kernels so that the two copies of channel c are neighbouring
// lanes, C in canonical parity).  Key k of the lane reads channel o mod
// mul_k (the cyclic routing of native_o2.py:128-129).  A thread's x, y (and
// cotangent / adjoint) values of every key live in LDS slots private to the
// thread (slot s of thread t at s * blockDim + t, so a wave touches 64
// consecutive banks): path terms index them by the table's runtime indices.
// Copy-1 values are turned into the canonical basis on load and back on store
// (fast_o2.py:61-73).
//
// The weight adjoint is a separate kernel over (row group, lane tile, chunk of
// kChunk paths): each thread keeps the chunk's accumulators in registers over
// the group's rows and writes one partial row; a fixed-order column sum
// finishes dw (deterministic, no atomics).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "o2mi_tp_generic.hpp"

namespace o2mi {
namespace generic {

namespace {

constexpr int kInfo = 25;   // ints per path record
constexpr int kChunk = 32;  // paths per weight-adjoint block

struct KeyGeom {
  int start, mul, dim;
  bool freq;
};

// Key k of the plan (keys 0e, [0o], 1..M): closed form of the row layout.
__device__ __forceinline__ KeyGeom key_geom(const Geom& g, int k) {
  const int scalars = g.full ? 2 : 1;
  KeyGeom kg;
  if (k < scalars) {
    kg.start = k * g.channels;
    kg.mul = g.channels;
    kg.dim = 1;
    kg.freq = false;
  } else {
    const int block = (g.full ? 4 : 2) * g.channels;
    kg.start = scalars * g.channels + (k - scalars) * block;
    kg.mul = (g.full ? 2 : 1) * g.channels;
    kg.dim = 2;
    kg.freq = true;
  }
  return kg;
}

// Key index of a key record's start offset (the inverse of key_geom), clamped
// into [0, n_keys) so that a malformed table cannot address outside LDS.
__device__ __forceinline__ int key_of_start(const Geom& g, int start) {
  const int scalars = g.full ? 2 : 1;
  int k;
  if (start < scalars * g.channels) {
    k = start / g.channels;
  } else {
    k = scalars + (start - scalars * g.channels) / ((g.full ? 4 : 2) * g.channels);
  }
  return k < 0 ? 0 : (k >= g.n_keys ? g.n_keys - 1 : k);
}

// Position of (key, channel o, component) in a row (triton_o2.py:110-121).
__device__ __forceinline__ int64_t element(const Geom& g, const KeyGeom& kg, int o, int comp) {
  if (kg.dim == 1) return kg.start + o;
  if (g.layout == 0) return kg.start + 2 * o + comp;
  if (g.layout == 1) return kg.start + comp * kg.mul + o;
  return kg.start + (o / g.channels) * 2 * g.channels + comp * g.channels + o % g.channels;
}

__device__ __forceinline__ int lane_channel(const Geom& g, int lane) {
  return g.full ? (lane & 1) * g.channels + (lane >> 1) : lane;
}

// Slot of (array a, key k, component c) of the calling thread.
struct Slots {
  float* base;
  int stride;  // blockDim.x
  int keys;
  __device__ __forceinline__ float& at(int a, int k, int c) const {
    return base[((a * keys + k) * 2 + c) * stride];
  }
};

// Loads every key of `row` for channel o into array a, canonical basis.
// Keys whose multiplicity is <= o are not this lane's outputs: with
// `own_only` they read 0 (the cotangent of a scalar output for the copy-1
// lane), otherwise the routed channel o mod mul.
__device__ __forceinline__ void load_keys(const Geom& g, const float* __restrict__ src,
                                          int64_t row, int o, const Slots& s, int a,
                                          bool own_only) {
  const float* r = src + row * g.width;
  for (int k = 0; k < g.n_keys; ++k) {
    const KeyGeom kg = key_geom(g, k);
    const bool own = o < kg.mul;
    const int ok = o % kg.mul;
    float v0 = 0.f, v1 = 0.f;
    if (own || !own_only) {
      v0 = r[element(g, kg, ok, 0)];
      if (kg.dim == 2) v1 = r[element(g, kg, ok, 1)];
    }
    if (g.full && kg.freq && ok >= g.channels) {  // copy 1: (v0, v1) -> (-v1, v0)
      const float t = v0;
      v0 = -v1;
      v1 = t;
    }
    s.at(a, k, 0) = v0;
    s.at(a, k, 1) = v1;
  }
}

// Stores array a's keys that channel o owns (o < mul), restoring copy 1.
__device__ __forceinline__ void store_keys(const Geom& g, float* __restrict__ dst, int64_t row,
                                           int o, const Slots& s, int a) {
  float* r = dst + row * g.width;
  for (int k = 0; k < g.n_keys; ++k) {
    const KeyGeom kg = key_geom(g, k);
    if (o >= kg.mul) continue;
    float v0 = s.at(a, k, 0), v1 = s.at(a, k, 1);
    if (g.full && kg.freq && o >= g.channels) {  // back to copy 1: (v0, v1) -> (v1, -v0)
      const float t = v0;
      v0 = v1;
      v1 = -t;
    }
    r[element(g, kg, o, 0)] = v0;
    if (kg.dim == 2) r[element(g, kg, o, 1)] = v1;
  }
}

struct PathRecord {
  int k1, k2, k3, mul3, ws;  // mul3: output channels of the path (0 if malformed)
  int i[4], j[4], k[4];
  float c[4];
};

__device__ __forceinline__ PathRecord read_path(const Geom& g, const int32_t* __restrict__ info,
                                                const float* __restrict__ coef, int p) {
  const int32_t* row = info + (int64_t)p * kInfo;
  PathRecord r;
  r.k1 = key_of_start(g, row[0]);
  r.k2 = key_of_start(g, row[4]);
  r.k3 = key_of_start(g, row[8]);
  r.mul3 = row[9];
  r.ws = row[12];
  // A path whose weights would lie outside the packed weight is skipped.
  if (r.ws < 0 || r.mul3 < 0 || (int64_t)r.ws + r.mul3 > g.weight_numel) r.mul3 = 0;
  for (int t = 0; t < 4; ++t) {
    // Components are 0 or 1; mask malformed values into range.
    r.i[t] = row[13 + 3 * t] & 1;
    r.j[t] = row[14 + 3 * t] & 1;
    r.k[t] = row[15 + 3 * t] & 1;
    r.c[t] = coef[(int64_t)p * 4 + t];
  }
  return r;
}

// LDS arrays: forward X, Y, A (3); input adjoint X, Y, G, DX, DY (5); weight
// adjoint X, Y, G (3).
enum { kX = 0, kY = 1, kG = 2, kA = 2, kDX = 3, kDY = 4 };

__global__ __launch_bounds__(256) void forward_kernel(const float* __restrict__ x,
                                                      const float* __restrict__ y,
                                                      const float* __restrict__ w,
                                                      float* __restrict__ out,
                                                      const int32_t* __restrict__ info,
                                                      const float* __restrict__ coef,
                                                      Geom g) {
  extern __shared__ float lds[];
  const Slots s{lds + threadIdx.x, (int)blockDim.x, g.n_keys};
  const int64_t items = g.n_rows * g.lanes;
  for (int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; item < items;
       item += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = item / g.lanes;
    const int o = lane_channel(g, (int)(item - row * g.lanes));
    load_keys(g, x, row, o, s, kX, false);
    load_keys(g, y, row, o, s, kY, false);
    for (int k = 0; k < g.n_keys; ++k) s.at(kA, k, 0) = s.at(kA, k, 1) = 0.f;
    for (int p = 0; p < g.n_paths; ++p) {
      const PathRecord pr = read_path(g, info, coef, p);
      if (o >= pr.mul3) continue;
      float f[2] = {0.f, 0.f};
      for (int t = 0; t < 4; ++t) {
        if (pr.c[t] == 0.f) continue;  // absent term
        f[pr.k[t]] = fmaf(pr.c[t] * s.at(kX, pr.k1, pr.i[t]), s.at(kY, pr.k2, pr.j[t]),
                          f[pr.k[t]]);
      }
      const float wv = w[pr.ws + o];
      s.at(kA, pr.k3, 0) = fmaf(wv, f[0], s.at(kA, pr.k3, 0));
      s.at(kA, pr.k3, 1) = fmaf(wv, f[1], s.at(kA, pr.k3, 1));
    }
    store_keys(g, out, row, o, s, kA);
  }
}

// dx and dy (triton_o2.py:452-501).  The two lanes of channel c (copies 0 and
// 1) both feed the scalar inputs' channel c: their sums are combined with one
// lane swap; the copy-0 lane stores them.
__global__ __launch_bounds__(256) void input_adjoint_kernel(
    const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ w,
    const float* __restrict__ gout, float* __restrict__ dx, float* __restrict__ dy,
    const int32_t* __restrict__ info, const float* __restrict__ coef, Geom g, int needed) {
  extern __shared__ float lds[];
  const Slots s{lds + threadIdx.x, (int)blockDim.x, g.n_keys};
  const int64_t items = g.n_rows * g.lanes;
  // Every lane pair runs the same iterations (lanes is even in full parity),
  // so the partner of a swap is always active.
  for (int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; item < items;
       item += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = item / g.lanes;
    const int o = lane_channel(g, (int)(item - row * g.lanes));
    load_keys(g, x, row, o, s, kX, false);
    load_keys(g, y, row, o, s, kY, false);
    load_keys(g, gout, row, o, s, kG, true);
    for (int k = 0; k < g.n_keys; ++k)
      s.at(kDX, k, 0) = s.at(kDX, k, 1) = s.at(kDY, k, 0) = s.at(kDY, k, 1) = 0.f;
    for (int p = 0; p < g.n_paths; ++p) {
      const PathRecord pr = read_path(g, info, coef, p);
      if (o >= pr.mul3) continue;
      const float wv = w[pr.ws + o];
      const float h[2] = {wv * s.at(kG, pr.k3, 0), wv * s.at(kG, pr.k3, 1)};
      for (int t = 0; t < 4; ++t) {
        if (pr.c[t] == 0.f) continue;  // absent term
        const float hk = pr.c[t] * h[pr.k[t]];
        s.at(kDX, pr.k1, pr.i[t]) = fmaf(hk, s.at(kY, pr.k2, pr.j[t]), s.at(kDX, pr.k1, pr.i[t]));
        s.at(kDY, pr.k2, pr.j[t]) = fmaf(hk, s.at(kX, pr.k1, pr.i[t]), s.at(kDY, pr.k2, pr.j[t]));
      }
    }
    if (g.full) {
      for (int k = 0; k < (g.full ? 2 : 1); ++k) {
        s.at(kDX, k, 0) += __shfl_xor(s.at(kDX, k, 0), 1);
        s.at(kDY, k, 0) += __shfl_xor(s.at(kDY, k, 0), 1);
      }
    }
    if (needed & 1) store_keys(g, dx, row, o, s, kDX);
    if (needed & 2) store_keys(g, dy, row, o, s, kDY);
  }
}

// Weight adjoint partials (triton_o2.py:571-607): block (group, tile, chunk)
// sums coef * x * y * g over rows group, group + groups, ... for its lanes and
// the chunk's paths, and writes partial[group][ws + o].
__global__ __launch_bounds__(256) void weight_adjoint_kernel(
    const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ gout,
    float* __restrict__ partial, const int32_t* __restrict__ info,
    const float* __restrict__ coef, Geom g, int64_t groups) {
  extern __shared__ float lds[];
  const Slots s{lds + threadIdx.x, (int)blockDim.x, g.n_keys};
  const int64_t group = blockIdx.x;
  const int lane = blockIdx.y * blockDim.x + threadIdx.x;
  const int p0 = blockIdx.z * kChunk;
  if (lane >= g.lanes) return;
  const int o = lane_channel(g, lane);
  float acc[kChunk];
#pragma unroll
  for (int q = 0; q < kChunk; ++q) acc[q] = 0.f;
  for (int64_t row = group; row < g.n_rows; row += groups) {
    load_keys(g, x, row, o, s, kX, false);
    load_keys(g, y, row, o, s, kY, false);
    load_keys(g, gout, row, o, s, kG, true);
#pragma unroll
    for (int q = 0; q < kChunk; ++q) {
      const int p = p0 + q;
      if (p >= g.n_paths) break;
      const PathRecord pr = read_path(g, info, coef, p);
      float v = 0.f;
      for (int t = 0; t < 4; ++t) {
        if (pr.c[t] == 0.f) continue;  // absent term
        v = fmaf(pr.c[t] * s.at(kX, pr.k1, pr.i[t]),
                 s.at(kY, pr.k2, pr.j[t]) * s.at(kG, pr.k3, pr.k[t]), v);
      }
      acc[q] += v;
    }
  }
  float* prow = partial + group * g.weight_numel;
#pragma unroll
  for (int q = 0; q < kChunk; ++q) {
    const int p = p0 + q;
    if (p >= g.n_paths) break;
    const PathRecord pr = read_path(g, info, coef, p);
    if (o < pr.mul3) prow[pr.ws + o] = acc[q];
  }
}

hipError_t allow_lds(const void* kernel, size_t bytes) {
  if (bytes <= 64 * 1024) return hipSuccess;
  return hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

int threads_for(int n_keys, int arrays) {
  // LDS bytes per thread: arrays x keys x 2 floats; keep a block under 40 KiB
  // so that several blocks share a CU.
  const int per_thread = arrays * n_keys * 2 * 4;
  int t = 256;
  while (t > 64 && t * per_thread > 40 * 1024) t /= 2;
  return t;
}

}  // namespace

// 64 threads x 5 arrays x keys x 2 floats must fit one block's LDS.
int max_keys() { return 48; }

size_t lds_bytes(int n_keys, int arrays, int threads) {
  return (size_t)arrays * n_keys * 2 * sizeof(float) * threads;
}

hipError_t forward(const float* x, const float* y, const float* w, float* out,
                   const int32_t* info, const float* coef, const Geom& g, int cus,
                   hipStream_t stream) {
  const int t = threads_for(g.n_keys, 3);
  const size_t lds = lds_bytes(g.n_keys, 3, t);
  const hipError_t err = allow_lds(reinterpret_cast<const void*>(&forward_kernel), lds);
  if (err != hipSuccess) return err;
  const int64_t items = g.n_rows * g.lanes;
  const int64_t want = (items + t - 1) / t;
  const int grid = (int)(want < 8LL * cus ? want : 8LL * cus);
  hipLaunchKernelGGL(forward_kernel, dim3(grid), dim3(t), lds, stream, x, y, w, out, info, coef,
                     g);
  return hipGetLastError();
}

hipError_t input_adjoint(const float* x, const float* y, const float* w, const float* gout,
                         float* dx, float* dy, const int32_t* info, const float* coef,
                         const Geom& g, int needed, int cus, hipStream_t stream) {
  const int t = threads_for(g.n_keys, 5);
  const size_t lds = lds_bytes(g.n_keys, 5, t);
  const hipError_t err = allow_lds(reinterpret_cast<const void*>(&input_adjoint_kernel), lds);
  if (err != hipSuccess) return err;
  const int64_t items = g.n_rows * g.lanes;
  const int64_t want = (items + t - 1) / t;
  const int grid = (int)(want < 8LL * cus ? want : 8LL * cus);
  hipLaunchKernelGGL(input_adjoint_kernel, dim3(grid), dim3(t), lds, stream, x, y, w, gout, dx,
                     dy, info, coef, g, needed);
  return hipGetLastError();
}

WeightShape weight_shape(const Geom& g, int cus) {
  WeightShape ws;
  ws.threads = threads_for(g.n_keys, 3);
  ws.tiles = (g.lanes + ws.threads - 1) / ws.threads;
  ws.chunks = (g.n_paths + kChunk - 1) / kChunk;
  const int64_t per_group = (int64_t)ws.tiles * ws.chunks;
  int64_t groups = (4LL * cus + per_group - 1) / per_group;
  if (groups > g.n_rows) groups = g.n_rows;
  if (groups < 1) groups = 1;
  ws.groups = groups;
  return ws;
}

hipError_t weight_adjoint(const float* x, const float* y, const float* gout, float* partial,
                          const int32_t* info, const float* coef, const Geom& g,
                          const WeightShape& ws, hipStream_t stream) {
  const size_t lds = lds_bytes(g.n_keys, 3, ws.threads);
  const hipError_t err = allow_lds(reinterpret_cast<const void*>(&weight_adjoint_kernel), lds);
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(weight_adjoint_kernel, dim3((unsigned)ws.groups, ws.tiles, ws.chunks),
                     dim3(ws.threads), lds, stream, x, y, gout, partial, info, coef, g,
                     ws.groups);
  return hipGetLastError();
}

}  // namespace generic
}  // namespace o2mi
