// O(2) tensor-product kernels for gfx950 (CDNA4): forward and fused VJP.
//
// One plan P (generated per m_max / parity / normalization) supplies the
// key table, the path table and each path's sparse coupling terms as
// constexpr data; every loop over keys, paths and terms below is unrolled at
// compile time, so coefficients become sign modifiers or folded constants
// and the per-lane state lives in registers.
//
// Work mapping.  A flat row holds, per key, C scalars (0e, 0o) or 2C x 2
// floats (frequency blocks of full parity: [copy, channel, component]).  A
// "lane" is one (channel c, copy q) of a row: 2C lanes per row for full
// parity, C for canonical.  Neighbouring hardware lanes 2c, 2c+1 hold the two
// copies of channel c, so
//   * frequency outputs of copy q read copy q of frequency inputs and the
//     channel-c scalars (routing o mod mul of native_o2.py:128-129),
//   * scalar outputs read copy 0 only: they are produced by the q = 0 lane,
//   * the scalar input adjoints, which collect both copies, finish with one
//     DPP swap between the two lanes of a pair.
// Copy-1 values are turned into the canonical basis on load, (v0, v1) ->
// (-v1, v0), and back on store (fast_o2.py:61-73, triton_o2.py:133-164).
//
// Memory access.  Rows are read and written with buffer instructions: a
// per-iteration descriptor (SGPRs) whose base is the iteration's first row and
// whose size covers exactly the valid rows, a loop-invariant per-lane byte
// offset (VGPR) and a per-key uniform offset (SGPR).  Rows past the end and
// idle lanes fall outside the descriptor, so their loads return 0 and their
// stores are dropped by the hardware: no branches, no masks.
//
// Both kernels are persistent: block b owns a fixed set of row chunks (b,
// b + G, b + 2G, ... of G blocks; the backward walks them from the last chunk
// down) and a fixed set of lanes, so the backward keeps one weight-adjoint
// accumulator per path and lane in registers across all its rows and writes
// one partial row at the end; a fixed-order column sum finishes dw.  There
// are no atomics and the result is bitwise reproducible.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

namespace o2mi {

struct KeySpec {
  int off;  // offset in the row, in units of C
  int dim;  // 1 for scalars, 2 for frequency keys
};

struct PathSpec {
  int k1, k2, k3;  // key indices
  int wunits;      // first packed weight, in units of C
  int t0, nt;      // terms[t0 .. t0 + nt)
  float mag;       // common |coefficient| of the terms
};

struct TermSpec {
  int i, j, k;  // first, second and output component
  int sign;     // +1 or -1
};

// Cache policies of row loads and stores (bits: 1 sc0, 2 nt, 16 sc1).  Every
// row is touched once per kernel, so loads are non-temporal; the forward's
// stores are non-temporal + sc1, the backward's non-temporal (measured best
// at the headline shape: forward 0.938 -> 0.890 ms, backward 1.722 -> 1.659
// ms together with the reverse row order of the backward).  Default
// (allocating) loads measured slower in either kernel (forward +3.6%,
// backward +2.5%).
constexpr int kForwardLoadPolicy = 2;
constexpr int kBackwardLoadPolicy = 2;
constexpr int kForwardStorePolicy = 18;
constexpr int kBackwardStorePolicy = 2;

// Threads per block and the lanes of one row a block covers (a row of more
// lanes is split over several blocks, "tiles").  The forward keeps each
// lane's path weights in registers for the whole persistent kernel and runs
// at up to 3 waves per SIMD (plans with many paths stage them in LDS
// instead: forward_lds below); the backward holds one weight-adjoint
// accumulator per path and lane in registers and needs 2 waves per SIMD to
// hide its dependent FMA chains and LDS weight reads.  These are the defaults;
// forward_block, forward_tile and backward_tile below pick per plan.
constexpr int kBlock = 256;
constexpr int kBackwardBlock = 256;  // 512 (two rows per iteration, one block per CU): same time
constexpr int kForwardTile = 256;
constexpr int kForwardWaves = 1;   // minimum waves per SIMD requested
constexpr int kBackwardWaves = 2;
static_assert(kForwardTile % 2 == 0 && kForwardTile <= kBlock, "tile must be even, <= block");
// Byte offset given to lanes with nothing to load or store: beyond any
// descriptor size used here (< 2^31), with room to add key offsets.
constexpr uint32_t kIdle = 0x80000000u;
// Word 3 of a raw gfx9 buffer descriptor (32-bit data format).
constexpr int kRsrcFlags = 0x00020000;

template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  [&]<int... I>(std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
  }(std::make_integer_sequence<int, N>{});
}

// Launch geometry, computed on the host (o2mi_capi.hip).
struct TPGeom {
  int64_t n_rows;
  int64_t groups;          // blocks along the rows (grid = groups * tiles)
  int channels;            // C
  int width;               // W, floats per row
  int lanes;               // lanes per row: 2C (full) or C (canonical)
  int tile_lanes;          // lanes of one row handled by a block: min(lanes, tile)
  int rows_per_iter;       // rows a block advances per iteration
  int tiles;               // blocks sharing one row range: ceil(lanes / tile)
  int weight_numel;        // P_w
};

struct Lane {
  int c;     // channel (clamped to 0 on idle lanes)
  int q;     // copy (always 0 for canonical parity)
  int jloc;  // lane index inside the block's tile (2 cloc + q for full parity)
  int cloc;  // channel index inside the block's tile
  int slot;  // row slot inside one iteration
  bool active;
};

template <bool kFull, int kTile>
__device__ __forceinline__ Lane make_lane(const TPGeom& g, int tile) {
  Lane l;
  const int t = threadIdx.x;
  l.slot = t / g.tile_lanes;
  const int jloc = t - l.slot * g.tile_lanes;
  const int j = tile * kTile + jloc;
  l.active = l.slot < g.rows_per_iter && j < g.lanes;
  l.jloc = jloc;
  const int jj = l.active ? j : 0;
  l.c = kFull ? (jj >> 1) : jj;
  l.q = kFull ? (jj & 1) : 0;
  l.cloc = kFull ? (jloc >> 1) : jloc;
  return l;
}

// Per-lane byte offsets inside one iteration's rows.
struct LaneOffsets {
  uint32_t scalar;       // scalar keys
  uint32_t freq;         // frequency keys, component 0
  uint32_t scalar_own;   // scalar keys of the copy-0 lane only (idle on copy 1)
};

template <bool kFull, int kLayout>
__device__ __forceinline__ LaneOffsets lane_offsets(const TPGeom& g, const Lane& l) {
  LaneOffsets o;
  const int row = l.slot * g.width;
  const int f = (kFull ? l.q * 2 * g.channels : 0) + (kLayout == 0 ? 2 * l.c : l.c);
  o.scalar = l.active ? (uint32_t)(row + l.c) * 4u : kIdle;
  o.freq = l.active ? (uint32_t)(row + f) * 4u : kIdle;
  o.scalar_own = (l.active && l.q == 0) ? o.scalar : kIdle;
  return o;
}

// Descriptor over rows [row0, row0 + rows) of a [*, width] f32 tensor.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const float* base, int64_t row0,
                                                            int width, int rows) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base) + row0 * width, 0,
                                           rows * width * 4, kRsrcFlags);
}

template <int kCpol>
__device__ __forceinline__ float bload(__amdgpu_buffer_rsrc_t r, uint32_t voff, int soff) {
  return __builtin_bit_cast(float,
                            __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, soff, kCpol));
}

using f32x2 = float __attribute__((ext_vector_type(2)));
using u32x2 = uint32_t __attribute__((ext_vector_type(2)));

// Whole-vector bit casts only: hipcc 7.2 miscompiles __builtin_bit_cast of a
// single vector element (both elements read as element 0).
template <int kCpol>
__device__ __forceinline__ void bload2(__amdgpu_buffer_rsrc_t r, uint32_t voff, int soff,
                                       float& a, float& b) {
  const f32x2 v = __builtin_bit_cast(
      f32x2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, soff, kCpol));
  a = v.x;
  b = v.y;
}

template <int kCpol>
__device__ __forceinline__ void bstore(__amdgpu_buffer_rsrc_t r, float v, uint32_t voff,
                                       int soff) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, (int)voff, soff,
                                        kCpol);
}

template <int kCpol>
__device__ __forceinline__ void bstore2(__amdgpu_buffer_rsrc_t r, float a, float b,
                                        uint32_t voff, int soff) {
  f32x2 v;
  v.x = a;
  v.y = b;
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), r, (int)voff, soff,
                                        kCpol);
}

// Exchange a value between the two lanes of a copy pair (quad_perm 1,0,3,2).
__device__ __forceinline__ float pair_swap(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
}

template <class P, int kLayout, bool kVec2, int K, int kCpol>
__device__ __forceinline__ void load_key(__amdgpu_buffer_rsrc_t r, int C, const Lane& l,
                                         uint32_t voff, float& v0, float& v1) {
  constexpr KeySpec ks = P::keys[K];
  const int soff = ks.off * C * 4;
  if constexpr (ks.dim == 1) {
    v0 = bload<kCpol>(r, voff, soff);
    v1 = 0.f;
  } else {
    float a0, a1;
    if constexpr (kLayout == 0 && kVec2) {
      bload2<kCpol>(r, voff, soff, a0, a1);
    } else if constexpr (kLayout == 0) {
      a0 = bload<kCpol>(r, voff, soff);
      a1 = bload<kCpol>(r, voff + 4u, soff);
    } else {
      a0 = bload<kCpol>(r, voff, soff);
      a1 = bload<kCpol>(r, voff, soff + C * 4);
    }
    if constexpr (P::kFull) {
      const bool odd = l.q != 0;
      v0 = odd ? -a1 : a0;
      v1 = odd ? a0 : a1;
    } else {
      v0 = a0;
      v1 = a1;
    }
  }
}

template <class P, int kLayout, bool kVec2, int K, int kCpol>
__device__ __forceinline__ void store_key(__amdgpu_buffer_rsrc_t r, int C, const Lane& l,
                                          uint32_t voff, float v0, float v1) {
  constexpr KeySpec ks = P::keys[K];
  const int soff = ks.off * C * 4;
  if constexpr (ks.dim == 1) {
    bstore<kCpol>(r, v0, voff, soff);
  } else {
    float s0 = v0, s1 = v1;
    if constexpr (P::kFull) {
      const bool odd = l.q != 0;
      s0 = odd ? v1 : v0;
      s1 = odd ? -v0 : v1;
    }
    if constexpr (kLayout == 0 && kVec2) {
      bstore2<kCpol>(r, s0, s1, voff, soff);
    } else if constexpr (kLayout == 0) {
      bstore<kCpol>(r, s0, voff, soff);
      bstore<kCpol>(r, s1, voff + 4u, soff);
    } else {
      bstore<kCpol>(r, s0, voff, soff);
      bstore<kCpol>(r, s1, voff, soff + C * 4);
    }
  }
}

// Loads every key of one row set: x and y, and optionally the cotangent.
template <class P, int kLayout, bool kVec2, int kCpol>
__device__ __forceinline__ void load_row(__amdgpu_buffer_rsrc_t r, int C, const Lane& l,
                                         const LaneOffsets& o, bool copy0_scalars,
                                         float (&V)[P::kKeys][2]) {
  static_for<P::kKeys>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    const uint32_t voff =
        P::keys[k].dim == 1 ? (copy0_scalars ? o.scalar_own : o.scalar) : o.freq;
    load_key<P, kLayout, kVec2, k, kCpol>(r, C, l, voff, V[k][0], V[k][1]);
  });
}

template <class P, int kLayout, bool kVec2, int kCpol>
__device__ __forceinline__ void store_row(__amdgpu_buffer_rsrc_t r, int C, const Lane& l,
                                          const LaneOffsets& o, const float (&V)[P::kKeys][2]) {
  static_for<P::kKeys>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    // Scalar keys are written by the copy-0 lane only.
    const uint32_t voff = P::keys[k].dim == 1 ? o.scalar_own : o.freq;
    store_key<P, kLayout, kVec2, k, kCpol>(r, C, l, voff, V[k][0], V[k][1]);
  });
}

template <class P, int kPath>
__device__ __forceinline__ void path_value(const float (&X)[P::kKeys][2],
                                           const float (&Y)[P::kKeys][2], float& f0, float& f1) {
  constexpr PathSpec ps = P::paths[kPath];
  f0 = 0.f;
  f1 = 0.f;
  static_for<ps.nt>([&](auto tc) {
    constexpr TermSpec ts = P::terms[ps.t0 + decltype(tc)::value];
    const float a = ts.sign > 0 ? X[ps.k1][ts.i] : -X[ps.k1][ts.i];
    if constexpr (ts.k == 0) {
      f0 = fmaf(a, Y[ps.k2][ts.j], f0);
    } else {
      f1 = fmaf(a, Y[ps.k2][ts.j], f1);
    }
  });
}

template <class P>
constexpr bool out_is_freq(int p) {
  return P::keys[P::paths[p].k3].dim == 2;
}


// ---------------------------------------------------------------------------
// Path weights, times each path's coupling magnitude, staged in LDS for the
// block's tile: path p starts at wunits * U floats (U = kTile / 2 for full
// parity, kTile for canonical).  Frequency-output paths of full parity hold
// both copies interleaved by lane (index 2 c + q), so neighbouring lanes read
// neighbouring banks; scalar-output paths hold one value per channel.
template <class P, int kTile>
constexpr int lds_unit() {
  return P::kFull ? kTile / 2 : kTile;
}

template <class P, int kTile>
constexpr size_t lds_bytes() {
  return sizeof(float) * (size_t)P::kUnits * (size_t)lds_unit<P, kTile>();
}

// Lanes of a row one backward block covers (backward_tile<P>() below): 256,
// or 128 where a 256-lane stage of the path weights would need more than
// 80 KiB of LDS (m7 full and larger plans), so that two blocks still share a
// CU (the backward runs at two waves per SIMD).
template <class P>
constexpr int backward_tile() {
  return lds_bytes<P, 256>() > 80 * 1024 ? 128 : 256;
}
static_assert(128 <= kBackwardBlock && 256 <= kBackwardBlock, "tiles must fit a block");

// The forward keeps a lane's path weights in registers; with more than 100
// paths in full parity (m7, m8) those registers leave 3 waves per SIMD at
// one row per 4-wave iteration, and the kernel runs latency-bound (3.6 TB/s).
// Those plans stage the weights in LDS like the backward instead, with
// 128-lane tiles and 512-thread blocks (4 rows per iteration), so that LDS,
// not registers, sets the occupancy (6 waves per SIMD at m7 full).
template <class P>
constexpr bool forward_lds() {
  return P::kFull && P::kPaths > 100;
}
template <class P>
constexpr int forward_block() {
  return forward_lds<P>() ? 512 : kBlock;
}
template <class P>
constexpr int forward_tile() {
  return forward_lds<P>() ? 128 : kForwardTile;
}

template <class P, int kTile>
__device__ __forceinline__ void stage_weights(float* lds, const float* __restrict__ w, int C,
                                              int tile) {
  constexpr int U = lds_unit<P, kTile>();
  const int c0 = tile * U;
  const int t = threadIdx.x;
  static_for<P::kPaths>([&](auto pc) {
    constexpr int p = decltype(pc)::value;
    constexpr PathSpec ps = P::paths[p];
    if constexpr (P::kFull && out_is_freq<P>(p)) {
      if (t < kTile) {
        const int c = c0 + (t >> 1);
        lds[ps.wunits * U + t] = c < C ? w[(ps.wunits + (t & 1)) * C + c] * ps.mag : 0.f;
      }
    } else {
      if (t < U) {
        const int c = c0 + t;
        lds[ps.wunits * U + t] = c < C ? w[ps.wunits * C + c] * ps.mag : 0.f;
      }
    }
  });
}

// LDS column of this lane for frequency-output and scalar-output paths.
template <class P>
struct WeightColumns {
  int freq, scalar;
};

template <class P>
__device__ __forceinline__ WeightColumns<P> weight_columns(const Lane& l) {
  return {P::kFull ? l.jloc : l.cloc, l.cloc};
}

template <class P, int kTile, int kPath>
__device__ __forceinline__ float staged_weight(const float* lds, const WeightColumns<P>& col) {
  constexpr PathSpec ps = P::paths[kPath];
  constexpr int U = lds_unit<P, kTile>();
  return lds[(out_is_freq<P>(kPath) ? col.freq : col.scalar) + ps.wunits * U];
}

// Rows visited by one block.  Iteration `it` covers rows [row0(it),
// row0(it) + rows(it)); the buffer descriptors cover exactly those rows.
// Strided order keeps all blocks inside one contiguous window of the tensors
// at any time (page and DRAM locality); the contiguous order gives each block
// one range.  Either way the assignment is fixed, so dw is reproducible.
struct RowSchedule {
  int64_t first, step, limit;
  int iters;
  int rows_per_iter;

  __host__ __device__ __forceinline__ int64_t row0(int it) const {
    return first + (int64_t)it * step;
  }
  // Rows of iteration `it`; 0 for any iteration outside [0, iters) (a
  // prefetch of iteration `iters`, which in reverse order would start before
  // row 0), so its descriptor covers nothing.
  __host__ __device__ __forceinline__ int rows(int it) const {
    if (it < 0 || it >= iters) return 0;
    const int64_t r0 = row0(it);
    const int64_t left = limit - r0;
    return (r0 < 0 || left <= 0) ? 0 : (left < rows_per_iter ? (int)left : rows_per_iter);
  }
};

// Strided order: block b takes row chunks b, b + G, b + 2G, ... (all blocks
// sweep one contiguous window of the tensors at any time); with kReverse the
// chunks are taken from the last one down.
template <bool kReverse>
__host__ __device__ __forceinline__ RowSchedule row_schedule(const TPGeom& g, int64_t group) {
  RowSchedule s;
  s.rows_per_iter = g.rows_per_iter;
  s.limit = g.n_rows;
  if constexpr (kReverse) {
    // Chunk k = T - 1 - (b + it * G).
    const int64_t chunks = (g.n_rows + g.rows_per_iter - 1) / g.rows_per_iter;
    s.first = (chunks - 1 - group) * g.rows_per_iter;
    s.step = -g.groups * g.rows_per_iter;
    s.iters = group < chunks ? (int)((chunks - group + g.groups - 1) / g.groups) : 0;
  } else {
    s.first = group * g.rows_per_iter;
    s.step = g.groups * g.rows_per_iter;
    s.iters = s.first < g.n_rows ? (int)((g.n_rows - s.first + s.step - 1) / s.step) : 0;
  }
  return s;
}

// ---------------------------------------------------------------------------
// Forward: out = sum over paths of w * CG(x, y)  (native_o2.py:209-221).
template <class P, int kLayout, bool kVec2>
__global__ __launch_bounds__(forward_block<P>(), kForwardWaves) void tp_forward_kernel(
    const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ w,
    float* __restrict__ out, TPGeom g) {
  constexpr int kTile = forward_tile<P>();
  constexpr bool kLds = forward_lds<P>();
  extern __shared__ float lds_w[];
  const int tile = blockIdx.x % g.tiles;
  const int64_t group = blockIdx.x / g.tiles;
  const Lane l = make_lane<P::kFull, kTile>(g, tile);
  const LaneOffsets o = lane_offsets<P::kFull, kLayout>(g, l);
  const int C = g.channels;
  // This lane's weight of every path (times the coupling magnitude): in
  // registers, or staged in LDS for the block's lanes (forward_lds).
  float wreg[kLds ? 1 : P::kPaths];
  WeightColumns<P> col{};
  if constexpr (kLds) {
    stage_weights<P, kTile>(lds_w, w, C, tile);
    __syncthreads();
    col = weight_columns<P>(l);
  } else {
    static_for<P::kPaths>([&](auto pc) {
      constexpr int p = decltype(pc)::value;
      constexpr PathSpec ps = P::paths[p];
      const int unit = (P::kFull && out_is_freq<P>(p)) ? ps.wunits + l.q : ps.wunits;
      wreg[p] = l.active ? w[unit * C + l.c] * ps.mag : 0.f;
    });
  }

  const RowSchedule sched = row_schedule<false>(g, group);
  float X[P::kKeys][2], Y[P::kKeys][2];
  for (int it = 0; it < sched.iters; ++it) {
    const int64_t row0 = sched.row0(it);
    const int rows = sched.rows(it);
    load_row<P, kLayout, kVec2, kForwardLoadPolicy>(rows_rsrc(x, row0, g.width, rows), C, l, o,
                                                    false, X);
    load_row<P, kLayout, kVec2, kForwardLoadPolicy>(rows_rsrc(y, row0, g.width, rows), C, l, o,
                                                    false, Y);
    float A[P::kKeys][2];
    static_for<P::kKeys>([&](auto kc) {
      A[decltype(kc)::value][0] = 0.f;
      A[decltype(kc)::value][1] = 0.f;
    });
    if constexpr (kLds) asm volatile("" : "+v"(col.freq), "+v"(col.scalar));
    static_for<P::kPaths>([&](auto pc) {
      constexpr int p = decltype(pc)::value;
      constexpr PathSpec ps = P::paths[p];
      float wv;
      if constexpr (kLds) wv = staged_weight<P, kTile, p>(lds_w, col);
      else wv = wreg[p];
      float f0, f1;
      path_value<P, p>(X, Y, f0, f1);
      A[ps.k3][0] = fmaf(wv, f0, A[ps.k3][0]);
      if constexpr (out_is_freq<P>(p)) A[ps.k3][1] = fmaf(wv, f1, A[ps.k3][1]);
    });
    store_row<P, kLayout, kVec2, kForwardStorePolicy>(rows_rsrc(out, row0, g.width, rows), C, l,
                                                      o, A);
  }
}

// ---------------------------------------------------------------------------
// Fused VJP: dx, dy and the weight adjoint in one pass over x, y, g.
//   dx[k1][i] += w * coef * g[k3][k] * y[k2][j]       (triton_o2.py:452-501)
//   dy[k2][j] += w * coef * g[k3][k] * x[k1][i]
//   dw[p, o]  += coef * x[k1][i] * y[k2][j] * g[k3][k] (triton_o2.py:571-607)
template <class P, int kLayout, bool kVec2>
__global__ __launch_bounds__(kBackwardBlock, kBackwardWaves) void tp_backward_kernel(
    const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ w,
    const float* __restrict__ gout, float* __restrict__ dx, float* __restrict__ dy,
    float* __restrict__ partial, TPGeom g, int needed) {
  constexpr int kTile = backward_tile<P>();
  extern __shared__ float lds_w[];
  const int tile = blockIdx.x % g.tiles;
  const int64_t group = blockIdx.x / g.tiles;
  const Lane l = make_lane<P::kFull, kTile>(g, tile);
  const LaneOffsets o = lane_offsets<P::kFull, kLayout>(g, l);
  const int C = g.channels;
  stage_weights<P, kTile>(lds_w, w, C, tile);
  __syncthreads();
  WeightColumns<P> col = weight_columns<P>(l);

  float dwacc[P::kPaths];
  static_for<P::kPaths>([&](auto pc) { dwacc[decltype(pc)::value] = 0.f; });

  // Reverse order: the first rows visited are the ones the forward touched
  // last, still in the memory-side cache.
  const RowSchedule sched = row_schedule<true>(g, group);
  // Stores of roles that were not requested go to idle offsets (dropped).
  LaneOffsets ox = o, oy = o;
  if (!(needed & 1)) ox.scalar_own = ox.freq = kIdle;
  if (!(needed & 2)) oy.scalar_own = oy.freq = kIdle;

  // Scalar outputs belong to the copy-0 lane; the copy-1 lane reads a zero
  // cotangent there, which removes its (wrong-copy) contributions.  The first
  // iteration's loads are issued before the loop (measured: loading at the
  // top of every iteration instead made the compiler schedule the loop body
  // differently and doubled the kernel's time at the headline shape).
  float X[P::kKeys][2], Y[P::kKeys][2], G[P::kKeys][2];
  {
    const int64_t row0 = sched.row0(0);
    const int rows = sched.rows(0);
    load_row<P, kLayout, kVec2, kBackwardLoadPolicy>(rows_rsrc(x, row0, g.width, rows), C, l, o,
                                                     false, X);
    load_row<P, kLayout, kVec2, kBackwardLoadPolicy>(rows_rsrc(y, row0, g.width, rows), C, l, o,
                                                     false, Y);
    load_row<P, kLayout, kVec2, kBackwardLoadPolicy>(rows_rsrc(gout, row0, g.width, rows), C, l,
                                                     o, true, G);
  }
  for (int it = 0; it < sched.iters; ++it) {
    const int64_t row0 = sched.row0(it);
    const int rows = sched.rows(it);
    if (it > 0) {
      load_row<P, kLayout, kVec2, kBackwardLoadPolicy>(rows_rsrc(x, row0, g.width, rows), C, l,
                                                       o, false, X);
      load_row<P, kLayout, kVec2, kBackwardLoadPolicy>(rows_rsrc(y, row0, g.width, rows), C, l,
                                                       o, false, Y);
      load_row<P, kLayout, kVec2, kBackwardLoadPolicy>(rows_rsrc(gout, row0, g.width, rows), C,
                                                       l, o, true, G);
    }

    float DX[P::kKeys][2], DY[P::kKeys][2];
    static_for<P::kKeys>([&](auto kc) {
      constexpr int k = decltype(kc)::value;
      DX[k][0] = DX[k][1] = DY[k][0] = DY[k][1] = 0.f;
    });
    // Re-read the weights from LDS every iteration: hoisting the loop-invariant
    // reads out of the loop would cost as many registers.
    asm volatile("" : "+v"(col.freq), "+v"(col.scalar));
    static_for<P::kPaths>([&](auto pc) {
      constexpr int p = decltype(pc)::value;
      constexpr PathSpec ps = P::paths[p];
      constexpr bool freq3 = out_is_freq<P>(p);
      const float wv = staged_weight<P, kTile, p>(lds_w, col);
      float f0, f1;
      path_value<P, p>(X, Y, f0, f1);
      dwacc[p] = fmaf(G[ps.k3][0], f0, dwacc[p]);
      if constexpr (freq3) dwacc[p] = fmaf(G[ps.k3][1], f1, dwacc[p]);
      const float h[2] = {wv * G[ps.k3][0], freq3 ? wv * G[ps.k3][1] : 0.f};
      static_for<ps.nt>([&](auto tc) {
        constexpr TermSpec ts = P::terms[ps.t0 + decltype(tc)::value];
        const float hk = ts.sign > 0 ? h[ts.k] : -h[ts.k];
        DX[ps.k1][ts.i] = fmaf(hk, Y[ps.k2][ts.j], DX[ps.k1][ts.i]);
        DY[ps.k2][ts.j] = fmaf(hk, X[ps.k1][ts.i], DY[ps.k2][ts.j]);
      });
    });
    if constexpr (P::kFull) {
      static_for<P::kKeys>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        if constexpr (P::keys[k].dim == 1) {
          DX[k][0] += pair_swap(DX[k][0]);
          DY[k][0] += pair_swap(DY[k][0]);
        }
      });
    }
    store_row<P, kLayout, kVec2, kBackwardStorePolicy>(rows_rsrc(dx, row0, g.width, rows), C, l,
                                                       ox, DX);
    store_row<P, kLayout, kVec2, kBackwardStorePolicy>(rows_rsrc(dy, row0, g.width, rows), C, l,
                                                       oy, DY);
  }

  if ((needed & 4) && l.active) {
    float* prow = partial + (group * g.rows_per_iter + l.slot) * (int64_t)g.weight_numel;
    static_for<P::kPaths>([&](auto pc) {
      constexpr int p = decltype(pc)::value;
      constexpr PathSpec ps = P::paths[p];
      if (out_is_freq<P>(p) || l.q == 0) {
        const int oc = ((out_is_freq<P>(p) && P::kFull) ? l.q * C : 0) + l.c;
        prow[ps.wunits * C + oc] = dwacc[p] * ps.mag;
      }
    });
  }
}

}  // namespace o2mi
