// Fused radial affine + V=1 O(2) uvu product for gfx950 (CDNA4).
//
// RadialUvuTensorProduct (radial_uvu.py:10-66, radial_streamed.py:37-57):
//   W[e, p*C + u] = sum_h hidden[e, h] alpha[p*C + u, h] + bias[p*C + u]
//   out[e, k, u, :] += W[e, p*C + u] * CG_p(x[e, i, u, :], y[e, j, :])
// The affine map runs on the fp32 matrix cores (v_mfma_f32_16x16x4_f32) and
// each 16-channel x 16-edge weight tile is consumed in registers by the
// product, so generated weights never reach memory.
//
// MFMA 16x16x4 f32 operand layout (checked on gfx950): lane l supplies
// A[l%16][l/16] and B[l/16][l%16]; D[4*(l/16) + r][l%16] is accumulator r of
// lane l.  Below, g = lane/16 and j = lane%16.
//
// Forward / input adjoints: o2mi_radial_streamed.hpp.  The weight tile is
// computed as W^T[channel, edge]: A = alpha (lane: row j, h = KH*g+s), B =
// hidden (lane: edge j, h = KH*g+s), so lane (g, j) ends up holding the
// weights of edge j for channels u0 + 4g + r, r = 0..3, and loads x, g and
// writes out / dx for exactly those (edge, channel) pairs.  The hidden
// adjoint, dh[e, h] = sum_{p,u} gw[e, p, u] alpha[p*C + u, h], reuses the
// weight adjoint gw in that accumulator layout as the B operand (K index =
// channel 4g + s at step s) against alpha read transposed from LDS.
//
// Affine-parameter adjoints (radial_weight_kernel, for structures with few
// paths; radial_weight_streamed_kernel otherwise).  dalpha = gw^T hidden and
// dbias = sum_e gw are sums over all edges.  A block owns one channel tile and
// a contiguous slice of edges; each wave owns the paths p = wave (mod 8) and
// keeps their dalpha tiles in accumulators for the whole slice.  Per 32 edges
// the block stages x, g (the tile's channels), y and hidden in LDS (double
// buffered, next tile prefetched into registers during compute); lane (g, j)
// forms gw for channel u0 + j and edge 4s + g at step s, which is the B
// operand of dalpha^T[h, channel] += hidden^T[h, edge] gw[edge, channel].
// Slice partials are summed in a fixed order afterwards: no atomics, the
// result is bitwise reproducible for a given edge count and device.
//
// Coupling values come from the module's fp32 [P][2][2][2] buffer at run time
// (any normalisation); which of the 8 slots are non-zero is fixed by the plan.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

namespace o2mi {
namespace radial {

struct REntry {
  int off;   // first input: offset in units of C; second input (V = 1): absolute offset
  int dim;   // 1 or 2
  int base;  // first input: component index within one (edge, channel); second: within the row
};

struct RPath {
  int i, j, k;
  int mask;  // bit (c*4 + a*2 + b): coupling slot [out c][in1 a][in2 b] is non-zero
  int neg;   // bit set: that slot's coupling is negative (all slots share one magnitude)
};

// Slot of the lowest non-zero coupling of a path.
constexpr int first_slot(int mask) {
  int s = 0;
  while (s < 8 && !((mask >> s) & 1)) ++s;
  return s;
}

using f4 = float __attribute__((ext_vector_type(4)));
using u32x4 = uint32_t __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kEdgesPerWave = 16;
constexpr uint32_t kIdle = 0x80000000u;
constexpr int kRsrcFlags = 0x00020000;

template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  [&]<int... I>(std::integer_sequence<int, I...>) __attribute__((always_inline)) {
    (f(std::integral_constant<int, I>{}), ...);
  }(std::make_integer_sequence<int, N>{});
}

template <int KH>
struct Geom {
  static constexpr int kHid = 4 * KH;      // padded hidden width
  static constexpr int kRow = kHid + 4;    // LDS row stride of the alpha tile (floats)
  static constexpr int kTiles = kHid / 16; // 16-row tiles of the hidden / alpha adjoints
  static_assert(KH % 4 == 0, "KH must be a multiple of 4");
};

struct Args {
  int64_t n;  // edges
  int C;      // channels (multiple of 16)
  int H;      // hidden width (multiple of 4, <= 4*KH)
  int W1;     // C * components of the first input
  int W2;     // width of the second input
  int V;      // copies of the second input (shared-weight uvu; 1 otherwise)
  const float* x;
  const float* y;
  const float* hidden;
  const float* alpha;  // [P*C, H]
  const float* bias;   // [P*C] or null
  const float* coef;   // [P][2][2][2]
  // Gathered first input: null, x row e for edge e; else x is a table of
  // x_rows rows (x_rows * W1 * 4 < 2^31 bytes) and edge e reads row
  // xindex[e]; an index outside [0, x_rows) reads zeros.
  const int64_t* xindex;
  int64_t x_rows;
  // Streamed kernels: channels per block along grid y (a multiple of 16; C
  // unless few edge blocks leave CUs idle).  Input adjoints split this way
  // write per-split dy / dhidden partials (part_dy [splits][n][W2], part_gh
  // [splits][n][H]) that a fixed-order sum finishes.
  int tile_span;
  float* part_dy;
  float* part_gh;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const float* base, int64_t row0,
                                                            int width, int64_t rows) {
  const int64_t valid = rows < 0 ? 0 : rows;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base) + row0 * width, 0,
                                           (int)(valid * width * 4), kRsrcFlags);
}

// First-input descriptor of the edges [e0, e0 + rows): those rows of x, or
// the whole node table when the first input is gathered.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t x_rsrc(const Args& a, int64_t e0,
                                                         int64_t rows) {
  return a.xindex ? rows_rsrc(a.x, 0, a.W1, a.x_rows) : rows_rsrc(a.x, e0, a.W1, rows);
}

// Byte offset of edge e0 + j's first-input row inside x_rsrc(a, e0, rows)
// (kIdle past the last edge or for an index outside the table).
__device__ __forceinline__ uint32_t x_row_off(const Args& a, int64_t e0, int64_t rows, int j) {
  if (!a.xindex) return (uint32_t)(j * a.W1) * 4u;
  if (j >= rows) return kIdle;
  const int64_t id = a.xindex[e0 + j];
  return (id >= 0 && id < a.x_rows) ? (uint32_t)id * (uint32_t)a.W1 * 4u : kIdle;
}

__device__ __forceinline__ float ld1(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, 0, 0));
}

__device__ __forceinline__ f4 ld4(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, 0, 0));
}

__device__ __forceinline__ void st4(__amdgpu_buffer_rsrc_t r, f4 v, uint32_t voff) {
  // Default (write-back) policy: a wave's 16-byte stores fill a 128-byte line
  // in two instructions, and a 16-channel tile fills half a line of a
  // one-component entry; L2 merges the parts into whole-line writes.  As
  // non-temporal stores the parts reached HBM separately (writes measured
  // 1.15x the output bytes, against 1.00x here).
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, (int)voff, 0, 0);
}

__device__ __forceinline__ f4 mfma(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// The couplings of path p from the [P][8] LDS table: the halves the path
// uses as 16-byte reads (one LDS instruction per half, not one per slot).
template <int Mask>
struct PathCoefs {
  f4 lo, hi;
};

template <int Mask>
__device__ __forceinline__ PathCoefs<Mask> load_coefs(const float* cf, int p) {
  PathCoefs<Mask> c;
  if constexpr ((Mask & 0x0F) != 0) c.lo = *reinterpret_cast<const f4*>(cf + p * 8);
  if constexpr ((Mask & 0xF0) != 0) c.hi = *reinterpret_cast<const f4*>(cf + p * 8 + 4);
  return c;
}

template <int Slot, int Mask>
__device__ __forceinline__ float coef_at(const PathCoefs<Mask>& c) {
  if constexpr (Slot < 4) return c.lo[Slot];
  else return c.hi[Slot - 4];
}

// The 4 x dim values of one first-input entry for channels u .. u+3 of one row.
template <int Dim>
__device__ __forceinline__ void load_entry(__amdgpu_buffer_rsrc_t r, uint32_t row_off, int off_c,
                                           int u, float* dst) {
  const uint32_t voff = row_off + (uint32_t)(off_c + Dim * u) * 4u;
  const f4 v0 = ld4(r, voff);
  dst[0] = v0.x; dst[1] = v0.y; dst[2] = v0.z; dst[3] = v0.w;
  if constexpr (Dim == 2) {
    const f4 v1 = ld4(r, voff + 16u);
    dst[4] = v1.x; dst[5] = v1.y; dst[6] = v1.z; dst[7] = v1.w;
  }
}

// Number of one-component first-input entries before entry e.
template <class Plan>
constexpr int dim1_before(int e) {
  int n = 0;
  for (int k = 0; k < e; ++k) n += Plan::e1[k].dim == 1;
  return n;
}

// Channel tiles taken in pairs (u0, u0 + 16).  A 16-channel tile covers a
// whole 128-byte line of a two-component entry but only half a line of a
// one-component entry; read in two tiles, that line is evicted from L2
// between them and fetched twice.  In the first tile of a pair (lo) a lane
// also loads its 4 channels of the second tile and carries them over; the
// second tile (hi) takes them from the carry and its own load is idle (an
// out-of-range buffer load moves no data).  Both flags are wave-uniform.
struct TilePair {
  bool lo, hi;
};

// The pairing of channel tile u0 of [u_begin, u_end) (all-false: unpaired).
__device__ __forceinline__ TilePair tile_pair(bool enable, int u0, int u_begin, int u_end) {
  const bool odd = ((u0 - u_begin) >> 4) & 1;
  return TilePair{enable && !odd && u0 + 16 < u_end, enable && odd};
}

// load_entry for a paired tile; carry holds 4 floats of a one-component entry.
template <int Dim>
__device__ __forceinline__ void load_entry_paired(__amdgpu_buffer_rsrc_t r, uint32_t row_off,
                                                  int off_c, int u, float* dst, float* carry,
                                                  TilePair tp) {
  if constexpr (Dim == 1) {
    const uint32_t voff = row_off + (uint32_t)(off_c + u) * 4u;
    if (tp.hi) {
      dst[0] = carry[0]; dst[1] = carry[1]; dst[2] = carry[2]; dst[3] = carry[3];
    } else {
      const f4 v = ld4(r, voff);
      dst[0] = v.x; dst[1] = v.y; dst[2] = v.z; dst[3] = v.w;
    }
    if (tp.lo) {
      const f4 next = ld4(r, voff + 64u);
      carry[0] = next.x; carry[1] = next.y; carry[2] = next.z; carry[3] = next.w;
    }
  } else {
    load_entry<Dim>(r, row_off, off_c, u, dst);
  }
}

template <int Dim>
__device__ __forceinline__ void store_entry(__amdgpu_buffer_rsrc_t r, uint32_t row_off, int off_c,
                                            int u, const float* src) {
  const uint32_t voff = row_off + (uint32_t)(off_c + Dim * u) * 4u;
  st4(r, f4{src[0], src[1], src[2], src[3]}, voff);
  if constexpr (Dim == 2) st4(r, f4{src[4], src[5], src[6], src[7]}, voff + 16u);
}

template <class Plan>
__device__ __forceinline__ void load_row(__amdgpu_buffer_rsrc_t r, uint32_t row_off, int C, int u,
                                         float* v) {
  static_for<Plan::kEntries1>([&](auto ec) {
    constexpr REntry e = Plan::e1[decltype(ec)::value];
    load_entry<e.dim>(r, row_off, e.off * C, u, v + 4 * e.base);
  });
}

// load_row for a paired tile; carry: 4 floats per one-component entry.
template <class Plan>
__device__ __forceinline__ void load_row_paired(__amdgpu_buffer_rsrc_t r, uint32_t row_off, int C,
                                                int u, float* v, float* carry, TilePair tp) {
  static_for<Plan::kEntries1>([&](auto ec) {
    constexpr int k = decltype(ec)::value;
    constexpr REntry e = Plan::e1[k];
    load_entry_paired<e.dim>(r, row_off, e.off * C, u, v + 4 * e.base,
                             carry + 4 * dim1_before<Plan>(k), tp);
  });
}

template <class Plan>
__device__ __forceinline__ void store_row(__amdgpu_buffer_rsrc_t r, uint32_t row_off, int C,
                                          int u, const float* v) {
  static_for<Plan::kEntries1>([&](auto ec) {
    constexpr REntry e = Plan::e1[decltype(ec)::value];
    store_entry<e.dim>(r, row_off, e.off * C, u, v + 4 * e.base);
  });
}

// hidden[edge j][KH*g + s], zero past the hidden width.
template <int KH>
__device__ __forceinline__ void load_hidden(__amdgpu_buffer_rsrc_t rh, int H, int g, int j,
                                            float* hid) {
  static_for<KH / 4>([&](auto qc) {
    constexpr int q = decltype(qc)::value;
    const int h = KH * g + 4 * q;
    const uint32_t voff = h < H ? (uint32_t)(j * H + h) * 4u : kIdle;
    const f4 v = ld4(rh, voff);
    hid[4 * q] = v.x; hid[4 * q + 1] = v.y; hid[4 * q + 2] = v.z; hid[4 * q + 3] = v.w;
  });
}

// W^T tile of the path staged in LDS slot p: bias + sum_h alpha[path*C + u0 +
// 4g + r, h] hidden[j, h].  bias_off (the slot-0 bias + 4g) and arow_off (the
// slot-0 alpha row j + KH*g) are the lane's base offsets, laundered by the
// caller.
template <int KH>
__device__ __forceinline__ f4 weight_tile(const float* s_mem, int bias_off, int arow_off, int p,
                                          const float* hid) {
  using G = Geom<KH>;
  f4 w = *reinterpret_cast<const f4*>(s_mem + bias_off + p * 16);
  const float* arow = s_mem + arow_off + p * 16 * G::kRow;
  static_for<KH / 4>([&](auto qc) {
    constexpr int q = decltype(qc)::value;
    const f4 av = *reinterpret_cast<const f4*>(arow + 4 * q);
    w = mfma(av.x, hid[4 * q], w);
    w = mfma(av.y, hid[4 * q + 1], w);
    w = mfma(av.z, hid[4 * q + 2], w);
    w = mfma(av.w, hid[4 * q + 3], w);
  });
  return w;
}

// Staged tile of the affine-adjoint kernel: Plan::kWeightEdges edges of x and g
// (this block's 16 channels), y and hidden.  Row strides are odd / 16 mod 32
// so the per-step LDS reads of 4 edges x 16 channels do not collide in banks
// (kXPad 1).  An even x row stride (kXPad 2) keeps the two components of an
// entry 8-byte aligned: they are then read as one 64-bit word at a 16-bit
// offset, with no address arithmetic.
template <class Plan, int KH, int NT = kThreads, int kXPad = 1>
struct WTile {
  static constexpr int kWeightEdges = Plan::kWeightEdges;
  static constexpr int kXS = 16 * Plan::kComps1 + kXPad;
  static constexpr int kYS = Plan::kComps2;
  static constexpr int kHS = Geom<KH>::kHid + 16;
  static constexpr int kX = kWeightEdges * kXS;
  static constexpr int kY = kWeightEdges * kYS;
  static constexpr int kH = kWeightEdges * kHS;
  static constexpr int kFloats = 2 * kX + kY + kH;
  // Per-thread staging registers: ceil(elements / threads) per part.
  static constexpr int kXPer = (kWeightEdges * 16 * Plan::kComps1 + NT - 1) / NT;
  static constexpr int kYPer = (kY + NT - 1) / NT;
  static constexpr int kHPer = (kWeightEdges * Geom<KH>::kHid + NT - 1) / NT;
};

template <class Plan, int KH, int NT = kThreads>
struct WPrefetch {
  using T = WTile<Plan, KH, NT>;
  float x[T::kXPer], g[T::kXPer];
  float y[T::kYPer], h[T::kHPer];
};

// Element idx of the x/g part of a tile: edge idx / (16 NC), then the
// channel-tile component (entry-major, [channel][component] inside an entry).
template <class Plan>
__device__ __forceinline__ int tile_x_offset(int idx_in_edge, int C, int u0) {
  int off = 0;
  static_for<Plan::kEntries1>([&](auto ec) {
    constexpr REntry e = Plan::e1[decltype(ec)::value];
    const int lo = 16 * e.base, hi = 16 * (e.base + e.dim);
    if (idx_in_edge >= lo && idx_in_edge < hi) off = e.off * C + e.dim * u0 + (idx_in_edge - lo);
  });
  return off;
}

// Gathered first input: lane L of every wave holds the table row of edge
// t0 + (L % 32) of a tile (-1 past the end).  Loaded one tile ahead of its use,
// so the x loads of a tile never wait on a dependent index load.
__device__ __forceinline__ int64_t tile_rows(const Args& a, int64_t t0, int64_t t_end) {
  if (!a.xindex) return 0;
  const int64_t e = t0 + (threadIdx.x & 31);
  return e < t_end ? a.xindex[e] : -1;
}

// Byte offset of tile edge `edge`'s table row (kIdle if outside the table),
// taken from the lane that loaded it.
__device__ __forceinline__ uint32_t tile_row_off(const Args& a, int64_t rows_of_tile, int edge) {
  const int lo = __shfl((int)(uint32_t)(uint64_t)rows_of_tile, edge);
  const int hi = __shfl((int)(uint32_t)((uint64_t)rows_of_tile >> 32), edge);
  const int64_t id = (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
  return (id >= 0 && id < a.x_rows) ? (uint32_t)id * (uint32_t)a.W1 * 4u : kIdle;
}

// Byte offsets of this thread's x / g tile elements inside a tile's edge rows
// (kIdle past the tile), and their column part: the same for every tile of a
// block, so computed once (the entry lookup is a compare chain per element).
template <class Plan, int KH, int NT = kThreads>
struct WCols {
  uint32_t voff[WTile<Plan, KH, NT>::kXPer], col[WTile<Plan, KH, NT>::kXPer];
};

template <class Plan, int KH, int NT = kThreads>
__device__ __forceinline__ void weight_cols(WCols<Plan, KH, NT>& c, const Args& a, int u0) {
  using T = WTile<Plan, KH, NT>;
  constexpr int XE = 16 * Plan::kComps1;
  static_for<T::kXPer>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    const int idx = threadIdx.x + k * NT;
    c.voff[k] = c.col[k] = kIdle;
    if (idx < Plan::kWeightEdges * XE) {
      const int edge = idx / XE;
      c.col[k] = (uint32_t)tile_x_offset<Plan>(idx - edge * XE, a.C, u0) * 4u;
      c.voff[k] = (uint32_t)(edge * a.W1) * 4u + c.col[k];
    }
  });
}

template <class Plan, int KH, int NT = kThreads>
__device__ __forceinline__ void weight_fetch(WPrefetch<Plan, KH, NT>& pf, const Args& a,
                                             const float* gout, int64_t t0, int64_t t_end,
                                             const WCols<Plan, KH, NT>& cols,
                                             int64_t rows_of_tile) {
  using T = WTile<Plan, KH, NT>;
  constexpr int XE = 16 * Plan::kComps1;
  constexpr int kWeightEdges = Plan::kWeightEdges;
  const int64_t rows = t_end - t0 < kWeightEdges ? t_end - t0 : kWeightEdges;
  const auto rx = x_rsrc(a, t0, rows);
  const auto rg = rows_rsrc(gout, t0, a.W1, rows);
  const auto ry = rows_rsrc(a.y, t0, a.W2, rows);
  const auto rh = rows_rsrc(a.hidden, t0, a.H, rows);
  // Offsets first (the table rows come from other lanes), then every load, so
  // no load of the tile waits behind another.
  uint32_t xoff[T::kXPer];
  static_for<T::kXPer>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    xoff[k] = cols.voff[k];
    if (a.xindex) {
      const int edge = (threadIdx.x + k * NT) / XE;
      const uint32_t row = (cols.col[k] != kIdle && edge < rows)
                               ? tile_row_off(a, rows_of_tile, edge) : kIdle;
      xoff[k] = row == kIdle ? kIdle : row + cols.col[k];
    }
  });
  __builtin_amdgcn_sched_barrier(0);
  static_for<T::kXPer>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    pf.x[k] = ld1(rx, xoff[k]);
    pf.g[k] = ld1(rg, cols.voff[k]);
  });
  static_for<T::kYPer>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    const int idx = threadIdx.x + k * NT;
    pf.y[k] = ld1(ry, idx < T::kY ? (uint32_t)idx * 4u : kIdle);  // rows of y are contiguous
  });
  static_for<T::kHPer>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    const int idx = threadIdx.x + k * NT;
    const int edge = idx / Geom<KH>::kHid, h = idx - edge * Geom<KH>::kHid;
    const bool ok = idx < kWeightEdges * Geom<KH>::kHid && h < a.H;
    pf.h[k] = ld1(rh, ok ? (uint32_t)(edge * a.H + h) * 4u : kIdle);
  });
}

template <class Plan, int KH, int NT = kThreads>
__device__ __forceinline__ void weight_commit(const WPrefetch<Plan, KH, NT>& pf, float* buf) {
  using T = WTile<Plan, KH, NT>;
  constexpr int XE = 16 * Plan::kComps1;
  constexpr int kWeightEdges = Plan::kWeightEdges;
  float* sx = buf;
  float* sg = buf + T::kX;
  float* sy = buf + 2 * T::kX;
  float* sh = sy + T::kY;
  static_for<T::kXPer>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    const int idx = threadIdx.x + k * NT;
    if (idx < kWeightEdges * XE) {
      const int edge = idx / XE, rest = idx - edge * XE;
      sx[edge * T::kXS + rest] = pf.x[k];
      sg[edge * T::kXS + rest] = pf.g[k];
    }
  });
  static_for<T::kYPer>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    const int idx = threadIdx.x + k * NT;
    if (idx < T::kY) sy[idx] = pf.y[k];
  });
  static_for<T::kHPer>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    const int idx = threadIdx.x + k * NT;
    if (idx < kWeightEdges * Geom<KH>::kHid) {
      const int edge = idx / Geom<KH>::kHid, h = idx - edge * Geom<KH>::kHid;
      sh[edge * T::kHS + h] = pf.h[k];
    }
  });
}

// dalpha / dbias partials of paths [P0, P0 + NP) over one edge slice and one
// channel tile; wave w owns the paths P0 + w (mod 8).
template <class Plan, int KH, int P0, int NP>
__device__ __forceinline__ void weight_body(float* s_mem, const Args& a, const float* gout,
                                            int64_t edges_per_slice, float* part_alpha,
                                            float* part_bias) {
  using G = Geom<KH>;
  using T = WTile<Plan, KH>;
  constexpr int P = Plan::kPaths;
  constexpr int kWeightEdges = Plan::kWeightEdges;
  constexpr int NPW = (NP + kWaves - 1) / kWaves;
  constexpr int kCoefPad = (P * 8 + 3) / 4 * 4;
  float* s_coef = s_mem;
  float* s_tile = s_mem + kCoefPad;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
  const int g = lane >> 4, j = lane & 15;
  const int u0 = blockIdx.y * 16;
  const int64_t begin = (int64_t)blockIdx.x * edges_per_slice;
  const int64_t end = begin + edges_per_slice < a.n ? begin + edges_per_slice : a.n;
  const int tiles = end > begin ? (int)((end - begin + kWeightEdges - 1) / kWeightEdges) : 0;

  for (int idx = threadIdx.x; idx < P * 8; idx += kThreads) s_coef[idx] = a.coef[idx];
  f4 ga[NPW][G::kTiles];
  float gb[NPW];
  static_for<NPW>([&](auto qc) {
    constexpr int q = decltype(qc)::value;
    gb[q] = 0.f;
    static_for<G::kTiles>([&](auto tc) { ga[q][decltype(tc)::value] = f4{0.f, 0.f, 0.f, 0.f}; });
  });

  WCols<Plan, KH> cols;
  weight_cols<Plan, KH>(cols, a, u0);
  WPrefetch<Plan, KH> pf;
  if (tiles > 0) {
    weight_fetch<Plan, KH>(pf, a, gout, begin, end, cols, tile_rows(a, begin, end));
    weight_commit<Plan, KH>(pf, s_tile);
  }
  int64_t next_rows = tile_rows(a, begin + kWeightEdges, end);
  __syncthreads();
  for (int t = 0; t < tiles; ++t) {
    const bool more = t + 1 < tiles;
    if (more) {
      const int64_t t1 = begin + (int64_t)(t + 1) * kWeightEdges;
      weight_fetch<Plan, KH>(pf, a, gout, t1, end, cols, next_rows);
      next_rows = tile_rows(a, t1 + kWeightEdges, end);
    }
    const float* buf = s_tile + (t & 1) * T::kFloats;
    const float* sx = buf;
    const float* sg = buf + T::kX;
    const float* sy = buf + 2 * T::kX;
    const float* sh = sy + T::kY;
    // Unrolled by 4 so a wave issues the next steps' LDS reads while its
    // MFMAs run (-7% against no unrolling at configs[4]; the couplings stay
    // re-read per step: hoisting them spills).
#pragma unroll 4
    for (int s = 0; s < kWeightEdges / 4; ++s) {
      const int edge = 4 * s + g;
      int coef_off = 0;
      asm volatile("" : "+v"(coef_off));  // re-read couplings per step, do not hoist
      const float* cf_step = s_coef + coef_off;
      float xv[Plan::kComps1], gv[Plan::kComps1], yv[Plan::kComps2], hv[G::kTiles];
      static_for<Plan::kEntries1>([&](auto ec) {
        constexpr REntry e = Plan::e1[decltype(ec)::value];
        static_for<e.dim>([&](auto dc) {
          constexpr int d = decltype(dc)::value;
          const int o = edge * T::kXS + 16 * e.base + j * e.dim + d;
          xv[e.base + d] = sx[o];
          gv[e.base + d] = sg[o];
        });
      });
      static_for<Plan::kComps2>([&](auto cc) {
        yv[decltype(cc)::value] = sy[edge * T::kYS + decltype(cc)::value];
      });
      static_for<G::kTiles>([&](auto tc) {
        hv[decltype(tc)::value] = sh[edge * T::kHS + 16 * decltype(tc)::value + j];
      });
      static_for<NP>([&](auto pc) {
        constexpr int p = P0 + decltype(pc)::value;
        constexpr int q = decltype(pc)::value / kWaves;
        if (wave == decltype(pc)::value % kWaves) {
          constexpr RPath ps = Plan::paths[p];
          constexpr REntry X = Plan::e1[ps.i];
          constexpr REntry Y = Plan::e2[ps.j];
          constexpr REntry O = Plan::e1[ps.k];
          float gw = 0.f;
          // Scalar coupling reads here: the 16-byte form measured slower in
          // this resident kernel (more live registers across the path loop).
          static_for<8>([&](auto sc) {
            constexpr int slot = decltype(sc)::value;
            constexpr int c = slot >> 2, ia = (slot >> 1) & 1, ib = slot & 1;
            if constexpr ((ps.mask >> slot) & 1)
              gw += cf_step[p * 8 + slot] * yv[Y.base + ib] * (xv[X.base + ia] * gv[O.base + c]);
          });
          gb[q] += gw;
          static_for<G::kTiles>([&](auto tc) {
            constexpr int tt = decltype(tc)::value;
            ga[q][tt] = mfma(hv[tt], gw, ga[q][tt]);
          });
        }
      });
    }
    if (more) weight_commit<Plan, KH>(pf, s_tile + ((t + 1) & 1) * T::kFloats);
    __syncthreads();
  }

  const int64_t PC = (int64_t)P * a.C;
  float* pa = part_alpha + (int64_t)blockIdx.x * PC * a.H;
  float* pb = part_bias + (int64_t)blockIdx.x * PC;
  static_for<NP>([&](auto pc) {
    constexpr int p = P0 + decltype(pc)::value;
    constexpr int q = decltype(pc)::value / kWaves;
    if (wave == decltype(pc)::value % kWaves) {
      const int64_t row = (int64_t)p * a.C + u0 + j;
      static_for<G::kTiles>([&](auto tc) {
        constexpr int tt = decltype(tc)::value;
        const int h = 16 * tt + 4 * g;
        if (h < a.H) *reinterpret_cast<f4*>(pa + row * a.H + h) = ga[q][tt];
      });
      float b = gb[q];
      b += __shfl_xor(b, 16);
      b += __shfl_xor(b, 32);
      if (g == 0) pb[row] = b;
    }
  });
}

// A plan with another edge count per staged tile.
template <class Plan, int E>
struct WithEdges : Plan {
  static constexpr int kWeightEdges = E;
};

// Largest staged tile (32, 16 or 8 edges) whose double buffer fits LDS.
template <class Plan, int KH>
constexpr int dw_edges() {
  constexpr int kCoefPad = (Plan::kPaths * 8 + 3) / 4 * 4;
  if constexpr (4 * (kCoefPad + 2 * WTile<WithEdges<Plan, 32>, KH>::kFloats) <= 160 * 1024)
    return 32;
  else if constexpr (4 * (kCoefPad + 2 * WTile<WithEdges<Plan, 16>, KH>::kFloats) <= 160 * 1024)
    return 16;
  else
    return 8;
}

// Grid (slices, C/16).  part_alpha: [slices][P*C][H]; part_bias: [slices][P*C].
template <class Plan, int KH>
__global__ __launch_bounds__(kThreads, 1) void radial_weight_kernel(
    Args a, const float* gout, int64_t edges_per_slice, float* part_alpha, float* part_bias) {
  using T = WTile<Plan, KH>;
  constexpr int P = Plan::kPaths;
  constexpr int kCoefPad = (P * 8 + 3) / 4 * 4;
  __shared__ __attribute__((aligned(16))) float s_mem[kCoefPad + 2 * T::kFloats];
  weight_body<Plan, KH, 0, P>(s_mem, a, gout, edges_per_slice, part_alpha, part_bias);
}

}  // namespace radial
}  // namespace o2mi
