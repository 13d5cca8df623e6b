// O(2) uvu product kernels for gfx950 with runtime path tables.
//
// uvu plans vary with (C, V, m_max, parities, normalisations), so the path
// table is data: the int32 records of the reference's register_metadata
// (uvu_triton.py:39-67) and the padded [P][2][2][2] couplings.  Paths,
// entries and coupling values are read with wave-uniform indices (scalar
// loads); rows and channels vary per lane.
//
//   out[k][n,u,l] += sum_ij c[p][l][i][j] x[i][n,u,i] (sum_v w[p,u,v] y[j][n,v,j])
//   dx  = sum_{l,j} g c p_j,    r_j = sum_{i,l} x g c  (d out / d proj_j)
//   dy[j][n,v,:] += sum_u w[p,u,v] r(u, :),   dw[p,u,v] = sum_j r_j y[v,j]
//
// One writer per output element, fixed summation order: deterministic.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>

#include "ictc_o2_hp_amd.h"
#include "o2mi_error.hpp"

namespace o2mi {
namespace uvu {

struct Problem {
  int64_t n;
  int C, V, P, NO, NX, NY, W1, W2;
  int64_t wnum;  // P * C * V
  int shared;
  const int* info;
  const float* coef;
  const int* order1;
  const int* order2;
};

struct PathRec {
  int xo, yo, oo, xd, yd, od, wo;
};

__device__ __forceinline__ PathRec path_rec(const Problem& pr, int p) {
  const int* r = pr.info + 7 * p;
  return {r[0], r[1], r[2], r[3], r[4], r[5], r[6]};
}

// Entry record: (offset, dim, begin, end) of output (role 0), first (1) or
// second (2) entries.
__device__ __forceinline__ void entry_rec(const Problem& pr, int role, int e, int& off, int& dim,
                                          int& begin, int& end) {
  const int base = pr.P + (role >= 1 ? pr.NO : 0) + (role == 2 ? pr.NX : 0) + e;
  const int* r = pr.info + 7 * base;
  off = r[0];
  dim = r[1];
  begin = r[2];
  end = r[3];
}

// proj_j = sum_v w[v] y[v, j] for one (row, u).
__device__ __forceinline__ void project(const float* __restrict__ wp, const float* __restrict__ yr,
                                        int yo, int yd, int V, float& p0, float& p1) {
  p0 = 0.f;
  p1 = 0.f;
  if (yd == 2) {
    for (int v = 0; v < V; ++v) {
      const float wv = wp[v];
      p0 = fmaf(wv, yr[yo + 2 * v], p0);
      p1 = fmaf(wv, yr[yo + 2 * v + 1], p1);
    }
  } else {
    for (int v = 0; v < V; ++v) p0 = fmaf(wp[v], yr[yo + v], p0);
  }
}

__global__ __launch_bounds__(256) void uvu_forward_kernel(Problem pr, const float* __restrict__ x,
                                                          const float* __restrict__ y,
                                                          const float* __restrict__ w,
                                                          float* __restrict__ out) {
  const int64_t item = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (item >= pr.n * pr.C) return;  // no barriers below
  const int64_t n = item / pr.C;
  const int u = (int)(item - n * pr.C);
  const float* xr = x + n * pr.W1;
  const float* yr = y + n * pr.W2;
  float* orow = out + n * pr.W1;
  const float* wr = pr.shared ? w : w + n * pr.wnum;
  for (int k = 0; k < pr.NO; ++k) {
    int oo, od, begin, end;
    entry_rec(pr, 0, k, oo, od, begin, end);
    float acc0 = 0.f, acc1 = 0.f;
    for (int p = begin; p < end; ++p) {
      const PathRec r = path_rec(pr, p);
      const float* c = pr.coef + 8 * p;
      const float a0 = xr[r.xo + u * r.xd];
      const float a1 = r.xd == 2 ? xr[r.xo + u * r.xd + 1] : 0.f;
      float p0, p1;
      project(wr + r.wo + (int64_t)u * pr.V, yr, r.yo, r.yd, pr.V, p0, p1);
      acc0 += a0 * (c[0] * p0 + c[1] * p1) + a1 * (c[2] * p0 + c[3] * p1);
      acc1 += a0 * (c[4] * p0 + c[5] * p1) + a1 * (c[6] * p0 + c[7] * p1);
    }
    orow[oo + u * od] = acc0;
    if (od == 2) orow[oo + u * od + 1] = acc1;
  }
}

// dx (bit 1) and per-row dw (bit 4), one (row, u) per thread, paths grouped
// by first-input entry so each dx element has one writer.
__global__ __launch_bounds__(256) void uvu_backward_x_kernel(
    Problem pr, const float* __restrict__ x, const float* __restrict__ y,
    const float* __restrict__ w, const float* __restrict__ g, float* __restrict__ gx,
    float* __restrict__ gw, int needed) {
  const int64_t item = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (item >= pr.n * pr.C) return;
  const int64_t n = item / pr.C;
  const int u = (int)(item - n * pr.C);
  const float* xr = x + n * pr.W1;
  const float* yr = y + n * pr.W2;
  const float* gr = g + n * pr.W1;
  const float* wr = pr.shared ? w : w + n * pr.wnum;
  const bool want_x = needed & 1;
  const bool want_w = (needed & 4) && !pr.shared;
  for (int i = 0; i < pr.NX; ++i) {
    int xo, xd, begin, end;
    entry_rec(pr, 1, i, xo, xd, begin, end);
    float d0 = 0.f, d1 = 0.f;
    for (int q = begin; q < end; ++q) {
      const int p = pr.order1[q];
      const PathRec r = path_rec(pr, p);
      const float* c = pr.coef + 8 * p;
      const float g0 = gr[r.oo + u * r.od];
      const float g1 = r.od == 2 ? gr[r.oo + u * r.od + 1] : 0.f;
      if (want_x) {
        float p0, p1;
        project(wr + r.wo + (int64_t)u * pr.V, yr, r.yo, r.yd, pr.V, p0, p1);
        d0 += g0 * (c[0] * p0 + c[1] * p1) + g1 * (c[4] * p0 + c[5] * p1);
        d1 += g0 * (c[2] * p0 + c[3] * p1) + g1 * (c[6] * p0 + c[7] * p1);
      }
      if (want_w) {
        const float a0 = xr[r.xo + u * r.xd];
        const float a1 = r.xd == 2 ? xr[r.xo + u * r.xd + 1] : 0.f;
        const float r0 = a0 * (c[0] * g0 + c[4] * g1) + a1 * (c[2] * g0 + c[6] * g1);
        const float r1 = a0 * (c[1] * g0 + c[5] * g1) + a1 * (c[3] * g0 + c[7] * g1);
        float* dst = gw + n * pr.wnum + r.wo + (int64_t)u * pr.V;
        if (r.yd == 2) {
          for (int v = 0; v < pr.V; ++v) dst[v] = r0 * yr[r.yo + 2 * v] + r1 * yr[r.yo + 2 * v + 1];
        } else {
          for (int v = 0; v < pr.V; ++v) dst[v] = r0 * yr[r.yo + v];
        }
      }
    }
    if (want_x) {
      gx[n * pr.W1 + xo + u * xd] = d0;
      if (xd == 2) gx[n * pr.W1 + xo + u * xd + 1] = d1;
    }
  }
}

__device__ __forceinline__ float wave_sum(float v) {
  for (int s = 32; s > 0; s >>= 1) v += __shfl_xor(v, s, 64);
  return v;
}

// dy (bit 2): one wave per row, lanes over u; paths grouped by second entry.
__global__ __launch_bounds__(256) void uvu_backward_y_kernel(Problem pr,
                                                             const float* __restrict__ x,
                                                             const float* __restrict__ w,
                                                             const float* __restrict__ g,
                                                             float* __restrict__ gy) {
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= pr.n) return;  // whole waves leave together; no barriers below
  const float* xr = x + n * pr.W1;
  const float* gr = g + n * pr.W1;
  const float* wr = pr.shared ? w : w + n * pr.wnum;
  for (int j = 0; j < pr.NY; ++j) {
    int yo, yd, begin, end;
    entry_rec(pr, 2, j, yo, yd, begin, end);
    for (int v = 0; v < pr.V; ++v) {
      float s0 = 0.f, s1 = 0.f;
      for (int q = begin; q < end; ++q) {
        const int p = pr.order2[q];
        const PathRec r = path_rec(pr, p);
        const float* c = pr.coef + 8 * p;
        for (int u = lane; u < pr.C; u += 64) {
          const float a0 = xr[r.xo + u * r.xd];
          const float a1 = r.xd == 2 ? xr[r.xo + u * r.xd + 1] : 0.f;
          const float g0 = gr[r.oo + u * r.od];
          const float g1 = r.od == 2 ? gr[r.oo + u * r.od + 1] : 0.f;
          const float r0 = a0 * (c[0] * g0 + c[4] * g1) + a1 * (c[2] * g0 + c[6] * g1);
          const float r1 = a0 * (c[1] * g0 + c[5] * g1) + a1 * (c[3] * g0 + c[7] * g1);
          const float wv = wr[r.wo + (int64_t)u * pr.V + v];
          s0 = fmaf(wv, r0, s0);
          s1 = fmaf(wv, r1, s1);
        }
      }
      s0 = wave_sum(s0);
      s1 = wave_sum(s1);
      if (lane == 0) {
        gy[n * pr.W2 + yo + v * yd] = s0;
        if (yd == 2) gy[n * pr.W2 + yo + v * yd + 1] = s1;
      }
    }
  }
}

// ---- Per-row weights with V = 1 (the radial product's composed path) --------
// Same mapping as the generic kernels (thread = (row, u), so a wave covers
// consecutive channels of one row and each path's weights are one coalesced
// load), but paths are taken kV1Batch at a time: their records, weights and
// x / g / y operands are all loaded before any is used, so a wave has
// kV1Batch independent loads in flight instead of one.  Each output element
// still sums its paths in table order (deterministic, as above).
constexpr int kV1Batch = 8;

__global__ __launch_bounds__(256) void uvu_v1_forward_kernel(Problem pr,
                                                             const float* __restrict__ x,
                                                             const float* __restrict__ y,
                                                             const float* __restrict__ w,
                                                             float* __restrict__ out) {
  const int64_t item = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (item >= pr.n * pr.C) return;  // no barriers below
  const int64_t n = item / pr.C;
  const int u = (int)(item - n * pr.C);
  const float* xr = x + n * pr.W1;
  const float* yr = y + n * pr.W2;
  const float* wr = w + n * pr.wnum + u;
  float* orow = out + n * pr.W1;
  for (int k = 0; k < pr.NO; ++k) {
    int oo, od, begin, end;
    entry_rec(pr, 0, k, oo, od, begin, end);
    float acc0 = 0.f, acc1 = 0.f;
    for (int p0 = begin; p0 < end; p0 += kV1Batch) {
      float wv[kV1Batch], a0[kV1Batch], a1[kV1Batch], y0[kV1Batch], y1[kV1Batch];
#pragma unroll
      for (int b = 0; b < kV1Batch; ++b) {
        if (p0 + b < end) {
          const PathRec r = path_rec(pr, p0 + b);
          wv[b] = wr[r.wo];
          a0[b] = xr[r.xo + u * r.xd];
          a1[b] = r.xd == 2 ? xr[r.xo + u * r.xd + 1] : 0.f;
          y0[b] = yr[r.yo];
          y1[b] = r.yd == 2 ? yr[r.yo + 1] : 0.f;
        }
      }
#pragma unroll
      for (int b = 0; b < kV1Batch; ++b) {
        if (p0 + b < end) {
          const float* c = pr.coef + 8 * (p0 + b);
          const float p0v = wv[b] * y0[b], p1v = wv[b] * y1[b];
          acc0 += a0[b] * (c[0] * p0v + c[1] * p1v) + a1[b] * (c[2] * p0v + c[3] * p1v);
          acc1 += a0[b] * (c[4] * p0v + c[5] * p1v) + a1[b] * (c[6] * p0v + c[7] * p1v);
        }
      }
    }
    orow[oo + u * od] = acc0;
    if (od == 2) orow[oo + u * od + 1] = acc1;
  }
}

// dx (bit 1) and dw (bit 4) for V = 1, paths grouped by first entry.
__global__ __launch_bounds__(256) void uvu_v1_backward_x_kernel(
    Problem pr, const float* __restrict__ x, const float* __restrict__ y,
    const float* __restrict__ w, const float* __restrict__ g, float* __restrict__ gx,
    float* __restrict__ gw, int needed) {
  const int64_t item = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (item >= pr.n * pr.C) return;
  const int64_t n = item / pr.C;
  const int u = (int)(item - n * pr.C);
  const float* xr = x + n * pr.W1;
  const float* yr = y + n * pr.W2;
  const float* gr = g + n * pr.W1;
  const float* wr = w + n * pr.wnum + u;
  float* dwr = gw + n * pr.wnum + u;
  const bool want_x = needed & 1;
  const bool want_w = (needed & 4) != 0;
  for (int i = 0; i < pr.NX; ++i) {
    int xo, xd, begin, end;
    entry_rec(pr, 1, i, xo, xd, begin, end);
    const float a0 = xr[xo + u * xd];
    const float a1 = xd == 2 ? xr[xo + u * xd + 1] : 0.f;
    float d0 = 0.f, d1 = 0.f;
    for (int q0 = begin; q0 < end; q0 += kV1Batch) {
      int pb[kV1Batch], wo[kV1Batch];
      float wv[kV1Batch], g0[kV1Batch], g1[kV1Batch], y0[kV1Batch], y1[kV1Batch];
#pragma unroll
      for (int b = 0; b < kV1Batch; ++b) {
        if (q0 + b < end) {
          pb[b] = pr.order1[q0 + b];
          const PathRec r = path_rec(pr, pb[b]);
          wo[b] = r.wo;
          wv[b] = want_x ? wr[r.wo] : 0.f;
          g0[b] = gr[r.oo + u * r.od];
          g1[b] = r.od == 2 ? gr[r.oo + u * r.od + 1] : 0.f;
          y0[b] = yr[r.yo];
          y1[b] = r.yd == 2 ? yr[r.yo + 1] : 0.f;
        }
      }
#pragma unroll
      for (int b = 0; b < kV1Batch; ++b) {
        if (q0 + b < end) {
          const float* c = pr.coef + 8 * pb[b];
          if (want_x) {
            const float p0v = wv[b] * y0[b], p1v = wv[b] * y1[b];
            d0 += g0[b] * (c[0] * p0v + c[1] * p1v) + g1[b] * (c[4] * p0v + c[5] * p1v);
            d1 += g0[b] * (c[2] * p0v + c[3] * p1v) + g1[b] * (c[6] * p0v + c[7] * p1v);
          }
          if (want_w) {
            const float r0 = a0 * (c[0] * g0[b] + c[4] * g1[b]) + a1 * (c[2] * g0[b] + c[6] * g1[b]);
            const float r1 = a0 * (c[1] * g0[b] + c[5] * g1[b]) + a1 * (c[3] * g0[b] + c[7] * g1[b]);
            __builtin_nontemporal_store(r0 * y0[b] + r1 * y1[b], dwr + wo[b]);
          }
        }
      }
    }
    if (want_x) {
      gx[n * pr.W1 + xo + u * xd] = d0;
      if (xd == 2) gx[n * pr.W1 + xo + u * xd + 1] = d1;
    }
  }
}

// dy (bit 2) for V = 1: one wave per row, lanes over u; paths grouped by
// second entry, kV1Batch at a time; lane partials summed by shuffles.
__global__ __launch_bounds__(256) void uvu_v1_backward_y_kernel(Problem pr,
                                                                const float* __restrict__ x,
                                                                const float* __restrict__ w,
                                                                const float* __restrict__ g,
                                                                float* __restrict__ gy) {
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= pr.n) return;  // whole waves leave together; no barriers below
  const float* xr = x + n * pr.W1;
  const float* gr = g + n * pr.W1;
  const float* wr = w + n * pr.wnum;
  for (int j = 0; j < pr.NY; ++j) {
    int yo, yd, begin, end;
    entry_rec(pr, 2, j, yo, yd, begin, end);
    float s0 = 0.f, s1 = 0.f;
    for (int u = lane; u < pr.C; u += 64) {
      for (int q0 = begin; q0 < end; q0 += kV1Batch) {
        int pb[kV1Batch];
        float wv[kV1Batch], a0[kV1Batch], a1[kV1Batch], g0[kV1Batch], g1[kV1Batch];
#pragma unroll
        for (int b = 0; b < kV1Batch; ++b) {
          if (q0 + b < end) {
            pb[b] = pr.order2[q0 + b];
            const PathRec r = path_rec(pr, pb[b]);
            wv[b] = wr[r.wo + u];
            a0[b] = xr[r.xo + u * r.xd];
            a1[b] = r.xd == 2 ? xr[r.xo + u * r.xd + 1] : 0.f;
            g0[b] = gr[r.oo + u * r.od];
            g1[b] = r.od == 2 ? gr[r.oo + u * r.od + 1] : 0.f;
          }
        }
#pragma unroll
        for (int b = 0; b < kV1Batch; ++b) {
          if (q0 + b < end) {
            const float* c = pr.coef + 8 * pb[b];
            const float r0 = a0[b] * (c[0] * g0[b] + c[4] * g1[b]) + a1[b] * (c[2] * g0[b] + c[6] * g1[b]);
            const float r1 = a0[b] * (c[1] * g0[b] + c[5] * g1[b]) + a1[b] * (c[3] * g0[b] + c[7] * g1[b]);
            s0 = fmaf(wv[b], r0, s0);
            s1 = fmaf(wv[b], r1, s1);
          }
        }
      }
    }
    s0 = wave_sum(s0);
    s1 = wave_sum(s1);
    if (lane == 0) {
      gy[n * pr.W2 + yo] = s0;
      if (yd == 2) gy[n * pr.W2 + yo + 1] = s1;
    }
  }
}

// Shared-weight dw partials: block (chunk of u*V, path p, split s) sums rows
// of split s; a fixed-order column sum over the splits follows.
__global__ __launch_bounds__(256) void uvu_weight_shared_kernel(
    Problem pr, const float* __restrict__ x, const float* __restrict__ y,
    const float* __restrict__ g, int64_t rows_per_split, float* __restrict__ partial) {
  const int p = blockIdx.y;
  const int64_t uv = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (uv >= (int64_t)pr.C * pr.V) return;
  const int u = (int)(uv / pr.V);
  const int v = (int)(uv - (int64_t)u * pr.V);
  const PathRec r = path_rec(pr, p);
  const float* c = pr.coef + 8 * p;
  const int64_t n0 = (int64_t)blockIdx.z * rows_per_split;
  const int64_t n1 = min(pr.n, n0 + rows_per_split);
  float acc = 0.f;
  for (int64_t n = n0; n < n1; ++n) {
    const float* xr = x + n * pr.W1;
    const float* gr = g + n * pr.W1;
    const float* yr = y + n * pr.W2;
    const float a0 = xr[r.xo + u * r.xd];
    const float a1 = r.xd == 2 ? xr[r.xo + u * r.xd + 1] : 0.f;
    const float g0 = gr[r.oo + u * r.od];
    const float g1 = r.od == 2 ? gr[r.oo + u * r.od + 1] : 0.f;
    const float r0 = a0 * (c[0] * g0 + c[4] * g1) + a1 * (c[2] * g0 + c[6] * g1);
    const float r1 = a0 * (c[1] * g0 + c[5] * g1) + a1 * (c[3] * g0 + c[7] * g1);
    const float y0 = yr[r.yo + v * r.yd];
    const float y1 = r.yd == 2 ? yr[r.yo + v * r.yd + 1] : 0.f;
    acc = fmaf(r0, y0, acc);
    acc = fmaf(r1, y1, acc);
  }
  partial[(int64_t)blockIdx.z * pr.wnum + r.wo + uv] = acc;
}

// ---- Per-row weights, V a multiple of 4 with V/4 dividing 64 ---------------
// The weight stream ([N][P][C][V], 4 bytes per (row, path, u, v)) dominates:
// one block per row reads that row's weights once, 16 bytes per lane per
// load.  Within a path, lane q covers (u = q / G, v = 4 (q % G) .. +3) with
// G = V / 4, so an aligned group of G lanes holds one u and the projection
// sum_v w[u, v] y[v, :] finishes with log2(G) xor shuffles.  Thread t
// handles q = t + 256 i for every path, so it always owns the same u values:
// the row's output (forward) and dx (backward) accumulators live in LDS with
// a single writer per element and need no atomics.  x, y and g of the row are
// staged in LDS.  Coupling slot order is [out c][in1 a][in2 b].
constexpr int kRowThreads = 256;
constexpr int kRowBatch = 8;  // weight loads in flight per thread (4: +3% step time)
using f4v = float __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float group_sum(float v, int group) {
  for (int o = 1; o < group; o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}

struct RowPath {
  PathRec r;
  float c[8];
};

__device__ __forceinline__ RowPath row_path(const Problem& pr, int p) {
  RowPath rp;
  rp.r = path_rec(pr, p);
  for (int k = 0; k < 8; ++k) rp.c[k] = pr.coef[8 * p + k];
  return rp;
}

// sum_v w[v] y[v, b] over this lane's 4 values of v.
__device__ __forceinline__ void lane_project(const f4v wv, const float* sy, int yo, int yd,
                                             int v0, float& p0, float& p1) {
  if (yd == 2) {
    const float* yv = sy + yo + 2 * v0;
    p0 = wv.x * yv[0] + wv.y * yv[2] + wv.z * yv[4] + wv.w * yv[6];
    p1 = wv.x * yv[1] + wv.y * yv[3] + wv.z * yv[5] + wv.w * yv[7];
  } else {
    const float* yv = sy + yo + v0;
    p0 = wv.x * yv[0] + wv.y * yv[1] + wv.z * yv[2] + wv.w * yv[3];
    p1 = 0.f;
  }
}

__global__ __launch_bounds__(kRowThreads) void uvu_row_forward_kernel(
    Problem pr, const float* __restrict__ x, const float* __restrict__ y,
    const float* __restrict__ w, float* __restrict__ out) {
  extern __shared__ float s_row[];
  float* sx = s_row;
  float* sy = sx + pr.W1;
  float* so = sy + pr.W2;
  const int64_t n = blockIdx.x;
  for (int i = threadIdx.x; i < pr.W1; i += kRowThreads) {
    sx[i] = x[n * pr.W1 + i];
    so[i] = 0.f;
  }
  for (int i = threadIdx.x; i < pr.W2; i += kRowThreads) sy[i] = y[n * pr.W2 + i];
  __syncthreads();
  const int G = pr.V / 4;
  const int per_path = pr.C * G;
  const f4v* wrow = reinterpret_cast<const f4v*>(w + n * pr.wnum);
  for (int p = 0; p < pr.P; ++p) {
    const RowPath rp = row_path(pr, p);
    const f4v* wp = wrow + rp.r.wo / 4;
    // kRowBatch weight loads per thread are issued before any of them is used,
    // so each wave keeps kRowBatch KiB of the weight stream in flight.
    for (int q0 = threadIdx.x; q0 < per_path; q0 += kRowBatch * kRowThreads) {
      f4v wv[kRowBatch];
#pragma unroll
      for (int k = 0; k < kRowBatch; ++k) {
        const int q = q0 + k * kRowThreads;
        if (q < per_path) wv[k] = __builtin_nontemporal_load(wp + q);
      }
#pragma unroll
      for (int k = 0; k < kRowBatch; ++k) {
        const int q = q0 + k * kRowThreads;
        if (q >= per_path) break;
        const int u = q / G, v0 = 4 * (q - u * G);
        float p0, p1;
        lane_project(wv[k], sy, rp.r.yo, rp.r.yd, v0, p0, p1);
        p0 = group_sum(p0, G);
        p1 = group_sum(p1, G);
        if (v0 == 0) {
          const float a0 = sx[rp.r.xo + u * rp.r.xd];
          const float a1 = rp.r.xd == 2 ? sx[rp.r.xo + u * rp.r.xd + 1] : 0.f;
          float* o = so + rp.r.oo + u * rp.r.od;
          const float* c = rp.c;
          o[0] += a0 * (c[0] * p0 + c[1] * p1) + a1 * (c[2] * p0 + c[3] * p1);
          if (rp.r.od == 2) o[1] += a0 * (c[4] * p0 + c[5] * p1) + a1 * (c[6] * p0 + c[7] * p1);
        }
      }
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < pr.W1; i += kRowThreads) out[n * pr.W1 + i] = so[i];
}

// dx (bit 1), dy (bit 2) and per-row dw (bit 4) in one pass over the row's
// weights.  Paths are visited grouped by second-input entry (second_order),
// so each lane keeps its dy partials for its 4 values of v in registers for
// one entry at a time; they are summed over u by shuffles (lanes with equal
// q % G) and over the 4 waves in LDS, in a fixed order.
__global__ __launch_bounds__(kRowThreads) void uvu_row_backward_kernel(
    Problem pr, const float* __restrict__ x, const float* __restrict__ y,
    const float* __restrict__ w, const float* __restrict__ g, float* __restrict__ gx,
    float* __restrict__ gy, float* __restrict__ gw, int needed) {
  extern __shared__ float s_row[];
  float* sx = s_row;
  float* sg = sx + pr.W1;
  float* sdx = sg + pr.W1;
  float* sy = sdx + pr.W1;
  float* sdy = sy + pr.W2;  // [4 waves][W2]
  const int64_t n = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int i = threadIdx.x; i < pr.W1; i += kRowThreads) {
    sx[i] = x[n * pr.W1 + i];
    sg[i] = g[n * pr.W1 + i];
    sdx[i] = 0.f;
  }
  for (int i = threadIdx.x; i < pr.W2; i += kRowThreads) sy[i] = y[n * pr.W2 + i];
  __syncthreads();
  const bool want_x = needed & 1, want_y = (needed & 2) != 0, want_w = (needed & 4) != 0;
  const bool read_w = want_x || want_y;
  const int G = pr.V / 4;
  const int per_path = pr.C * G;
  const f4v* wrow = reinterpret_cast<const f4v*>(w + n * pr.wnum);
  f4v* dwrow = reinterpret_cast<f4v*>(gw + n * pr.wnum);
  for (int j = 0; j < pr.NY; ++j) {
    int yo, yd, begin, end;
    entry_rec(pr, 2, j, yo, yd, begin, end);
    float dy[4][2] = {{0.f, 0.f}, {0.f, 0.f}, {0.f, 0.f}, {0.f, 0.f}};
    for (int k = begin; k < end; ++k) {
      const RowPath rp = row_path(pr, pr.order2[k]);
      const float* c = rp.c;
      const f4v* wp = wrow + rp.r.wo / 4;
      for (int q0 = threadIdx.x; q0 < per_path; q0 += kRowBatch * kRowThreads) {
        f4v wb[kRowBatch];
        if (read_w) {
#pragma unroll
          for (int b = 0; b < kRowBatch; ++b) {
            const int q = q0 + b * kRowThreads;
            if (q < per_path) wb[b] = __builtin_nontemporal_load(wp + q);
          }
        }
#pragma unroll
        for (int b = 0; b < kRowBatch; ++b) {
          const int q = q0 + b * kRowThreads;
          if (q >= per_path) break;
          const int u = q / G, v0 = 4 * (q - u * G);
          const float a0 = sx[rp.r.xo + u * rp.r.xd];
          const float a1 = rp.r.xd == 2 ? sx[rp.r.xo + u * rp.r.xd + 1] : 0.f;
          const float g0 = sg[rp.r.oo + u * rp.r.od];
          const float g1 = rp.r.od == 2 ? sg[rp.r.oo + u * rp.r.od + 1] : 0.f;
          // r_b = d out / d proj_b for this (row, path, u).
          const float r0 = a0 * (c[0] * g0 + c[4] * g1) + a1 * (c[2] * g0 + c[6] * g1);
          const float r1 = a0 * (c[1] * g0 + c[5] * g1) + a1 * (c[3] * g0 + c[7] * g1);
          const float* yv = sy + yo + yd * v0;
          if (want_w) {
            f4v d;
            if (yd == 2) {
              d.x = r0 * yv[0] + r1 * yv[1];
              d.y = r0 * yv[2] + r1 * yv[3];
              d.z = r0 * yv[4] + r1 * yv[5];
              d.w = r0 * yv[6] + r1 * yv[7];
            } else {
              d.x = r0 * yv[0];
              d.y = r0 * yv[1];
              d.z = r0 * yv[2];
              d.w = r0 * yv[3];
            }
            __builtin_nontemporal_store(d, dwrow + rp.r.wo / 4 + q);
          }
          if (read_w) {
            const f4v wv = wb[b];
            dy[0][0] += wv.x * r0; dy[0][1] += wv.x * r1;
            dy[1][0] += wv.y * r0; dy[1][1] += wv.y * r1;
            dy[2][0] += wv.z * r0; dy[2][1] += wv.z * r1;
            dy[3][0] += wv.w * r0; dy[3][1] += wv.w * r1;
            if (want_x) {
              float p0, p1;
              lane_project(wv, sy, yo, yd, v0, p0, p1);
              p0 = group_sum(p0, G);
              p1 = group_sum(p1, G);
              if (v0 == 0) {
                float* d = sdx + rp.r.xo + u * rp.r.xd;
                d[0] += g0 * (c[0] * p0 + c[1] * p1) + g1 * (c[4] * p0 + c[5] * p1);
                if (rp.r.xd == 2) d[1] += g0 * (c[2] * p0 + c[3] * p1) + g1 * (c[6] * p0 + c[7] * p1);
              }
            }
          }
        }
      }
    }
    if (want_y) {
      // Sum over the lanes of this wave that share v0 (equal lane % G).
      for (int o = G; o < 64; o <<= 1)
        for (int v = 0; v < 4; ++v) {
          dy[v][0] += __shfl_xor(dy[v][0], o, 64);
          dy[v][1] += __shfl_xor(dy[v][1], o, 64);
        }
      if (lane < G) {
        for (int v = 0; v < 4; ++v) {
          sdy[wave * pr.W2 + yo + yd * (4 * lane + v)] = dy[v][0];
          if (yd == 2) sdy[wave * pr.W2 + yo + yd * (4 * lane + v) + 1] = dy[v][1];
        }
      }
    }
  }
  __syncthreads();
  if (want_x)
    for (int i = threadIdx.x; i < pr.W1; i += kRowThreads) gx[n * pr.W1 + i] = sdx[i];
  if (want_y)
    for (int i = threadIdx.x; i < pr.W2; i += kRowThreads)
      gy[n * pr.W2 + i] = (sdy[i] + sdy[pr.W2 + i]) + (sdy[2 * pr.W2 + i] + sdy[3 * pr.W2 + i]);
}

// ---- Per-row weights, 3 <= V <= 7 not a multiple of 4: one wave per row ----
// The row-streaming kernels above need V = 4 G.  Here a wave owns a row: its
// x, y (and g) and the out / dx accumulators live in LDS, and lane l owns the
// channels l, l + 64, ... for every path (one writer per element), so its V
// weights of a channel are one contiguous run and the wave's loads of a path
// one coalesced stream.  Compiled per V; paths are taken wave_batch<V>() at
// a time (larger batches measured slower: the accumulators are read and
// written in LDS per path).  dy is summed per second-input entry over the
// wave's lanes by shuffles, in a fixed order, reading x and g once for all V
// copies (the generic dy kernel reads them once per copy).  Rows per block =
// blockDim.x / 64; every wave reaches every barrier.  V = 1 and 2 measured
// slower here than with the generic kernels and keep those.
constexpr int kWaveMaxV = 8;

template <int V>
constexpr int wave_batch() {
  return 4;
}

__device__ __forceinline__ float wave_sum_all(float v) {
  for (int s = 32; s > 0; s >>= 1) v += __shfl_xor(v, s, 64);
  return v;
}

template <int V>
__global__ __launch_bounds__(256) void uvu_wave_forward_kernel(Problem pr,
                                                               const float* __restrict__ x,
                                                               const float* __restrict__ y,
                                                               const float* __restrict__ w,
                                                               float* __restrict__ out) {
  extern __shared__ float s_wave[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t n = (int64_t)blockIdx.x * (blockDim.x >> 6) + wave;
  const bool active = n < pr.n;
  const int per = 2 * pr.W1 + pr.W2;
  float* sx = s_wave + wave * per;
  float* so = sx + pr.W1;
  float* sy = so + pr.W1;
  if (active) {
    for (int i = lane; i < pr.W1; i += 64) {
      sx[i] = x[n * pr.W1 + i];
      so[i] = 0.f;
    }
    for (int i = lane; i < pr.W2; i += 64) sy[i] = y[n * pr.W2 + i];
  }
  __syncthreads();
  if (active) {
    constexpr int B = wave_batch<V>();
    const float* wr = w + n * pr.wnum;
    for (int u = lane; u < pr.C; u += 64) {
      for (int p0 = 0; p0 < pr.P; p0 += B) {
        float wv[B][V];
#pragma unroll
        for (int b = 0; b < B; ++b) {
          const int p = p0 + b < pr.P ? p0 + b : pr.P - 1;
          const float* src = wr + pr.info[7 * p + 6] + (int64_t)u * V;
#pragma unroll
          for (int v = 0; v < V; ++v) wv[b][v] = src[v];
        }
#pragma unroll
        for (int b = 0; b < B; ++b) {
          const int p = p0 + b;
          if (p >= pr.P) break;
          const PathRec r = path_rec(pr, p);
          const float* c = pr.coef + 8 * p;
          float p0v = 0.f, p1v = 0.f;
#pragma unroll
          for (int v = 0; v < V; ++v) {
            p0v = fmaf(wv[b][v], sy[r.yo + v * r.yd], p0v);
            if (r.yd == 2) p1v = fmaf(wv[b][v], sy[r.yo + v * r.yd + 1], p1v);
          }
          const float a0 = sx[r.xo + u * r.xd];
          const float a1 = r.xd == 2 ? sx[r.xo + u * r.xd + 1] : 0.f;
          float* o = so + r.oo + u * r.od;
          o[0] += a0 * (c[0] * p0v + c[1] * p1v) + a1 * (c[2] * p0v + c[3] * p1v);
          if (r.od == 2) o[1] += a0 * (c[4] * p0v + c[5] * p1v) + a1 * (c[6] * p0v + c[7] * p1v);
        }
      }
    }
  }
  __syncthreads();
  if (active)
    for (int i = lane; i < pr.W1; i += 64) out[n * pr.W1 + i] = so[i];
}

// dx (bit 1), dy (bit 2) and per-row dw (bit 4), paths grouped by
// second-input entry (second_order).
template <int V>
__global__ __launch_bounds__(256) void uvu_wave_backward_kernel(
    Problem pr, const float* __restrict__ x, const float* __restrict__ y,
    const float* __restrict__ w, const float* __restrict__ g, float* __restrict__ gx,
    float* __restrict__ gy, float* __restrict__ gw, int needed) {
  extern __shared__ float s_wave[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t n = (int64_t)blockIdx.x * (blockDim.x >> 6) + wave;
  const bool active = n < pr.n;
  const int per = 3 * pr.W1 + 2 * pr.W2;
  float* sx = s_wave + wave * per;
  float* sg = sx + pr.W1;
  float* sdx = sg + pr.W1;
  float* sy = sdx + pr.W1;
  float* sdy = sy + pr.W2;
  if (active) {
    for (int i = lane; i < pr.W1; i += 64) {
      sx[i] = x[n * pr.W1 + i];
      sg[i] = g[n * pr.W1 + i];
      sdx[i] = 0.f;
    }
    for (int i = lane; i < pr.W2; i += 64) sy[i] = y[n * pr.W2 + i];
  }
  __syncthreads();
  const bool want_x = needed & 1, want_y = (needed & 2) != 0, want_w = (needed & 4) != 0;
  const bool read_w = want_x || want_y;
  if (active) {
    constexpr int B = wave_batch<V>();
    const float* wr = w + n * pr.wnum;
    float* dwr = want_w ? gw + n * pr.wnum : nullptr;
    for (int j = 0; j < pr.NY; ++j) {
      int yo, yd, begin, end;
      entry_rec(pr, 2, j, yo, yd, begin, end);
      float dy[V][2];
#pragma unroll
      for (int v = 0; v < V; ++v) dy[v][0] = dy[v][1] = 0.f;
      for (int u = lane; u < pr.C; u += 64) {
        for (int k0 = begin; k0 < end; k0 += B) {
          float wv[B][V];
          if (read_w) {
#pragma unroll
            for (int b = 0; b < B; ++b) {
              const int p = pr.order2[k0 + b < end ? k0 + b : end - 1];
              const float* src = wr + pr.info[7 * p + 6] + (int64_t)u * V;
#pragma unroll
              for (int v = 0; v < V; ++v) wv[b][v] = src[v];
            }
          }
#pragma unroll
          for (int b = 0; b < B; ++b) {
            if (k0 + b >= end) break;
            const int p = pr.order2[k0 + b];
            const PathRec r = path_rec(pr, p);
            const float* c = pr.coef + 8 * p;
            const float a0 = sx[r.xo + u * r.xd];
            const float a1 = r.xd == 2 ? sx[r.xo + u * r.xd + 1] : 0.f;
            const float g0 = sg[r.oo + u * r.od];
            const float g1 = r.od == 2 ? sg[r.oo + u * r.od + 1] : 0.f;
            // r_b = d out / d proj_b for this (row, path, u).
            const float r0 = a0 * (c[0] * g0 + c[4] * g1) + a1 * (c[2] * g0 + c[6] * g1);
            const float r1 = a0 * (c[1] * g0 + c[5] * g1) + a1 * (c[3] * g0 + c[7] * g1);
            if (want_w) {
              float* dst = dwr + r.wo + (int64_t)u * V;
#pragma unroll
              for (int v = 0; v < V; ++v)
                dst[v] = yd == 2 ? r0 * sy[yo + 2 * v] + r1 * sy[yo + 2 * v + 1] : r0 * sy[yo + v];
            }
            if (read_w) {
              float p0v = 0.f, p1v = 0.f;
#pragma unroll
              for (int v = 0; v < V; ++v) {
                dy[v][0] = fmaf(wv[b][v], r0, dy[v][0]);
                dy[v][1] = fmaf(wv[b][v], r1, dy[v][1]);
                p0v = fmaf(wv[b][v], sy[yo + v * yd], p0v);
                if (yd == 2) p1v = fmaf(wv[b][v], sy[yo + v * yd + 1], p1v);
              }
              if (want_x) {
                float* d = sdx + r.xo + u * r.xd;
                d[0] += g0 * (c[0] * p0v + c[1] * p1v) + g1 * (c[4] * p0v + c[5] * p1v);
                if (r.xd == 2) d[1] += g0 * (c[2] * p0v + c[3] * p1v) + g1 * (c[6] * p0v + c[7] * p1v);
              }
            }
          }
        }
      }
      if (want_y) {
#pragma unroll
        for (int v = 0; v < V; ++v) {
          const float s0 = wave_sum_all(dy[v][0]);
          const float s1 = wave_sum_all(dy[v][1]);
          if (lane == 0) {
            sdy[yo + v * yd] = s0;
            if (yd == 2) sdy[yo + v * yd + 1] = s1;
          }
        }
      }
    }
  }
  __syncthreads();
  if (active) {
    if (want_x)
      for (int i = lane; i < pr.W1; i += 64) gx[n * pr.W1 + i] = sdx[i];
    if (want_y)
      for (int i = lane; i < pr.W2; i += 64) gy[n * pr.W2 + i] = sdy[i];
  }
}

__global__ __launch_bounds__(256) void uvu_column_sum_kernel(const float* __restrict__ in,
                                                             int64_t rows, int64_t cols,
                                                             float* __restrict__ out) {
  const int64_t col = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (col >= cols) return;
  float s = 0.f;
  for (int64_t r = 0; r < rows; ++r) s += in[r * cols + col];
  out[col] = s;
}

__global__ __launch_bounds__(256) void uvu_fill_kernel(float* __restrict__ out, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = 0.f;
}

int fail(int status, const char* message) {
  o2mi_error_slot() = message;
  return status;
}

bool to_problem(const o2mi_uvu_problem* in, Problem* pr) {
  if (!in || in->n_rows < 0 || in->channels < 1 || in->channels_in2 < 1 || in->n_paths < 0 ||
      in->n_out_entries < 1 || in->n_in2_entries < 1 || in->width1 < 1 || in->width2 < 1)
    return false;
  if (!in->info || (in->n_paths > 0 && !in->coefficients) || !in->first_order ||
      !in->second_order)
    return false;
  pr->n = in->n_rows;
  pr->C = in->channels;
  pr->V = in->channels_in2;
  pr->P = in->n_paths;
  pr->NO = in->n_out_entries;
  pr->NX = in->n_out_entries;
  pr->NY = in->n_in2_entries;
  pr->W1 = in->width1;
  pr->W2 = in->width2;
  pr->wnum = (int64_t)in->n_paths * in->channels * in->channels_in2;
  pr->shared = in->shared_weights != 0;
  pr->info = in->info;
  pr->coef = in->coefficients;
  pr->order1 = in->first_order;
  pr->order2 = in->second_order;
  return true;
}

int64_t shared_splits(const Problem& pr) {
  const int64_t chunks = std::max<int64_t>(1, (int64_t)pr.P * ((pr.C * pr.V + 255) / 256));
  int64_t splits = std::max<int64_t>(1, 4096 / chunks);
  splits = std::min<int64_t>(splits, 64);
  return std::max<int64_t>(1, std::min<int64_t>(splits, pr.n));
}

unsigned blocks_for(int64_t items) { return (unsigned)((items + 255) / 256); }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// LDS bytes of the per-row kernels, or 0 when they do not apply: per-row
// weights, V = 4 G with G dividing 64, 16-byte aligned weight rows and row
// state within the default 64 KB of dynamic LDS.
size_t row_kernel_lds(const Problem& pr, bool backward, const void* w, const void* gw) {
  if (pr.shared || pr.V % 4 != 0 || 64 % (pr.V / 4) != 0 || pr.n > 0x7fffffff) return 0;
  if ((w && !aligned16(w)) || (gw && !aligned16(gw))) return 0;
  const size_t floats = backward ? (size_t)3 * pr.W1 + (size_t)5 * pr.W2
                                 : (size_t)2 * pr.W1 + (size_t)pr.W2;
  const size_t bytes = floats * sizeof(float);
  return bytes <= 65536 ? bytes : 0;
}

// Rows per block of the wave-per-row kernels (per-row weights, 3 <= V <= 7
// not a multiple of 4), or 0 when they do not apply: as many rows as the
// default 64 KB of dynamic LDS holds, up to 4.
int wave_kernel_rows(const Problem& pr, bool backward) {
  if (pr.shared || pr.V < 3 || pr.V > kWaveMaxV || pr.V % 4 == 0 || pr.n > 0x7fffffff) return 0;
  const size_t floats = backward ? (size_t)3 * pr.W1 + (size_t)2 * pr.W2
                                 : (size_t)2 * pr.W1 + (size_t)pr.W2;
  const size_t rows = 65536 / (floats * sizeof(float));
  return (int)std::min<size_t>(rows, 4);
}

}  // namespace uvu
}  // namespace o2mi

using namespace o2mi::uvu;

extern "C" {

int o2mi_uvu_forward_f32(const o2mi_uvu_problem* problem, const float* x, const float* y,
                         const float* w, float* out, void* stream) {
  Problem pr;
  if (!to_problem(problem, &pr)) return fail(O2MI_ERR_INVALID_ARGUMENT, "invalid uvu problem");
  if (pr.n == 0) return O2MI_OK;
  if (!x || !y || !w || !out) return fail(O2MI_ERR_INVALID_ARGUMENT, "NULL tensor pointer");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (const size_t lds = row_kernel_lds(pr, false, w, nullptr)) {
    O2miTimed timed;
    const bool timing = o2mi_timing_begin(s, &timed, O2MI_TIMED_UVU_FORWARD);
    hipLaunchKernelGGL(uvu_row_forward_kernel, dim3((unsigned)pr.n), dim3(kRowThreads), lds, s,
                       pr, x, y, w, out);
    if (timing) o2mi_timing_end(s, &timed);
    return hipGetLastError() == hipSuccess ? O2MI_OK
                                           : fail(O2MI_ERR_HIP, "uvu forward launch failed");
  }
  if (const int rows = wave_kernel_rows(pr, false)) {
    O2miTimed timed;
    const bool timing = o2mi_timing_begin(s, &timed, O2MI_TIMED_UVU_FORWARD);
    const size_t lds = (size_t)rows * (2 * pr.W1 + pr.W2) * sizeof(float);
    const dim3 grid((unsigned)((pr.n + rows - 1) / rows)), block(64 * rows);
    switch (pr.V) {
      case 3: hipLaunchKernelGGL(uvu_wave_forward_kernel<3>, grid, block, lds, s, pr, x, y, w, out); break;
      case 5: hipLaunchKernelGGL(uvu_wave_forward_kernel<5>, grid, block, lds, s, pr, x, y, w, out); break;
      case 6: hipLaunchKernelGGL(uvu_wave_forward_kernel<6>, grid, block, lds, s, pr, x, y, w, out); break;
      default: hipLaunchKernelGGL(uvu_wave_forward_kernel<7>, grid, block, lds, s, pr, x, y, w, out); break;
    }
    if (timing) o2mi_timing_end(s, &timed);
    return hipGetLastError() == hipSuccess ? O2MI_OK
                                           : fail(O2MI_ERR_HIP, "uvu forward launch failed");
  }
  if (pr.V == 1 && !pr.shared)
    hipLaunchKernelGGL(uvu_v1_forward_kernel, dim3(blocks_for(pr.n * pr.C)), dim3(256), 0, s, pr,
                       x, y, w, out);
  else
    hipLaunchKernelGGL(uvu_forward_kernel, dim3(blocks_for(pr.n * pr.C)), dim3(256), 0, s, pr, x,
                       y, w, out);
  return hipGetLastError() == hipSuccess ? O2MI_OK
                                         : fail(O2MI_ERR_HIP, "uvu forward launch failed");
}

size_t o2mi_uvu_backward_workspace_bytes(const o2mi_uvu_problem* problem, int needed) {
  Problem pr;
  if (!to_problem(problem, &pr) || pr.n == 0 || !(needed & 4) || !pr.shared) return 0;
  return (size_t)shared_splits(pr) * (size_t)pr.wnum * sizeof(float);
}

int o2mi_uvu_backward_f32(const o2mi_uvu_problem* problem, const float* x, const float* y,
                          const float* w, const float* g, float* gx, float* gy, float* gw,
                          int needed, void* workspace, size_t workspace_bytes, void* stream) {
  Problem pr;
  if (!to_problem(problem, &pr)) return fail(O2MI_ERR_INVALID_ARGUMENT, "invalid uvu problem");
  if (needed & ~7) return fail(O2MI_ERR_INVALID_ARGUMENT, "needed must be a mask of 1, 2, 4");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (pr.n == 0) {
    // Empty inputs: shared dw is zero; the other adjoints (and per-row dw) are empty.
    if ((needed & 4) && pr.shared && pr.wnum > 0) {
      if (!gw) return fail(O2MI_ERR_INVALID_ARGUMENT, "NULL gw");
      hipLaunchKernelGGL(uvu_fill_kernel, dim3(blocks_for(pr.wnum)), dim3(256), 0, s, gw,
                         pr.wnum);
    }
    return hipGetLastError() == hipSuccess ? O2MI_OK : fail(O2MI_ERR_HIP, "uvu fill failed");
  }
  if (!x || !y || !w || !g) return fail(O2MI_ERR_INVALID_ARGUMENT, "NULL input pointer");
  if (((needed & 1) && !gx) || ((needed & 2) && !gy) || ((needed & 4) && !gw))
    return fail(O2MI_ERR_INVALID_ARGUMENT, "NULL output for a requested gradient");
  if (const size_t lds = row_kernel_lds(pr, true, w, (needed & 4) ? gw : nullptr)) {
    O2miTimed timed;
    const bool timing = o2mi_timing_begin(s, &timed, O2MI_TIMED_UVU_BACKWARD);
    hipLaunchKernelGGL(uvu_row_backward_kernel, dim3((unsigned)pr.n), dim3(kRowThreads), lds, s,
                       pr, x, y, w, g, gx, gy, gw, needed);
    if (timing) o2mi_timing_end(s, &timed);
    return hipGetLastError() == hipSuccess ? O2MI_OK
                                           : fail(O2MI_ERR_HIP, "uvu backward launch failed");
  }
  if (const int rows = wave_kernel_rows(pr, true)) {
    O2miTimed timed;
    const bool timing = o2mi_timing_begin(s, &timed, O2MI_TIMED_UVU_BACKWARD);
    const size_t lds = (size_t)rows * (3 * pr.W1 + 2 * pr.W2) * sizeof(float);
    const dim3 grid((unsigned)((pr.n + rows - 1) / rows)), block(64 * rows);
    switch (pr.V) {
      case 3: hipLaunchKernelGGL(uvu_wave_backward_kernel<3>, grid, block, lds, s, pr, x, y, w, g, gx, gy, gw, needed); break;
      case 5: hipLaunchKernelGGL(uvu_wave_backward_kernel<5>, grid, block, lds, s, pr, x, y, w, g, gx, gy, gw, needed); break;
      case 6: hipLaunchKernelGGL(uvu_wave_backward_kernel<6>, grid, block, lds, s, pr, x, y, w, g, gx, gy, gw, needed); break;
      default: hipLaunchKernelGGL(uvu_wave_backward_kernel<7>, grid, block, lds, s, pr, x, y, w, g, gx, gy, gw, needed); break;
    }
    if (timing) o2mi_timing_end(s, &timed);
    return hipGetLastError() == hipSuccess ? O2MI_OK
                                           : fail(O2MI_ERR_HIP, "uvu backward launch failed");
  }
  const bool v1 = pr.V == 1 && !pr.shared;
  if ((needed & 1) || ((needed & 4) && !pr.shared)) {
    if (v1)
      hipLaunchKernelGGL(uvu_v1_backward_x_kernel, dim3(blocks_for(pr.n * pr.C)), dim3(256), 0, s,
                         pr, x, y, w, g, gx, gw, needed);
    else
      hipLaunchKernelGGL(uvu_backward_x_kernel, dim3(blocks_for(pr.n * pr.C)), dim3(256), 0, s,
                         pr, x, y, w, g, gx, gw, needed);
  }
  if (needed & 2) {
    if (v1)
      hipLaunchKernelGGL(uvu_v1_backward_y_kernel, dim3((unsigned)((pr.n + 3) / 4)), dim3(256), 0,
                         s, pr, x, w, g, gy);
    else
      hipLaunchKernelGGL(uvu_backward_y_kernel, dim3((unsigned)((pr.n + 3) / 4)), dim3(256), 0, s,
                         pr, x, w, g, gy);
  }
  if ((needed & 4) && pr.shared && pr.P > 0) {
    const int64_t splits = shared_splits(pr);
    if (!workspace || workspace_bytes < (size_t)splits * pr.wnum * sizeof(float))
      return fail(O2MI_ERR_WORKSPACE, "workspace smaller than o2mi_uvu_backward_workspace_bytes");
    float* partial = static_cast<float*>(workspace);
    const int64_t per_split = (pr.n + splits - 1) / splits;
    dim3 grid(blocks_for((int64_t)pr.C * pr.V), (unsigned)pr.P, (unsigned)splits);
    hipLaunchKernelGGL(uvu_weight_shared_kernel, grid, dim3(256), 0, s, pr, x, y, g, per_split,
                       partial);
    hipLaunchKernelGGL(uvu_column_sum_kernel, dim3(blocks_for(pr.wnum)), dim3(256), 0, s, partial,
                       splits, pr.wnum, gw);
  }
  return hipGetLastError() == hipSuccess ? O2MI_OK
                                         : fail(O2MI_ERR_HIP, "uvu backward launch failed");
}

}  // extern "C"
