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
  if ((needed & 1) || ((needed & 4) && !pr.shared)) {
    hipLaunchKernelGGL(uvu_backward_x_kernel, dim3(blocks_for(pr.n * pr.C)), dim3(256), 0, s, pr,
                       x, y, w, g, gx, gw, needed);
  }
  if (needed & 2) {
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
