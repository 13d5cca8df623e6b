// The uvu product with shared weights and 2 <= V <= 8 copies of the second
// input, for the structures of the fused radial kernels (uvu_fused.py:7-160
// and uvu_triton.py:181-232 are the reference's kernels for this mode):
//
//   Z_c[e, u]   = sum_v w[p, u, v] y[e, v, c]        (the v projection)
//   out[e,u,k] += sum_slots coef x[e, u, ia] Z_ib[e, u]
//
// The projection has the shape of the radial affine W[e, u] = sum_h hidden[e,
// h] alpha[h, p, u] with K = V instead of H, so it runs on the fp32 matrix
// cores in the same lane layout: lane (g, j) holds channels u0+4g .. +3 of
// edge j.  The weights [P][C][V] are streamed through LDS per channel tile in
// double-buffered chunks of kVChunk paths, zero-padded to kVK = 8
// copies; the lane's copies 2g, 2g+1 of every second-input component of its
// edge are the B operands (zero past V).  The input adjoints form dy[e, v, c]
// = sum_u gz_c[e, u] w[p, u, v] as matrix products over the channels, two
// components per 16-row accumulator tile, and dw[p, u, v] = sum_e gz_c[e, u]
// y[e, v, c] as matrix products over the edges (rows = channels, columns =
// copies).  gz_c = sum_slots coef x g is the adjoint of Z_c.
#pragma once

#include "o2mi_radial.hpp"
#include "o2mi_radial_streamed.hpp"

namespace o2mi {
namespace radial {

constexpr int kVK = 8;  // copies of the second input a kernel covers (zero-padded)

// Paths per staged weight chunk: a path costs only 2 MFMAs per second-input
// component here, so chunks are deeper than the radial kernels' to amortise
// the chunk barrier.
constexpr int kVChunk = 32;

// Entry of the V = 1 second-input component c.
template <class Plan>
constexpr int y_entry_of(int c) {
  for (int e = 0; e < Plan::kEntries2; ++e)
    if (c >= Plan::e2[e].base && c < Plan::e2[e].base + Plan::e2[e].dim) return e;
  return 0;
}

// Offset of (copy v, component c) in a row of the second input with V copies:
// entry e starts at V * e.off and holds [V][e.dim] (uvu_o2.py:27-41).
template <class Plan, int c>
__device__ __forceinline__ int y_offset(int V, int v) {
  constexpr REntry E = Plan::e2[y_entry_of<Plan>(c)];
  return V * E.off + v * E.dim + (c - E.base);
}

// Weights of kVChunk consecutive paths of an order for channel tile u0, as
// [slot][16 channels][kVK] (copies >= V zero): global loads in registers.
template <class Plan, int NT>
struct VChunk {
  static constexpr int kFloats = kVChunk * 16 * kVK;
  static constexpr int kPer = (kFloats + NT - 1) / NT;
  static_assert(NT % (16 * kVK) == 0, "a pass covers whole path slots");
  float w[kPer];
};

template <class Plan, int NT, bool kBwd, int c>
__device__ __forceinline__ void vchunk_fetch(VChunk<Plan, NT>& pf, const Args& a, int u0) {
  using S = VChunk<Plan, NT>;
  constexpr int PC = kVChunk;
  constexpr int kSlotsPerPass = NT / (16 * kVK);
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));  // keep the slot -> path selects inside the channel loop
  static_for<S::kPer>([&](auto kc) __attribute__((always_inline)) {
    constexpr int k = decltype(kc)::value;
    const int idx = tid + k * NT;
    const int sub = tid / (16 * kVK);
    const int ch = (idx / kVK) & 15, v = idx & (kVK - 1);
    int path = -1;
    static_for<kSlotsPerPass>([&](auto sc) __attribute__((always_inline)) {
      constexpr int slot = k * kSlotsPerPass + decltype(sc)::value;
      constexpr int pos = c * PC + slot;
      if constexpr (slot < PC && pos < Plan::kPaths)
        if (sub == decltype(sc)::value) path = path_at<Plan, kBwd>(pos);
    });
    float val = 0.f;
    if (path >= 0 && v < a.V) val = a.alpha[((int64_t)path * a.C + u0 + ch) * a.V + v];
    pf.w[k] = val;
  });
}

template <class Plan, int NT>
__device__ __forceinline__ void vchunk_commit(const VChunk<Plan, NT>& pf, float* buf) {
  using S = VChunk<Plan, NT>;
  static_for<S::kPer>([&](auto kc) __attribute__((always_inline)) {
    constexpr int k = decltype(kc)::value;
    const int idx = threadIdx.x + k * NT;
    if (idx < S::kFloats) buf[idx] = pf.w[k];
  });
}

// B operands of the projection for every second-input component of edge j:
// yb[c][t] = y[j, copy 2g + t, component c], zero for copies >= V.
template <class Plan>
__device__ __forceinline__ void load_yb(__amdgpu_buffer_rsrc_t ry, const Args& a, int g, int j,
                                        float (&yb)[Plan::kComps2][2]) {
  static_for<Plan::kComps2>([&](auto cc) __attribute__((always_inline)) {
    constexpr int c = decltype(cc)::value;
    static_for<2>([&](auto tc) __attribute__((always_inline)) {
      constexpr int t = decltype(tc)::value;
      const int v = 2 * g + t;
      yb[c][t] = ld1(ry, v < a.V ? (uint32_t)(j * a.W2 + y_offset<Plan, c>(a.V, v)) * 4u : kIdle);
    });
  });
}

template <class Plan>
struct VLayout {
  static constexpr int kCoefPad = (Plan::kPaths * 8 + 3) / 4 * 4;
  static constexpr int kChunks = (Plan::kPaths + kVChunk - 1) / kVChunk;
  static constexpr int kBufFloats = kVChunk * 16 * kVK;
  static constexpr int kFloats = kCoefPad + 2 * kBufFloats;
};

// Grid (edge blocks of 128, channel splits); Args::alpha = w [P][C][V].
template <class Plan>
__global__ __launch_bounds__(64 * kSFwdWaves, 1) void uvu_vshared_forward_kernel(Args a,
                                                                               float* out) {
  constexpr int NT = 64 * kSFwdWaves;
  using L = VLayout<Plan>;
  constexpr int P = Plan::kPaths;
  constexpr int NC = Plan::kComps1;
  constexpr int PC = kVChunk;
  constexpr int NCH = L::kChunks;
  __shared__ __attribute__((aligned(16))) float s_mem[L::kFloats];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
  const int g = lane >> 4, j = lane & 15;
  const int64_t e0 = ((int64_t)blockIdx.x * (NT / 64) + wave) * kEdgesPerWave;
  const int64_t rows = a.n - e0 < kEdgesPerWave ? a.n - e0 : kEdgesPerWave;
  const auto rx = rows_rsrc(a.x, e0, a.W1, rows);
  const auto ry = rows_rsrc(a.y, e0, a.W2, rows);
  const auto ro = rows_rsrc(out, e0, a.W1, rows);
  const uint32_t xrow = (uint32_t)(j * a.W1) * 4u;

  for (int idx = threadIdx.x; idx < P * 8; idx += NT) s_mem[idx] = a.coef[idx];
  float yb[Plan::kComps2][2];
  load_yb<Plan>(ry, a, g, j, yb);

  const int u_begin = blockIdx.y * a.tile_span;
  const int u_end = u_begin + a.tile_span < a.C ? u_begin + a.tile_span : a.C;
  VChunk<Plan, NT> pf;
  vchunk_fetch<Plan, NT, false, 0>(pf, a, u_begin);
  vchunk_commit<Plan, NT>(pf, s_mem + L::kCoefPad);
  int parity = 0;  // LDS buffer of the current chunk
  for (int u0 = u_begin; u0 < u_end; u0 += 16) {
    __syncthreads();
    const int u = u0 + 4 * g;
    float xv[4 * NC];
    load_row<Plan>(rx, xrow, a.C, u, xv);
    static_for<Plan::kEntries1>([&](auto ec) __attribute__((always_inline)) {
      constexpr int e = decltype(ec)::value;
      constexpr REntry O = Plan::e1[e];
      if constexpr (!entry_used<Plan, true>(e)) store_zero_entry<O.dim>(ro, xrow, O.off * a.C, u);
    });
    float ov[8];
    static_for<NCH>([&](auto cc) __attribute__((always_inline)) {
      constexpr int c = decltype(cc)::value;
      if constexpr (c + 1 < NCH) {
        vchunk_fetch<Plan, NT, false, c + 1>(pf, a, u0);
      } else {
        if (u0 + 16 < u_end) vchunk_fetch<Plan, NT, false, 0>(pf, a, u0 + 16);
      }
      const int buf = L::kCoefPad + parity * L::kBufFloats;
      int coef_off = 0, w_off = buf + j * kVK + 2 * g;
      asm volatile("" : "+v"(coef_off), "+v"(w_off));
      const float* cf = s_mem + coef_off;
      static_for<(P - c * PC < PC ? P - c * PC : PC)>([&](auto sc) __attribute__((always_inline)) {
        constexpr int slot = decltype(sc)::value;
        constexpr int q = c * PC + slot;
        constexpr int p = Plan::fwd[q];
        constexpr RPath ps = Plan::paths[p];
        constexpr REntry X = Plan::e1[ps.i];
        constexpr REntry Y = Plan::e2[ps.j];
        constexpr REntry O = Plan::e1[ps.k];
        constexpr bool first = q == 0 || Plan::paths[Plan::fwd[q == 0 ? 0 : q - 1]].k != ps.k;
        constexpr bool last = q == P - 1 || Plan::paths[Plan::fwd[q == P - 1 ? q : q + 1]].k != ps.k;
        if constexpr (first) static_for<8>([&](auto ic) __attribute__((always_inline)) { ov[decltype(ic)::value] = 0.f; });
        const float* wl = s_mem + w_off + slot * 16 * kVK;
        const float w0 = wl[0], w1 = wl[1];
        f4 z[2];
        static_for<Y.dim>([&](auto bc) __attribute__((always_inline)) {
          constexpr int ib = decltype(bc)::value;
          z[ib] = mfma(w0, yb[Y.base + ib][0], f4{0.f, 0.f, 0.f, 0.f});
          z[ib] = mfma(w1, yb[Y.base + ib][1], z[ib]);
        });
        const auto cfs = load_coefs<ps.mask>(cf, p);
        static_for<8>([&](auto sc2) __attribute__((always_inline)) {
          constexpr int sl = decltype(sc2)::value;
          constexpr int oc = sl >> 2, ia = (sl >> 1) & 1, ib = sl & 1;
          if constexpr ((ps.mask >> sl) & 1) {
            const float cv = coef_at<sl>(cfs);
            static_for<4>([&](auto rc) __attribute__((always_inline)) {
              constexpr int r = decltype(rc)::value;
              ov[r * O.dim + oc] += cv * (xv[4 * X.base + r * X.dim + ia] * z[ib][r]);
            });
          }
        });
#pragma unroll
        for (int i = 0; i < 4 * O.dim; ++i) asm volatile("" : "+v"(ov[i]));
        if constexpr (last) store_entry<O.dim>(ro, xrow, O.off * a.C, u, ov);
      });
      if (c + 1 < NCH || u0 + 16 < u_end)
        vchunk_commit<Plan, NT>(pf, s_mem + L::kCoefPad + (parity ^ 1) * L::kBufFloats);
      parity ^= 1;
      __syncthreads();
    });
  }
}

// Input adjoints.  needed: 1 = x, 2 = y.  With channel splits (grid y) dy is
// written per split into Args::part_dy for a fixed-order sum.
template <class Plan>
__global__ __launch_bounds__(64 * kSBwdWaves, 1) void uvu_vshared_backward_kernel(
    Args a, const float* gout, float* gx, float* gy, int needed) {
  constexpr int NT = 64 * kSBwdWaves;
  using L = VLayout<Plan>;
  constexpr int P = Plan::kPaths;
  constexpr int NC = Plan::kComps1;
  constexpr int NY = Plan::kComps2;
  constexpr int NYT = (NY + 1) / 2;  // dy accumulator tiles: components 2t, 2t + 1
  constexpr int PC = kVChunk;
  constexpr int NCH = L::kChunks;
  __shared__ __attribute__((aligned(16))) float s_mem[L::kFloats];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
  const int g = lane >> 4, j = lane & 15;
  const int64_t e0 = ((int64_t)blockIdx.x * (NT / 64) + wave) * kEdgesPerWave;
  const int64_t rows = a.n - e0 < kEdgesPerWave ? a.n - e0 : kEdgesPerWave;
  const auto rx = rows_rsrc(a.x, e0, a.W1, rows);
  const auto rg = rows_rsrc(gout, e0, a.W1, rows);
  const auto ry = rows_rsrc(a.y, e0, a.W2, rows);
  const uint32_t xrow = (uint32_t)(j * a.W1) * 4u;
  const bool need_y = (needed & 2) != 0;
  const auto rdx = rows_rsrc(gx, e0, a.W1, (needed & 1) ? rows : 0);
  float* dy_base = a.part_dy ? a.part_dy + (int64_t)blockIdx.y * a.n * a.W2 : gy;

  for (int idx = threadIdx.x; idx < P * 8; idx += NT) s_mem[idx] = a.coef[idx];
  float yb[NY][2];
  load_yb<Plan>(ry, a, g, j, yb);
  f4 dyt[NYT];
  static_for<NYT>([&](auto tc) __attribute__((always_inline)) { dyt[decltype(tc)::value] = f4{0.f, 0.f, 0.f, 0.f}; });
  // Row j of a dy tile's A operand holds component parity j / 8, copy j % 8.
  const int a_par = j >> 3;

  const int u_begin = blockIdx.y * a.tile_span;
  const int u_end = u_begin + a.tile_span < a.C ? u_begin + a.tile_span : a.C;
  VChunk<Plan, NT> pf;
  vchunk_fetch<Plan, NT, true, 0>(pf, a, u_begin);
  vchunk_commit<Plan, NT>(pf, s_mem + L::kCoefPad);
  int parity = 0;
  for (int u0 = u_begin; u0 < u_end; u0 += 16) {
    __syncthreads();
    const int u = u0 + 4 * g;
    float gv[4 * NC];
    load_row<Plan>(rg, xrow, a.C, u, gv);
    static_for<Plan::kEntries1>([&](auto ec) __attribute__((always_inline)) {
      constexpr int e = decltype(ec)::value;
      constexpr REntry X = Plan::e1[e];
      if constexpr (!entry_used<Plan, false>(e)) store_zero_entry<X.dim>(rdx, xrow, X.off * a.C, u);
    });
    float xc[8], xn[8], dxc[8];
    {
      constexpr REntry X0 = Plan::e1[Plan::paths[Plan::bwd[0]].i];
      load_entry<X0.dim>(rx, xrow, X0.off * a.C, u, xn);
    }
    static_for<NCH>([&](auto cc) __attribute__((always_inline)) {
      constexpr int c = decltype(cc)::value;
      if constexpr (c + 1 < NCH) {
        vchunk_fetch<Plan, NT, true, c + 1>(pf, a, u0);
      } else {
        if (u0 + 16 < u_end) vchunk_fetch<Plan, NT, true, 0>(pf, a, u0 + 16);
      }
      const int buf = L::kCoefPad + parity * L::kBufFloats;
      int coef_off = 0, w_off = buf + j * kVK + 2 * g, wcol_off = buf + 4 * g * kVK + (j & 7);
      asm volatile("" : "+v"(coef_off), "+v"(w_off), "+v"(wcol_off));
      const float* cf = s_mem + coef_off;
      static_for<(P - c * PC < PC ? P - c * PC : PC)>([&](auto sc) __attribute__((always_inline)) {
        constexpr int slot = decltype(sc)::value;
        constexpr int q = c * PC + slot;
        constexpr int p = Plan::bwd[q];
        constexpr RPath ps = Plan::paths[p];
        constexpr REntry X = Plan::e1[ps.i];
        constexpr REntry Y = Plan::e2[ps.j];
        constexpr REntry O = Plan::e1[ps.k];
        constexpr bool first = q == 0 || Plan::paths[Plan::bwd[q == 0 ? 0 : q - 1]].i != ps.i;
        constexpr bool last = q == P - 1 || Plan::paths[Plan::bwd[q == P - 1 ? q : q + 1]].i != ps.i;
        if constexpr (first) {
          static_for<8>([&](auto ic) __attribute__((always_inline)) {
            xc[decltype(ic)::value] = xn[decltype(ic)::value];
            dxc[decltype(ic)::value] = 0.f;
          });
          if constexpr (q < P - 1) {
            constexpr int qn = [] {
              int t = q + 1;
              while (t < P && Plan::paths[Plan::bwd[t]].i == Plan::paths[Plan::bwd[q]].i) ++t;
              return t;
            }();
            if constexpr (qn < P) {
              constexpr REntry XN = Plan::e1[Plan::paths[Plan::bwd[qn]].i];
              load_entry<XN.dim>(rx, xrow, XN.off * a.C, u, xn);
            }
          }
        }
        const float* wl = s_mem + w_off + slot * 16 * kVK;
        const float w0 = wl[0], w1 = wl[1];
        const float* wc = s_mem + wcol_off + slot * 16 * kVK;
        const auto cfs = load_coefs<ps.mask>(cf, p);
        static_for<Y.dim>([&](auto bc) __attribute__((always_inline)) {
          constexpr int ib = decltype(bc)::value;
          f4 z = mfma(w0, yb[Y.base + ib][0], f4{0.f, 0.f, 0.f, 0.f});
          z = mfma(w1, yb[Y.base + ib][1], z);
          float gz[4] = {0.f, 0.f, 0.f, 0.f};
          static_for<8>([&](auto sc2) __attribute__((always_inline)) {
            constexpr int sl = decltype(sc2)::value;
            constexpr int oc = sl >> 2, ia = (sl >> 1) & 1;
            if constexpr (((ps.mask >> sl) & 1) && (sl & 1) == ib) {
              const float cv = coef_at<sl>(cfs);
              static_for<4>([&](auto rc) __attribute__((always_inline)) {
                constexpr int r = decltype(rc)::value;
                const float xr = xc[r * X.dim + ia];
                const float gr = gv[4 * O.base + r * O.dim + oc];
                gz[r] += cv * (xr * gr);
                dxc[r * X.dim + ia] += cv * (gr * z[r]);
              });
            }
          });
          if (need_y) {
            constexpr int comp = Y.base + ib;
            constexpr int t = comp >> 1;
            const bool mine = a_par == (comp & 1);
            static_for<4>([&](auto kc) __attribute__((always_inline)) {
              constexpr int s = decltype(kc)::value;
              const float av = mine ? wc[s * kVK] : 0.f;
              dyt[t] = mfma(av, gz[s], dyt[t]);
            });
          }
        });
#pragma unroll
        for (int i = 0; i < 4 * X.dim; ++i) asm volatile("" : "+v"(dxc[i]));
        if constexpr (last) store_entry<X.dim>(rdx, xrow, X.off * a.C, u, dxc);
        __builtin_amdgcn_sched_barrier(0);
      });
      if (c + 1 < NCH || u0 + 16 < u_end)
        vchunk_commit<Plan, NT>(pf, s_mem + L::kCoefPad + (parity ^ 1) * L::kBufFloats);
      parity ^= 1;
      __syncthreads();
    });
  }
  if (need_y && j < rows) {
    // Lane (g, j) holds rows 4g .. 4g+3 of each tile: component 2t + g / 2,
    // copies 4 (g % 2) .. +3, of edge j.
    float* dst = dy_base + (e0 + j) * a.W2;
    const int hi = g >> 1;
    static_for<NYT>([&](auto tc) __attribute__((always_inline)) {
      constexpr int t = decltype(tc)::value;
      constexpr int c0 = 2 * t, c1 = 2 * t + 1 < NY ? 2 * t + 1 : 2 * t;
      if (!hi || 2 * t + 1 < NY) {
        static_for<4>([&](auto rc) __attribute__((always_inline)) {
          constexpr int r = decltype(rc)::value;
          const int v = 4 * (g & 1) + r;
          if (v < a.V) {
            const int off = hi ? y_offset<Plan, c1>(a.V, v) : y_offset<Plan, c0>(a.V, v);
            dst[off] = dyt[t][r];
          }
        });
      }
    });
  }
}

#ifndef O2MI_VDW_PATHS
#define O2MI_VDW_PATHS 16
#endif

// Weight gradient: paths per wave (at most O2MI_VDW_PATHS) and path groups
// (grid z), edges per staged tile.  A wave keeps one 16 x 16 accumulator tile (channels x copies) per
// path.
template <class Plan>
constexpr int vdw_paths() {
  const int n = (Plan::kPaths + 7) / 8;
  return n < O2MI_VDW_PATHS ? n : O2MI_VDW_PATHS;
}

template <class Plan>
constexpr int vdw_groups() {
  return (Plan::kPaths + 8 * vdw_paths<Plan>() - 1) / (8 * vdw_paths<Plan>());
}

template <class Plan, int kE, int NT>
struct VTile {
  static constexpr int kXS = 16 * Plan::kComps1 + 1;  // odd row stride (banks)
  static constexpr int kX = kE * kXS;
  static constexpr int kY = kE * kVK * Plan::kComps2;  // rows of width W2 <= kVK * kComps2
  static constexpr int kFloats = (2 * kX + kY + 3) / 4 * 4;
  static constexpr int kXPer = (kE * 16 * Plan::kComps1 + NT - 1) / NT;
  static constexpr int kYPer = (kY + NT - 1) / NT;
};

template <class Plan>
constexpr int vdw_edges() {
  constexpr int kCoefPad = (Plan::kPaths * 8 + 3) / 4 * 4;
  return 4 * (kCoefPad + 2 * VTile<Plan, 32, kThreads>::kFloats) <= 160 * 1024 ? 32 : 16;
}

template <class Plan, int kE, int NT>
struct VPrefetch {
  using T = VTile<Plan, kE, NT>;
  float x[T::kXPer], g[T::kXPer], y[T::kYPer];
};

// Byte offsets of this thread's x / g tile elements in a tile's rows (the same
// for every tile; the entry lookup is a compare chain per element).
template <class Plan, int kE, int NT>
struct VCols {
  uint32_t voff[VTile<Plan, kE, NT>::kXPer];
};

template <class Plan, int kE, int NT>
__device__ __forceinline__ void vtile_fetch(VPrefetch<Plan, kE, NT>& pf, const Args& a,
                                            const float* gout, int64_t t0, int64_t t_end,
                                            const VCols<Plan, kE, NT>& cols) {
  using T = VTile<Plan, kE, NT>;
  const int64_t rows = t_end - t0 < kE ? t_end - t0 : kE;
  const auto rx = rows_rsrc(a.x, t0, a.W1, rows);
  const auto rg = rows_rsrc(gout, t0, a.W1, rows);
  const auto ry = rows_rsrc(a.y, t0, a.W2, rows);
  static_for<T::kXPer>([&](auto kc) __attribute__((always_inline)) {
    constexpr int k = decltype(kc)::value;
    pf.x[k] = ld1(rx, cols.voff[k]);
    pf.g[k] = ld1(rg, cols.voff[k]);
  });
  static_for<T::kYPer>([&](auto kc) __attribute__((always_inline)) {
    constexpr int k = decltype(kc)::value;
    const int idx = threadIdx.x + k * NT;
    pf.y[k] = ld1(ry, idx < kE * a.W2 ? (uint32_t)idx * 4u : kIdle);  // rows of y are contiguous
  });
}

template <class Plan, int kE, int NT>
__device__ __forceinline__ void vtile_commit(const VPrefetch<Plan, kE, NT>& pf, float* buf) {
  using T = VTile<Plan, kE, NT>;
  constexpr int XE = 16 * Plan::kComps1;
  float* sx = buf;
  float* sg = buf + T::kX;
  float* sy = buf + 2 * T::kX;
  static_for<T::kXPer>([&](auto kc) __attribute__((always_inline)) {
    constexpr int k = decltype(kc)::value;
    const int idx = threadIdx.x + k * NT;
    if (idx < kE * XE) {
      const int edge = idx / XE, rest = idx - edge * XE;
      sx[edge * T::kXS + rest] = pf.x[k];
      sg[edge * T::kXS + rest] = pf.g[k];
    }
  });
  static_for<T::kYPer>([&](auto kc) __attribute__((always_inline)) {
    constexpr int k = decltype(kc)::value;
    const int idx = threadIdx.x + k * NT;
    if (idx < T::kY) sy[idx] = pf.y[k];
  });
}

// One step of 4 edges for the wave's paths [Q0, Q0 + NPW) of Plan::wgt: lane
// (g, j) forms gz for edge 4s + g and channel u0 + j (the A operand) and
// supplies copy j of the edge's components (the B operand).
template <class Plan, int kE, int NT, int Q0, int NPW>
__device__ __forceinline__ void vdw_step(const float* buf, int V, int W2, int edge, int j,
                                         f4 (&acc)[vdw_paths<Plan>()]) {
  using T = VTile<Plan, kE, NT>;
  const float* sx = buf;
  const float* sg = buf + T::kX;
  const float* sy = buf + 2 * T::kX;
  float xv[Plan::kComps1], gv[Plan::kComps1], yv[Plan::kComps2];
  static_for<Plan::kEntries1>([&](auto ec) __attribute__((always_inline)) {
    constexpr int e = decltype(ec)::value;
    constexpr REntry E = Plan::e1[e];
    constexpr bool use_x = wgt_uses<Plan, 0>(Q0, NPW, e);
    constexpr bool use_g = wgt_uses<Plan, 2>(Q0, NPW, e);
    static_for<E.dim>([&](auto dc) __attribute__((always_inline)) {
      constexpr int d = decltype(dc)::value;
      const int o = edge * T::kXS + 16 * E.base + j * E.dim + d;
      if constexpr (use_x) xv[E.base + d] = sx[o];
      if constexpr (use_g) gv[E.base + d] = sg[o];
    });
  });
  const bool copy_ok = j < V;
  static_for<Plan::kEntries2>([&](auto ec) __attribute__((always_inline)) {
    constexpr int e = decltype(ec)::value;
    constexpr REntry E = Plan::e2[e];
    if constexpr (wgt_uses<Plan, 1>(Q0, NPW, e))
      static_for<E.dim>([&](auto dc) __attribute__((always_inline)) {
        constexpr int d = decltype(dc)::value;
        const float val = sy[edge * W2 + y_offset<Plan, E.base + d>(V, copy_ok ? j : 0)];
        yv[E.base + d] = copy_ok ? val : 0.f;
      });
  });
  static_for<NPW>([&](auto qc) __attribute__((always_inline)) {
    constexpr int q = decltype(qc)::value;
    constexpr int p = Plan::wgt[Q0 + q];
    constexpr RPath ps = Plan::paths[p];
    constexpr REntry X = Plan::e1[ps.i];
    constexpr REntry Y = Plan::e2[ps.j];
    constexpr REntry O = Plan::e1[ps.k];
    // The couplings' signs are compiled (one FMA per slot); their magnitude
    // scales the finished sums.
    static_for<Y.dim>([&](auto bc) __attribute__((always_inline)) {
      constexpr int ib = decltype(bc)::value;
      float gz = 0.f;
      static_for<8>([&](auto sc) __attribute__((always_inline)) {
        constexpr int sl = decltype(sc)::value;
        constexpr int oc = sl >> 2, ia = (sl >> 1) & 1;
        if constexpr (((ps.mask >> sl) & 1) && (sl & 1) == ib) {
          if constexpr ((ps.neg >> sl) & 1)
            gz -= xv[X.base + ia] * gv[O.base + oc];
          else
            gz += xv[X.base + ia] * gv[O.base + oc];
        }
      });
      acc[q] = mfma(gz, yv[Y.base + ib], acc[q]);
    });
  });
}

template <class Plan, int G0>
__device__ __forceinline__ void vdw_body(float* s_mem, const Args& a, const float* gout,
                                         int64_t edges_per_slice, float* part) {
  constexpr int NT = kThreads;
  constexpr int kE = vdw_edges<Plan>();
  constexpr int NPW = vdw_paths<Plan>();
  using T = VTile<Plan, kE, NT>;
  constexpr int P = Plan::kPaths;
  constexpr int XE = 16 * Plan::kComps1;
  // The first kCoefPad floats are unused (the couplings' signs are compiled);
  // they keep the tile size that vdw_edges() chose for this layout.
  constexpr int kCoefPad = (P * 8 + 3) / 4 * 4;
  float* s_tile = s_mem + kCoefPad;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
  const int g = lane >> 4, j = lane & 15;
  const int u0 = blockIdx.y * 16;
  const int64_t begin = (int64_t)blockIdx.x * edges_per_slice;
  const int64_t end = begin + edges_per_slice < a.n ? begin + edges_per_slice : a.n;
  const int tiles = end > begin ? (int)((end - begin + kE - 1) / kE) : 0;
  const int nv = a.V, w2 = a.W2;

  f4 acc[NPW];
  static_for<NPW>([&](auto qc) __attribute__((always_inline)) { acc[decltype(qc)::value] = f4{0.f, 0.f, 0.f, 0.f}; });

  VCols<Plan, kE, NT> cols;
  static_for<T::kXPer>([&](auto kc) __attribute__((always_inline)) {
    constexpr int k = decltype(kc)::value;
    const int idx = threadIdx.x + k * NT;
    cols.voff[k] = kIdle;
    if (idx < kE * XE) {
      const int edge = idx / XE;
      cols.voff[k] = (uint32_t)(edge * a.W1 + tile_x_offset<Plan>(idx - edge * XE, a.C, u0)) * 4u;
    }
  });
  VPrefetch<Plan, kE, NT> pf;
  if (tiles > 0) {
    vtile_fetch<Plan, kE, NT>(pf, a, gout, begin, end, cols);
    vtile_commit<Plan, kE, NT>(pf, s_tile);
  }
  __syncthreads();
  for (int t = 0; t < tiles; ++t) {
    const bool more = t + 1 < tiles;
    if (more) vtile_fetch<Plan, kE, NT>(pf, a, gout, begin + (int64_t)(t + 1) * kE, end, cols);
    const float* buf = s_tile + (t & 1) * T::kFloats;
    static_for<kWaves>([&](auto wc) __attribute__((always_inline)) {
      constexpr int w = decltype(wc)::value;
      constexpr int q0 = G0 * 8 * NPW + w * NPW;
      constexpr int np = P - q0 < NPW ? P - q0 : NPW;
      if constexpr (np > 0) {
        if (wave == w) {
#pragma unroll
          for (int s = 0; s < kE / 4; ++s)
            vdw_step<Plan, kE, NT, q0, np>(buf, nv, w2, 4 * s + g, j, acc);
        }
      }
    });
    if (more) vtile_commit<Plan, kE, NT>(pf, s_tile + ((t + 1) & 1) * T::kFloats);
    __syncthreads();
  }

  // Lane (g, j) holds dw[channel u0 + 4g + r][copy j].
  float* dst = part + (int64_t)blockIdx.x * P * a.C * a.V;
  static_for<kWaves>([&](auto wc) __attribute__((always_inline)) {
    constexpr int w = decltype(wc)::value;
    constexpr int q0 = G0 * 8 * NPW + w * NPW;
    constexpr int np = P - q0 < NPW ? P - q0 : NPW;
    if constexpr (np > 0) {
      if (wave == w && j < a.V) {
        static_for<np>([&](auto qc) __attribute__((always_inline)) {
          constexpr int q = decltype(qc)::value;
          constexpr int p = Plan::wgt[q0 + q];
          const int64_t row = (int64_t)p * a.C + u0 + 4 * g;
          const float mag = fabsf(a.coef[p * 8 + first_slot(Plan::paths[p].mask)]);
          static_for<4>([&](auto rc) __attribute__((always_inline)) {
            constexpr int r = decltype(rc)::value;
            dst[(row + r) * a.V + j] = acc[q][r] * mag;
          });
        });
      }
    }
  });
}

// Grid (slices, C/16, vdw_groups<Plan>()): part[slice][p][u][v].
template <class Plan>
__global__ __launch_bounds__(kThreads, 1) void uvu_vshared_dw_kernel(Args a, const float* gout,
                                                                     int64_t edges_per_slice,
                                                                     float* part) {
  constexpr int kCoefPad = (Plan::kPaths * 8 + 3) / 4 * 4;
  __shared__ __attribute__((aligned(16)))
  float s_mem[kCoefPad + 2 * VTile<Plan, vdw_edges<Plan>(), kThreads>::kFloats];
  static_for<vdw_groups<Plan>()>([&](auto gc) __attribute__((always_inline)) {
    constexpr int grp = decltype(gc)::value;
    if (blockIdx.z == grp) vdw_body<Plan, grp>(s_mem, a, gout, edges_per_slice, part);
  });
}

}  // namespace radial
}  // namespace o2mi
