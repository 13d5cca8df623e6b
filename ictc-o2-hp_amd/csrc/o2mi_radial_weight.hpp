// Affine-parameter adjoints of the fused radial product for structures of up
// to 32 paths (configs[4]'s C64 m4 canonical has 31):
//   dalpha[p*C + u, h] = sum_e gw[e, p, u] hidden[e, h],  dbias = sum_e gw,
//   gw[e, p, u] = sum_slots coef * y[e, j] * x[e, i, u] * g[e, k, u].
//
// A block of 8 waves owns a 16-channel tile and an edge slice, walked in
// tiles of 32 edges, and splits its waves by role:
//  * producers (waves 4-7, VALU): each thread takes one edge and two
//    neighbouring channels of the tile, reads their x and g values straight
//    from memory (16-byte loads for frequency entries) and the edge's y, forms
//    gw of every path once and writes it to LDS as [path][edge][channel]; it
//    also stages 8 of the edge's hidden values;
//  * consumers (waves 0-3, matrix cores): consumer w owns up to 8 consecutive
//    paths of Plan::wgt and keeps their dalpha tiles (64 hidden x 16
//    channels) in accumulators; per step of 4 edges it reads one gw value per
//    path and one hidden value per 16-row tile from LDS (the next step's read
//    ahead of this step's MFMAs) and issues up to 32 MFMAs
//    (dalpha^T[h, channel] += hidden^T[h, edge] gw[edge, channel]).
// Waves are placed on the SIMDs round-robin, so each SIMD holds one producer
// and one consumer: the producers' VALU work for tile t + 1 runs beside the
// consumers' matrix work on tile t (double-buffered LDS, one barrier per
// tile).  Producers load tile t + 2 while forming tile t + 1.
//
// The couplings' signs are compiled; gw is formed without the path's coupling
// magnitude, which scales the finished sums.  Slice partials are summed in a
// fixed order afterwards (bitwise reproducible).
#pragma once

#include "o2mi_radial.hpp"
#include "o2mi_radial_streamed.hpp"

namespace o2mi {
namespace radial {

constexpr int kGwConsumers = 4;
constexpr int kGwProducers = 4;
constexpr int kGwThreads = 64 * (kGwConsumers + kGwProducers);
constexpr int kGwEdges = 32;  // edges per tile
// Producer thread: one edge, channels 2c and 2c + 1 of the 16-channel tile.
static_assert(kGwEdges * 8 == 64 * kGwProducers, "producers cover a tile exactly");

template <class Plan, int KH>
struct GwLayout {
  static constexpr int kPerWave = (Plan::kPaths + kGwConsumers - 1) / kGwConsumers;
  static constexpr int kHS = Geom<KH>::kHid + 16;           // hidden row stride
  static constexpr int kGw = Plan::kPaths * kGwEdges * 16;  // one gw buffer
  static constexpr int kH = kGwEdges * kHS;                 // one hidden buffer
  static constexpr int kFloats = 2 * kGw + 2 * kH;
  static_assert(kPerWave <= 8, "up to 32 paths");
  static_assert(Geom<KH>::kHid == 4 * 16, "producers stage 64 hidden floats per edge");
};

using f2v = float __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f2v ld2(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  return __builtin_bit_cast(f2v, __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, 0, 0));
}

// A producer thread's operands of one tile, in registers: x and g of its two
// channels ([component][channel of the pair]), y, and 8 hidden values.
template <class Plan>
struct GwOperands {
  float x[Plan::kComps1][2], g[Plan::kComps1][2], y[Plan::kComps2];
  f4 h[2];
};

// Loads the operands of edge e0 + el, channels u0 + 2 cp, + 1; rows past
// `end` (or a gathered row outside the table) read zeros.  `row` is the
// edge's node row for a gathered first input.
template <class Plan, int KH>
__device__ __forceinline__ void gw_fetch(GwOperands<Plan>& op, const Args& a,
                                         const float* gout, int64_t e0, int64_t end, int el,
                                         int cp, int u0, int64_t row) {
  const int64_t rows = end - e0 < kGwEdges ? end - e0 : kGwEdges;
  const auto rx = x_rsrc(a, e0, rows);
  const auto rg = rows_rsrc(gout, e0, a.W1, rows);
  const auto ry = rows_rsrc(a.y, e0, a.W2, rows);
  const auto rh = rows_rsrc(a.hidden, e0, a.H, rows);
  uint32_t xrow = (uint32_t)(el * a.W1) * 4u;
  if (a.xindex) xrow = (el < rows && row >= 0 && row < a.x_rows)
                           ? (uint32_t)row * (uint32_t)a.W1 * 4u : kIdle;
  const uint32_t grow = (uint32_t)(el * a.W1) * 4u;
  static_for<Plan::kEntries1>([&](auto ec) __attribute__((always_inline)) {
    constexpr REntry E = Plan::e1[decltype(ec)::value];
    // The pair's E.dim x 2 values are contiguous: [channel][component].
    const uint32_t col = (uint32_t)(E.off * a.C + E.dim * (u0 + 2 * cp)) * 4u;
    const uint32_t xo = xrow == kIdle ? kIdle : xrow + col;
    if constexpr (E.dim == 2) {
      const f4 xv = ld4(rx, xo), gv = ld4(rg, grow + col);
      op.x[E.base][0] = xv.x; op.x[E.base + 1][0] = xv.y;
      op.x[E.base][1] = xv.z; op.x[E.base + 1][1] = xv.w;
      op.g[E.base][0] = gv.x; op.g[E.base + 1][0] = gv.y;
      op.g[E.base][1] = gv.z; op.g[E.base + 1][1] = gv.w;
    } else {
      const f2v xv = ld2(rx, xo), gv = ld2(rg, grow + col);
      op.x[E.base][0] = xv.x; op.x[E.base][1] = xv.y;
      op.g[E.base][0] = gv.x; op.g[E.base][1] = gv.y;
    }
  });
  static_for<Plan::kComps2>([&](auto cc) __attribute__((always_inline)) {
    constexpr int m = decltype(cc)::value;
    op.y[m] = ld1(ry, (uint32_t)(el * a.W2 + m) * 4u);
  });
  static_for<2>([&](auto kc) __attribute__((always_inline)) {
    constexpr int k = decltype(kc)::value;
    const int h = 8 * cp + 4 * k;
    op.h[k] = ld4(rh, h < a.H ? (uint32_t)(el * a.H + h) * 4u : kIdle);
  });
}

// Producer work for one tile: gw of every path (without its coupling
// magnitude) for the thread's edge and two channels into
// gw[path][edge][channel], and its 8 hidden values.
template <class Plan, int KH>
__device__ __forceinline__ void gw_form(const GwOperands<Plan>& op, float* gw, float* hb, int el,
                                        int cp) {
  using L = GwLayout<Plan, KH>;
  float z[2][2][2];  // [ia][ib][channel of the pair]
  static_for<Plan::kPaths>([&](auto qc) __attribute__((always_inline)) {
    constexpr int q = decltype(qc)::value;
    constexpr RPath ps = Plan::paths[Plan::wgt[q]];
    constexpr REntry X = Plan::e1[ps.i];
    constexpr REntry Y = Plan::e2[ps.j];
    constexpr REntry O = Plan::e1[ps.k];
    // The x y products of a (first, second) entry pair, shared by its paths
    // (consecutive in Plan::wgt); per output component T = sum of the signed
    // products, gw = sum over components of g T.
    constexpr bool first = q == 0 || Plan::paths[Plan::wgt[q == 0 ? 0 : q - 1]].i != ps.i ||
                           Plan::paths[Plan::wgt[q == 0 ? 0 : q - 1]].j != ps.j;
    if constexpr (first)
      static_for<X.dim * Y.dim * 2>([&](auto zc) __attribute__((always_inline)) {
        constexpr int ia = decltype(zc)::value / (2 * Y.dim);
        constexpr int ib = decltype(zc)::value / 2 % Y.dim, k = decltype(zc)::value % 2;
        z[ia][ib][k] = op.x[X.base + ia][k] * op.y[Y.base + ib];
      });
    f2v v = {0.f, 0.f};
    static_for<2>([&](auto kc) __attribute__((always_inline)) {
      constexpr int k = decltype(kc)::value;
      static_for<O.dim>([&](auto occ) __attribute__((always_inline)) {
        constexpr int oc = decltype(occ)::value;
        float t = 0.f;
        static_for<4>([&](auto sc) __attribute__((always_inline)) {
          constexpr int slot = oc * 4 + decltype(sc)::value;
          constexpr int ia = (slot >> 1) & 1, ib = slot & 1;
          if constexpr ((ps.mask >> slot) & 1) {
            if constexpr ((ps.neg >> slot) & 1)
              t -= z[ia][ib][k];
            else
              t += z[ia][ib][k];
          }
        });
        v[k] += op.g[O.base + oc][k] * t;
      });
    });
    *reinterpret_cast<f2v*>(gw + (q * kGwEdges + el) * 16 + 2 * cp) = v;
  });
  static_for<2>([&](auto kc) __attribute__((always_inline)) {
    constexpr int k = decltype(kc)::value;
    *reinterpret_cast<f4*>(hb + el * L::kHS + 8 * cp + 4 * k) = op.h[k];
  });
}

// Consumer W's paths over one tile: kGwEdges / 4 steps of 4 edges.
template <class Plan, int KH, int W>
__device__ __forceinline__ void gw_accumulate(
    const float* gw, const float* hb, int g, int j,
    f4 (&ga)[GwLayout<Plan, KH>::kPerWave][Geom<KH>::kTiles],
    float (&gb)[GwLayout<Plan, KH>::kPerWave]) {
  using G = Geom<KH>;
  using L = GwLayout<Plan, KH>;
  constexpr int q0 = W * L::kPerWave;
  constexpr int rest = Plan::kPaths - q0;
  constexpr int NP = rest < L::kPerWave ? (rest > 0 ? rest : 0) : L::kPerWave;
  constexpr int kSteps = kGwEdges / 4;
  float hv[2][G::kTiles], gv[2][NP > 0 ? NP : 1];
  auto read_step = [&](int s, int buf) __attribute__((always_inline)) {
    const int e = 4 * s + g;
    static_for<G::kTiles>([&](auto tc) __attribute__((always_inline)) {
      constexpr int t = decltype(tc)::value;
      hv[buf][t] = hb[e * L::kHS + 16 * t + j];
    });
    static_for<NP>([&](auto qc) __attribute__((always_inline)) {
      constexpr int q = decltype(qc)::value;
      gv[buf][q] = gw[((q0 + q) * kGwEdges + e) * 16 + j];
    });
  };
  read_step(0, 0);
  static_for<kSteps>([&](auto sc) __attribute__((always_inline)) {
    constexpr int s = decltype(sc)::value;
    constexpr int b = s & 1;
    if constexpr (s + 1 < kSteps) read_step(s + 1, b ^ 1);
    static_for<NP>([&](auto qc) __attribute__((always_inline)) {
      constexpr int q = decltype(qc)::value;
      gb[q] += gv[b][q];
      static_for<G::kTiles>([&](auto tc) __attribute__((always_inline)) {
        constexpr int t = decltype(tc)::value;
        ga[q][t] = mfma(hv[b][t], gv[b][q], ga[q][t]);
      });
    });
  });
}

// Grid (slices, C / 16); block kGwThreads.
template <class Plan, int KH>
__global__ __launch_bounds__(kGwThreads, 1) void radial_weight_gw_kernel(
    Args a, const float* gout, int64_t edges_per_slice, float* part_alpha, float* part_bias) {
  using G = Geom<KH>;
  using L = GwLayout<Plan, KH>;
  __shared__ __attribute__((aligned(16))) float s_mem[L::kFloats];
  float* s_gw = s_mem;
  float* s_h = s_mem + 2 * L::kGw;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
  const int u0 = blockIdx.y * 16;
  const int64_t begin = (int64_t)blockIdx.x * edges_per_slice;
  const int64_t end = begin + edges_per_slice < a.n ? begin + edges_per_slice : a.n;
  const int tiles = end > begin ? (int)((end - begin + kGwEdges - 1) / kGwEdges) : 0;

  if (wave >= kGwConsumers) {
    // Producer thread pt: edge pt / 8, channels 2 (pt % 8) and + 1.  Every
    // producer passes the same barriers as the consumers (tiles + 1).
    const int pt = threadIdx.x - 64 * kGwConsumers;
    const int el = pt >> 3, cp = pt & 7;
    // Node rows of a gathered first input, loaded a tile ahead of the x
    // loads that use them.
    auto node_row = [&](int t) -> int64_t {
      const int64_t e = begin + (int64_t)t * kGwEdges + el;
      return (a.xindex && t < tiles && e < end) ? a.xindex[e] : -1;
    };
    GwOperands<Plan> op;
    int64_t row_next = node_row(1);
    if (tiles > 0) {
      gw_fetch<Plan, KH>(op, a, gout, begin, end, el, cp, u0, node_row(0));
      gw_form<Plan, KH>(op, s_gw, s_h, el, cp);
    }
    // Operands of tile 1 (zeros past the slice).
    gw_fetch<Plan, KH>(op, a, gout, begin + kGwEdges, end, el, cp, u0, row_next);
    row_next = node_row(2);
    __syncthreads();
    for (int t = 0; t < tiles; ++t) {
      gw_form<Plan, KH>(op, s_gw + ((t + 1) & 1) * L::kGw, s_h + ((t + 1) & 1) * L::kH, el, cp);
      gw_fetch<Plan, KH>(op, a, gout, begin + (int64_t)(t + 2) * kGwEdges, end, el, cp, u0,
                         row_next);
      row_next = node_row(t + 3);
      __syncthreads();
    }
    return;
  }

  // Consumers.
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, j = lane & 15;
  f4 ga[L::kPerWave][G::kTiles];
  float gb[L::kPerWave];
  static_for<L::kPerWave>([&](auto qc) __attribute__((always_inline)) {
    constexpr int q = decltype(qc)::value;
    gb[q] = 0.f;
    static_for<G::kTiles>([&](auto tc) __attribute__((always_inline)) {
      ga[q][decltype(tc)::value] = f4{0.f, 0.f, 0.f, 0.f};
    });
  });
  __syncthreads();
  for (int t = 0; t < tiles; ++t) {
    const float* gw = s_gw + (t & 1) * L::kGw;
    const float* hb = s_h + (t & 1) * L::kH;
    static_for<kGwConsumers>([&](auto wc) __attribute__((always_inline)) {
      constexpr int w = decltype(wc)::value;
      if (wave == w) gw_accumulate<Plan, KH, w>(gw, hb, g, j, ga, gb);
    });
    __syncthreads();
  }

  // Partial sums of this slice, scaled by each path's coupling magnitude.
  const int64_t PC = (int64_t)Plan::kPaths * a.C;
  float* pa = part_alpha + (int64_t)blockIdx.x * PC * a.H;
  float* pb = part_bias + (int64_t)blockIdx.x * PC;
  static_for<kGwConsumers>([&](auto wc) __attribute__((always_inline)) {
    constexpr int w = decltype(wc)::value;
    constexpr int q0 = w * L::kPerWave;
    constexpr int rest = Plan::kPaths - q0;
    constexpr int np = rest < L::kPerWave ? (rest > 0 ? rest : 0) : L::kPerWave;
    if constexpr (np > 0) {
      if (wave == w) {
        static_for<np>([&](auto qc) __attribute__((always_inline)) {
          constexpr int q = decltype(qc)::value;
          constexpr int p = Plan::wgt[q0 + q];
          const float mag = fabsf(a.coef[p * 8 + first_slot(Plan::paths[p].mask)]);
          const int64_t prow = (int64_t)p * a.C + u0 + j;
          static_for<G::kTiles>([&](auto tc) __attribute__((always_inline)) {
            constexpr int tt = decltype(tc)::value;
            const int h = 16 * tt + 4 * g;
            if (h < a.H) *reinterpret_cast<f4*>(pa + prow * a.H + h) = ga[q][tt] * mag;
          });
          float b = gb[q];
          b += __shfl_xor(b, 16);
          b += __shfl_xor(b, 32);
          if (g == 0) pb[prow] = b * mag;
        });
      }
    }
  });
}

}  // namespace radial
}  // namespace o2mi
