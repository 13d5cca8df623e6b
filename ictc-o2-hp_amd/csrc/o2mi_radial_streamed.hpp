// Forward and input-adjoint kernels of the fused radial affine + V=1 uvu
// product (RadialUvuTensorProduct), and the affine-adjoint kernel for
// structures with many paths.  Alpha is streamed through LDS: the reference's
// m_max 6 full/canonical benchmark structure has 254 paths, 254 x 16 channels
// x 64 hidden floats = 1 MiB per channel tile, far more than LDS holds.
//
// A block of 8 waves owns 128 edges, 16 per wave, and walks the channels in
// tiles of 16 (see o2mi_radial.hpp for the MFMA weight tile and lane layout):
//  * alpha and bias are staged in chunks of Plan::kChunk paths, double
//    buffered: the global loads of chunk c + 1 are in flight while chunk c is
//    consumed, and land in the other LDS buffer before the chunk barrier.  The
//    chunk sequence runs on across channel tiles.
//  * paths are walked grouped by output entry (forward: one output entry of
//    accumulators live) or by first-input entry (input adjoints: one x and one
//    dx entry live, the next x entry loaded a group ahead), so the per-lane
//    state is one full row (4 channels x components) plus one entry.
//  * with fewer edge blocks than CUs the channel tiles are split over grid y;
//    the input adjoints then write dy / dhidden per split for a fixed-order sum.
#pragma once

#include "o2mi_radial.hpp"

namespace o2mi {
namespace radial {

// Waves per block: two per SIMD (256 registers each).  The input adjoints
// spill a few registers there (their state adds the hidden-adjoint
// accumulators and the next x entry), and still run 18% faster than at one
// wave per SIMD with 512 registers.
constexpr int kSFwdWaves = 8;
constexpr int kSBwdWaves = 8;

template <class Plan, int KH>
struct SLayout {
  static constexpr int kChunk = Plan::kChunk;
  static constexpr int kCoef = 0;
  static constexpr int kBuf0 = (Plan::kPaths * 8 + 3) / 4 * 4;
  static constexpr int kBias = 0;                  // within a buffer: [kChunk][16]
  static constexpr int kAlpha = kChunk * 16;       // within a buffer: [kChunk * 16][kRow]
  static constexpr int kBufFloats = kAlpha + kChunk * 16 * Geom<KH>::kRow;
  static constexpr int kFloats = kBuf0 + 2 * kBufFloats;
  static constexpr int kChunks = (Plan::kPaths + kChunk - 1) / kChunk;
  static_assert(kAlpha % 4 == 0 && kBufFloats % 4 == 0, "buffers must be 16-byte aligned");
  static_assert(Plan::kPaths * 16 <= 2 * kBufFloats, "shared uvu weights fit the chunk buffers");
};

// Per-thread registers of one chunk in flight: alpha rows as float4 (hidden
// zero-padded) and one bias value.
template <class Plan, int KH, int NT>
struct SChunk {
  static constexpr int kVec = Geom<KH>::kHid / 4;   // float4 per alpha row
  static constexpr int kPerPath = 16 * kVec;        // float4 per path and channel tile
  static_assert(NT % kPerPath == 0, "a thread's float4 must stay in one path slot");
  static constexpr int kSlotsPerPass = NT / kPerPath;
  static constexpr int kPer = (Plan::kChunk * kPerPath + NT - 1) / NT;
  f4 alpha[kPer];
  float bias;
};

// Path at traversal position q (Order = Plan::fwd or Plan::bwd).
template <class Plan, bool kBwd>
constexpr int path_at(int q) {
  return kBwd ? Plan::bwd[q] : Plan::fwd[q];
}

// Global loads of chunk c (positions c*kChunk ...) for channel tile u0.
template <class Plan, int KH, int NT, bool kBwd, int c>
__device__ __forceinline__ void chunk_fetch(SChunk<Plan, KH, NT>& pf, const Args& a, int u0) {
  using S = SChunk<Plan, KH, NT>;
  constexpr int PC = Plan::kChunk;
  // Laundered: the slot -> path selects of every chunk depend only on the
  // thread and would otherwise be hoisted out of the channel loop (and spill).
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  static_for<S::kPer>([&](auto kc) __attribute__((always_inline)) {
    constexpr int k = decltype(kc)::value;
    const int sub = tid / S::kPerPath;           // slot within this pass
    const int rest = tid - sub * S::kPerPath;    // r * kVec + qv
    const int r = rest / S::kVec, qv = rest - r * S::kVec;
    int path = -1;
    static_for<S::kSlotsPerPass>([&](auto sc) __attribute__((always_inline)) {
      constexpr int slot = k * S::kSlotsPerPass + decltype(sc)::value;
      constexpr int pos = c * PC + slot;
      if constexpr (slot < PC && pos < Plan::kPaths)
        if (sub == decltype(sc)::value) path = path_at<Plan, kBwd>(pos);
    });
    f4 v = {0.f, 0.f, 0.f, 0.f};
    if (path >= 0 && 4 * qv < a.H)
      v = *reinterpret_cast<const f4*>(a.alpha + (int64_t)(path * a.C + u0 + r) * a.H + 4 * qv);
    pf.alpha[k] = v;
  });
  pf.bias = 0.f;
  if (a.bias && tid < PC * 16) {
    const int slot = tid >> 4;
    int path = -1;
    static_for<PC>([&](auto sc) __attribute__((always_inline)) {
      constexpr int pos = c * PC + decltype(sc)::value;
      if constexpr (pos < Plan::kPaths)
        if (slot == decltype(sc)::value) path = path_at<Plan, kBwd>(pos);
    });
    if (path >= 0) pf.bias = a.bias[path * a.C + u0 + (tid & 15)];
  }
}

template <class Plan, int KH, int NT>
__device__ __forceinline__ void chunk_commit(const SChunk<Plan, KH, NT>& pf, float* buf) {
  using S = SChunk<Plan, KH, NT>;
  using G = Geom<KH>;
  using L = SLayout<Plan, KH>;
  const int tid = threadIdx.x;
  static_for<S::kPer>([&](auto kc) __attribute__((always_inline)) {
    constexpr int k = decltype(kc)::value;
    const int idx = tid + k * NT;
    if (idx < Plan::kChunk * S::kPerPath) {
      const int row = idx / S::kVec, qv = idx - row * S::kVec;   // row = slot * 16 + r
      *reinterpret_cast<f4*>(buf + L::kAlpha + row * G::kRow + 4 * qv) = pf.alpha[k];
    }
  });
  if (tid < Plan::kChunk * 16) buf[L::kBias + tid] = pf.bias;
}

// Whether first-input entry e is the output (kOut) or first input (!kOut)
// of some path.
template <class Plan, bool kOut>
constexpr bool entry_used(int e) {
  for (int p = 0; p < Plan::kPaths; ++p)
    if ((kOut ? Plan::paths[p].k : Plan::paths[p].i) == e) return true;
  return false;
}

// Shared uvu weights W[p][u] (V = 1) of channel tile u0, all paths: [P][16].
template <class Plan, int NT>
__device__ __forceinline__ void stage_shared_weights(float* dst, const Args& a, int u0) {
  for (int idx = threadIdx.x; idx < Plan::kPaths * 16; idx += NT)
    dst[idx] = a.alpha[(idx >> 4) * a.C + u0 + (idx & 15)];
}

template <int Dim>
__device__ __forceinline__ void store_zero_entry(__amdgpu_buffer_rsrc_t r, uint32_t row_off,
                                                 int off_c, int u) {
  const float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  store_entry<Dim>(r, row_off, off_c, u, z);
}

// Where the (edge, path, channel) weights come from: kAffineW, generated on
// the matrix cores from hidden and alpha (the radial product); kSharedW, the
// uvu product with shared weights (V = 1): a.alpha holds [P][C], staged per
// channel tile; kRowW, the uvu product with per-row weights (V = 1): a.alpha
// holds [n][P*C], each lane reading its edge's 4 channels of a path from
// memory.  The last two have no hidden, no bias and no matrix work.
constexpr int kAffineW = 0, kSharedW = 1, kRowW = 2;

// kRowW: a lane's weight loads run this many paths ahead of their use, in a
// ring of registers refilled per channel tile (position q uses slot q mod
// kRowAhead; the ring restarts at each tile, one load latency per tile).
constexpr int kRowAhead = 2;

// kRowW: the block's 4 wave pairs form 4 / row_pairs(C) edge groups of 16
// edges, and the row_pairs(C) pairs of a group take its 32-channel tiles
// round-robin.  A group then reads up to 512 contiguous bytes of each
// (edge, path) weight segment together and a block's weights are whole
// consecutive rows (2 MB at C128 m4 full), instead of 4 edge groups each
// revisiting its rows once per 32-channel tile.
__host__ __device__ constexpr int row_pairs(int C) { return C >= 128 ? 4 : (C >= 64 ? 2 : 1); }

// kRowW: what wave `wave` of block `block` (`waves` per block) covers: edges
// [e0, e0 + 16) and, within the block's channel span [u_begin, u_end), the
// 16 channels at u0 + 32 sub + 16 half of each round u0 = u_begin,
// u_begin + 32 pairs, ... that start below u_end.
struct RowWave {
  int64_t e0;
  int sub;    // the wave's pair among the edge group's pairs
  int pairs;  // pairs per edge group: row_pairs(C)
  int half;   // 16-channel half of the pair's 32-channel tile
};

__host__ __device__ constexpr RowWave row_wave(int C, int64_t block, int wave, int waves) {
  const int pairs = row_pairs(C);
  return RowWave{(block * ((waves / 2) / pairs) + (wave >> 1) / pairs) * kEdgesPerWave,
                 (wave >> 1) % pairs, pairs, wave & 1};
}

// kRowW: cache policy of the per-row weight-adjoint stores.  Default
// (write-back) lets L2 merge the two halves of a 128-byte line that the two
// waves of a pair write at about the same time; non-temporal 16-byte stores
// (2) measured 10% slower.
constexpr int kRowDwPolicy = 0;

// Ring slot refill at traversal position q: the weights of position q +
// kRowAhead of this channel tile.
template <class Plan, bool kBwd, int q>
__device__ __forceinline__ void row_refill(f4 (&ring)[kRowAhead], __amdgpu_buffer_rsrc_t rw,
                                           uint32_t wrow, int C) {
  constexpr int qn = q + kRowAhead;
  if constexpr (qn < Plan::kPaths)
    ring[q % kRowAhead] = ld4(rw, wrow + (uint32_t)(path_at<Plan, kBwd>(qn) * C) * 4u);
}

// kRowW ring at the start of a channel tile: positions 0 .. kRowAhead-1.
template <class Plan, bool kBwd>
__device__ __forceinline__ void row_prologue(f4 (&ring)[kRowAhead], __amdgpu_buffer_rsrc_t rw,
                                             uint32_t wrow, int C) {
  static_for<kRowAhead>([&](auto dc) __attribute__((always_inline)) {
    constexpr int d = decltype(dc)::value;
    if constexpr (d < Plan::kPaths)
      ring[d] = ld4(rw, wrow + (uint32_t)(path_at<Plan, kBwd>(d) * C) * 4u);
  });
}

template <class Plan, int KH, int kMode = kAffineW>
__global__ __launch_bounds__(64 * kSFwdWaves, 1) void radial_forward_streamed_kernel(Args a,
                                                                                   float* out) {
  constexpr int NT = 64 * kSFwdWaves;
  using G = Geom<KH>;
  using L = SLayout<Plan, KH>;
  constexpr int P = Plan::kPaths;
  constexpr int NC = Plan::kComps1;
  constexpr int PC = Plan::kChunk;
  constexpr int NCH = L::kChunks;
  __shared__ __attribute__((aligned(16))) float s_mem[L::kFloats];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
  const int g = lane >> 4, j = lane & 15;
  // kRowW: waves in pairs; the two waves of a pair take the two 16-channel
  // halves of a 32-channel tile, so the two halves of each 128-byte line of a
  // row's weights are read by one CU at about the same time (one 16-channel
  // tile per pass read every line twice from HBM).  Pairs sharing an edge
  // group (row_pairs) take its tiles round-robin, slot `rsub`.
  const RowWave wmap = row_wave(a.C, blockIdx.x, wave, NT / 64);
  const int half = kMode == kRowW ? wmap.half : 0;
  const int rpg = kMode == kRowW ? wmap.pairs : 1;
  const int rsub = kMode == kRowW ? wmap.sub : 0;
  const int64_t e0 = kMode == kRowW ? wmap.e0
                                    : ((int64_t)blockIdx.x * (NT / 64) + wave) * kEdgesPerWave;
  const int64_t rows = a.n - e0 < kEdgesPerWave ? a.n - e0 : kEdgesPerWave;
  const auto rx = x_rsrc(a, e0, rows);
  const auto ry = rows_rsrc(a.y, e0, a.W2, rows);
  const auto rh = rows_rsrc(a.hidden, e0, a.H, rows);
  const auto ro = rows_rsrc(out, e0, a.W1, rows);
  const auto rw = rows_rsrc(a.alpha, e0, P * a.C, rows);  // kRowW: the rows' weights
  const uint32_t xrow = (uint32_t)(j * a.W1) * 4u;  // edge row (out)
  const uint32_t xsrc = x_row_off(a, e0, rows, j);  // first-input row

  for (int idx = threadIdx.x; idx < P * 8; idx += NT) s_mem[L::kCoef + idx] = a.coef[idx];
  float hid[KH];
  if constexpr (kMode == kAffineW) load_hidden<KH>(rh, a.H, g, j, hid);
  float yv[Plan::kComps2];
  static_for<Plan::kComps2>([&](auto cc) __attribute__((always_inline)) {
    constexpr int c = decltype(cc)::value;
    yv[c] = ld1(ry, (uint32_t)(j * a.W2 + c) * 4u);
  });

  const int u_begin = blockIdx.y * a.tile_span;
  const int u_end = u_begin + a.tile_span < a.C ? u_begin + a.tile_span : a.C;
  SChunk<Plan, KH, NT> pf;
  if constexpr (kMode == kAffineW) {
    chunk_fetch<Plan, KH, NT, false, 0>(pf, a, u_begin);
    chunk_commit<Plan, KH, NT>(pf, s_mem + L::kBuf0);
  }
  f4 ring[kRowAhead];
  constexpr int ND1 = dim1_before<Plan>(Plan::kEntries1);
  float xcarry[4 * (ND1 > 0 ? ND1 : 1)] = {};
  int parity = 0;  // LDS buffer of the current chunk
  for (int u0 = u_begin; u0 < u_end; u0 += (kMode == kRowW ? 32 * rpg : 16)) {
    __syncthreads();
    if constexpr (kMode == kSharedW) {
      stage_shared_weights<Plan, NT>(s_mem + L::kBuf0, a, u0);
      __syncthreads();
    }
    const int ut = u0 + 32 * rsub;  // this pair's 32-channel tile (kRowW; u0 otherwise)
    if (kMode == kRowW && ut + 16 * half >= u_end) continue;  // wave-uniform; barriers stay paired
    const int u = ut + 16 * half + 4 * g;
    const uint32_t wrow = (uint32_t)(j * P * a.C + u) * 4u;  // kRowW: path 0 of this lane
    if constexpr (kMode == kRowW) row_prologue<Plan, false>(ring, rw, wrow, a.C);
    // kRowW: the two waves of a pair read both halves of a line already.
    const TilePair tp = tile_pair(kMode != kRowW, u0, u_begin, u_end);
    float xv[4 * NC];
    load_row_paired<Plan>(rx, xsrc, a.C, u, xv, xcarry, tp);
    static_for<Plan::kEntries1>([&](auto ec) __attribute__((always_inline)) {
      constexpr int e = decltype(ec)::value;
      constexpr REntry O = Plan::e1[e];
      if constexpr (!entry_used<Plan, true>(e)) store_zero_entry<O.dim>(ro, xrow, O.off * a.C, u);
    });
    float ov[8];
    static_for<NCH>([&](auto cc) __attribute__((always_inline)) {
      constexpr int c = decltype(cc)::value;
      if constexpr (kMode == kAffineW) {
        if constexpr (c + 1 < NCH) {
          chunk_fetch<Plan, KH, NT, false, c + 1>(pf, a, u0);
        } else {
          if (u0 + 16 < u_end) chunk_fetch<Plan, KH, NT, false, 0>(pf, a, u0 + 16);
        }
      }
      const int buf = L::kBuf0 + parity * L::kBufFloats;
      // Laundered per chunk so that neither addresses nor the uniform
      // coupling reads are hoisted into registers across chunks.
      int coef_off = L::kCoef, bias_off = buf + L::kBias + 4 * g;
      int arow_off = buf + L::kAlpha + j * G::kRow + KH * g, wsh_off = L::kBuf0 + 4 * g;
      asm volatile("" : "+v"(coef_off), "+v"(bias_off), "+v"(arow_off), "+v"(wsh_off));
      const float* cf = s_mem + coef_off;
      constexpr int kCount = (P - c * PC < PC ? P - c * PC : PC);
      // Next path's weight tile generated beside this path's products, as in
      // the input adjoints, where the forward already holds more than 128
      // registers (one block of two waves per SIMD either way); small rows
      // (4 kComps1 + kComps2 <= 45) keep 128 and two blocks per CU instead.
      constexpr bool kPipe = kMode == kAffineW && 4 * NC + Plan::kComps2 > 45;
      f4 wn;
      if constexpr (kPipe) wn = weight_tile<KH>(s_mem, bias_off, arow_off, 0, hid);
      static_for<kCount>([&](auto sc) __attribute__((always_inline)) {
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
        f4 w;
        if constexpr (kMode == kSharedW) w = *reinterpret_cast<const f4*>(s_mem + wsh_off + p * 16);
        else if constexpr (kMode == kRowW) {
          w = ring[q % kRowAhead];
          row_refill<Plan, false, q>(ring, rw, wrow, a.C);
        }
        else if constexpr (kPipe) {
          w = wn;
          if constexpr (slot + 1 < kCount)
            wn = weight_tile<KH>(s_mem, bias_off, arow_off, slot + 1, hid);
        } else {
          w = weight_tile<KH>(s_mem, bias_off, arow_off, slot, hid);
        }
        const auto cfs = load_coefs<ps.mask>(cf, p);
        static_for<8>([&](auto sc2) __attribute__((always_inline)) {
          constexpr int sl = decltype(sc2)::value;
          constexpr int oc = sl >> 2, ia = (sl >> 1) & 1, ib = sl & 1;
          if constexpr ((ps.mask >> sl) & 1) {
            const float cy = coef_at<sl>(cfs) * yv[Y.base + ib];
            static_for<4>([&](auto rc) __attribute__((always_inline)) {
              constexpr int r = decltype(rc)::value;
              ov[r * O.dim + oc] += cy * (xv[4 * X.base + r * X.dim + ia] * w[r]);
            });
          }
        });
        // Pinned per path: left alone, the compiler sinks the accumulation
        // chain towards the entry's store and keeps every product live.
#pragma unroll
        for (int i = 0; i < 4 * O.dim; ++i) asm volatile("" : "+v"(ov[i]));
        if constexpr (last) store_entry<O.dim>(ro, xrow, O.off * a.C, u, ov);
      });
      if constexpr (kMode == kAffineW) {
        if (c + 1 < NCH || u0 + 16 < u_end)
          chunk_commit<Plan, KH, NT>(pf, s_mem + L::kBuf0 + (parity ^ 1) * L::kBufFloats);
        parity ^= 1;
        __syncthreads();
      }
    });
  }
}

// needed: 1 = x, 2 = y, 4 = hidden (kAffineW) or the per-row weights (kRowW,
// written to ghid as [n][P*C]; kSharedW ignores it).
template <class Plan, int KH, int kMode = kAffineW>
__global__ __launch_bounds__(64 * kSBwdWaves, 1) void radial_backward_streamed_kernel(
    Args a, const float* gout, float* gx, float* gy, float* ghid, int needed) {
  constexpr int NT = 64 * kSBwdWaves;
  using G = Geom<KH>;
  using L = SLayout<Plan, KH>;
  constexpr int P = Plan::kPaths;
  constexpr int NC = Plan::kComps1;
  constexpr int NY = Plan::kComps2;
  constexpr int PC = Plan::kChunk;
  constexpr int NCH = L::kChunks;
  __shared__ __attribute__((aligned(16))) float s_mem[L::kFloats];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
  const int g = lane >> 4, j = lane & 15;
  // kRowW: waves in pairs; the two waves of a pair take the two 16-channel
  // halves of a 32-channel tile, so the two halves of each 128-byte line of a
  // row's weights are read by one CU at about the same time (one 16-channel
  // tile per pass read every line twice from HBM).  Pairs sharing an edge
  // group (row_pairs) take its tiles round-robin, slot `rsub`.
  const RowWave wmap = row_wave(a.C, blockIdx.x, wave, NT / 64);
  const int half = kMode == kRowW ? wmap.half : 0;
  const int rpg = kMode == kRowW ? wmap.pairs : 1;
  const int rsub = kMode == kRowW ? wmap.sub : 0;
  const int64_t e0 = kMode == kRowW ? wmap.e0
                                    : ((int64_t)blockIdx.x * (NT / 64) + wave) * kEdgesPerWave;
  const int64_t rows = a.n - e0 < kEdgesPerWave ? a.n - e0 : kEdgesPerWave;
  const auto rx = x_rsrc(a, e0, rows);
  const auto rg = rows_rsrc(gout, e0, a.W1, rows);
  const auto ry = rows_rsrc(a.y, e0, a.W2, rows);
  const auto rh = rows_rsrc(a.hidden, e0, a.H, rows);
  const uint32_t xrow = (uint32_t)(j * a.W1) * 4u;  // edge row (g, dx)
  const uint32_t xsrc = x_row_off(a, e0, rows, j);  // first-input row
  const bool need_y = (needed & 2) != 0;
  const auto rdx = rows_rsrc(gx, e0, a.W1, (needed & 1) ? rows : 0);
  // dy / dhidden: this block's channel split only, as partials, when the
  // channels are split over grid y.
  float* dy_base = a.part_dy ? a.part_dy + (int64_t)blockIdx.y * a.n * a.W2 : gy;
  const auto rgh = rows_rsrc(a.part_gh ? a.part_gh + (int64_t)blockIdx.y * a.n * a.H : ghid, e0,
                             a.H, (needed & 4) ? rows : 0);
  // kRowW: the rows' weights, and their adjoint in ghid ([n][P*C]) for bit 4.
  const auto rw = rows_rsrc(a.alpha, e0, P * a.C, rows);
  const bool need_w = (needed & 4) != 0;
  const auto rdw = rows_rsrc(ghid, e0, P * a.C, need_w ? rows : 0);

  for (int idx = threadIdx.x; idx < P * 8; idx += NT) s_mem[L::kCoef + idx] = a.coef[idx];
  float hid[KH];
  if constexpr (kMode == kAffineW) load_hidden<KH>(rh, a.H, g, j, hid);
  float yv[NY], dyv[NY];
  static_for<NY>([&](auto cc) __attribute__((always_inline)) {
    constexpr int c = decltype(cc)::value;
    yv[c] = ld1(ry, (uint32_t)(j * a.W2 + c) * 4u);
    dyv[c] = 0.f;
  });
  f4 gh[G::kTiles];
  static_for<G::kTiles>([&](auto tc) __attribute__((always_inline)) { gh[decltype(tc)::value] = f4{0.f, 0.f, 0.f, 0.f}; });

  const int u_begin = blockIdx.y * a.tile_span;
  const int u_end = u_begin + a.tile_span < a.C ? u_begin + a.tile_span : a.C;
  SChunk<Plan, KH, NT> pf;
  if constexpr (kMode == kAffineW) {
    chunk_fetch<Plan, KH, NT, true, 0>(pf, a, u_begin);
    chunk_commit<Plan, KH, NT>(pf, s_mem + L::kBuf0);
  }
  f4 ring[kRowAhead];
  constexpr int ND1 = dim1_before<Plan>(Plan::kEntries1);
  // Tile pairing carries 4 registers per one-component entry for x and for
  // g.  Taken where it costs no occupancy or spill: the affine mode with one
  // such entry (canonical first input) and a small row state (m_max <= 4
  // canonical, and m_max 5 canonical x canonical).
  constexpr bool kPair = kMode == kAffineW && ND1 == 1 && 4 * NC + 2 * NY <= 72;
  float gcarry[4 * (ND1 > 0 ? ND1 : 1)] = {}, xcarry[4 * (ND1 > 0 ? ND1 : 1)] = {};
  int parity = 0;
  for (int u0 = u_begin; u0 < u_end; u0 += (kMode == kRowW ? 32 * rpg : 16)) {
    __syncthreads();
    if constexpr (kMode == kSharedW) {
      stage_shared_weights<Plan, NT>(s_mem + L::kBuf0, a, u0);
      __syncthreads();
    }
    const int ut = u0 + 32 * rsub;  // this pair's 32-channel tile (kRowW; u0 otherwise)
    if (kMode == kRowW && ut + 16 * half >= u_end) continue;  // wave-uniform; barriers stay paired
    const int u = ut + 16 * half + 4 * g;
    const uint32_t wrow = (uint32_t)(j * P * a.C + u) * 4u;  // kRowW: path 0 of this lane
    if constexpr (kMode == kRowW) row_prologue<Plan, true>(ring, rw, wrow, a.C);
    const TilePair tp = tile_pair(kPair, u0, u_begin, u_end);
    float gv[4 * NC];
    load_row_paired<Plan>(rg, xrow, a.C, u, gv, gcarry, tp);
    static_for<Plan::kEntries1>([&](auto ec) __attribute__((always_inline)) {
      constexpr int e = decltype(ec)::value;
      constexpr REntry X = Plan::e1[e];
      if constexpr (!entry_used<Plan, false>(e)) store_zero_entry<X.dim>(rdx, xrow, X.off * a.C, u);
    });
    // x entry of the current first-input group, and of the next one (loaded a
    // group ahead of its use).
    float xc[8], xn[8], dxc[8];
    {
      constexpr int i0 = Plan::paths[Plan::bwd[0]].i;
      constexpr REntry X0 = Plan::e1[i0];
      load_entry_paired<X0.dim>(rx, xsrc, X0.off * a.C, u, xn, xcarry + 4 * dim1_before<Plan>(i0),
                                tp);
    }
    static_for<NCH>([&](auto cc) __attribute__((always_inline)) {
      constexpr int c = decltype(cc)::value;
      if constexpr (kMode == kAffineW) {
        if constexpr (c + 1 < NCH) {
          chunk_fetch<Plan, KH, NT, true, c + 1>(pf, a, u0);
        } else {
          if (u0 + 16 < u_end) chunk_fetch<Plan, KH, NT, true, 0>(pf, a, u0 + 16);
        }
      }
      const int buf = L::kBuf0 + parity * L::kBufFloats;
      int coef_off = L::kCoef, bias_off = buf + L::kBias + 4 * g;
      int arow_off = buf + L::kAlpha + j * G::kRow + KH * g;
      int acol_off = buf + L::kAlpha + 4 * g * G::kRow + j, wsh_off = L::kBuf0 + 4 * g;
      asm volatile("" : "+v"(coef_off), "+v"(bias_off), "+v"(arow_off), "+v"(acol_off),
                   "+v"(wsh_off));
      const float* cf = s_mem + coef_off;
      constexpr int kCount = (P - c * PC < PC ? P - c * PC : PC);
      // kAffineW: the weight tile of the chunk's next path is generated while
      // this path's products run (its MFMAs interleave with their VALU work;
      // 3-6% faster input adjoints).  The chunk's first tile has no
      // predecessor: the chunk's alpha is only in LDS after the barrier.
      f4 wn;
      if constexpr (kMode == kAffineW) wn = weight_tile<KH>(s_mem, bias_off, arow_off, 0, hid);
      static_for<kCount>([&](auto sc) __attribute__((always_inline)) {
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
            // First position of the next group.
            constexpr int qn = [] {
              int t = q + 1;
              while (t < P && Plan::paths[Plan::bwd[t]].i == Plan::paths[Plan::bwd[q]].i) ++t;
              return t;
            }();
            if constexpr (qn < P) {
              constexpr int in = Plan::paths[Plan::bwd[qn]].i;
              constexpr REntry XN = Plan::e1[in];
              load_entry_paired<XN.dim>(rx, xsrc, XN.off * a.C, u, xn,
                                        xcarry + 4 * dim1_before<Plan>(in), tp);
            }
          }
        }
        f4 w;
        if constexpr (kMode == kSharedW) w = *reinterpret_cast<const f4*>(s_mem + wsh_off + p * 16);
        else if constexpr (kMode == kRowW) {
          w = ring[q % kRowAhead];
          row_refill<Plan, true, q>(ring, rw, wrow, a.C);
        }
        else {
          w = wn;
          if constexpr (slot + 1 < kCount)
            wn = weight_tile<KH>(s_mem, bias_off, arow_off, slot + 1, hid);
        }
        // Per channel row r: G = g w per output component (shared by the
        // path's slots), T = sum of cy x per output component (gw = g . T),
        // and the dy contribution of a slot summed over the 4 rows before its
        // one coupling multiply.
        float G[2][4], T[2][4];
        static_for<O.dim>([&](auto occ) __attribute__((always_inline)) {
          constexpr int oc = decltype(occ)::value;
          static_for<4>([&](auto rc) __attribute__((always_inline)) {
            constexpr int r = decltype(rc)::value;
            G[oc][r] = gv[4 * O.base + r * O.dim + oc] * w[r];
            T[oc][r] = 0.f;
          });
        });
        const auto cfs = load_coefs<ps.mask>(cf, p);
        static_for<8>([&](auto sc2) __attribute__((always_inline)) {
          constexpr int sl = decltype(sc2)::value;
          constexpr int oc = sl >> 2, ia = (sl >> 1) & 1, ib = sl & 1;
          if constexpr ((ps.mask >> sl) & 1) {
            const float cfv = coef_at<sl>(cfs);
            const float cy = cfv * yv[Y.base + ib];
            float dsum = 0.f;
            static_for<4>([&](auto rc) __attribute__((always_inline)) {
              constexpr int r = decltype(rc)::value;
              const float xr = xc[r * X.dim + ia];
              T[oc][r] += cy * xr;
              dxc[r * X.dim + ia] += cy * G[oc][r];
              dsum += xr * G[oc][r];
            });
            dyv[Y.base + ib] += cfv * dsum;
          }
        });
        float gw[4];
        static_for<4>([&](auto rc) __attribute__((always_inline)) {
          constexpr int r = decltype(rc)::value;
          gw[r] = gv[4 * O.base + r * O.dim] * T[0][r];
          if constexpr (O.dim == 2) gw[r] += gv[4 * O.base + r * O.dim + 1] * T[1][r];
        });
        // Pinned per path (see the forward): unpinned, the dy and dx chains
        // are sunk towards their stores with all their products live.
        asm volatile("" : "+v"(dyv[Y.base]));
        if constexpr (Y.dim == 2) asm volatile("" : "+v"(dyv[Y.base + 1]));
#pragma unroll
        for (int i = 0; i < 4 * X.dim; ++i) asm volatile("" : "+v"(dxc[i]));
        if constexpr (kMode == kRowW) {
          if (need_w) {
            __builtin_amdgcn_raw_buffer_store_b128(
                __builtin_bit_cast(u32x4, f4{gw[0], gw[1], gw[2], gw[3]}), rdw,
                (int)(wrow + (uint32_t)(p * a.C) * 4u), 0, kRowDwPolicy);
          }
        }
        if constexpr (kMode == kAffineW) {
          const float* acol = s_mem + acol_off + slot * 16 * G::kRow;
          static_for<G::kTiles>([&](auto tc) __attribute__((always_inline)) {
            constexpr int t = decltype(tc)::value;
            gh[t] = mfma(acol[16 * t], gw[0], gh[t]);
            gh[t] = mfma(acol[G::kRow + 16 * t], gw[1], gh[t]);
            gh[t] = mfma(acol[2 * G::kRow + 16 * t], gw[2], gh[t]);
            gh[t] = mfma(acol[3 * G::kRow + 16 * t], gw[3], gh[t]);
          });
        }
        if constexpr (last) store_entry<X.dim>(rdx, xrow, X.off * a.C, u, dxc);
        __builtin_amdgcn_sched_barrier(0);
      });
      if constexpr (kMode == kAffineW) {
        if (c + 1 < NCH || u0 + 16 < u_end)
          chunk_commit<Plan, KH, NT>(pf, s_mem + L::kBuf0 + (parity ^ 1) * L::kBufFloats);
        parity ^= 1;
        __syncthreads();
      }
    });
  }
  if (need_y) {
    // Lanes j, j+16, j+32, j+48 hold the channel partial sums of edge j.
    static_for<NY>([&](auto cc) __attribute__((always_inline)) {
      constexpr int c = decltype(cc)::value;
      dyv[c] += __shfl_xor(dyv[c], 16);
      dyv[c] += __shfl_xor(dyv[c], 32);
    });
    if constexpr (kMode == kRowW) {
      static_assert((NT / 64) * 16 * NY <= 2 * L::kBufFloats, "dy exchange fits the buffers");
      // Every wave of an edge group but its first hands its channels' sums to
      // the first, which adds them in wave order (a fixed order).
      float* s_dy = s_mem + L::kBuf0;
      const int lead = wave - 2 * rsub - half;  // first wave of this edge group
      if (wave != lead && g == 0)
        static_for<NY>([&](auto cc) __attribute__((always_inline)) { s_dy[(wave * 16 + j) * NY + decltype(cc)::value] = dyv[decltype(cc)::value]; });
      __syncthreads();
      if (wave == lead)
        for (int k = 1; k < 2 * rpg; ++k)
          static_for<NY>([&](auto cc) __attribute__((always_inline)) { dyv[decltype(cc)::value] += s_dy[((lead + k) * 16 + j) * NY + decltype(cc)::value]; });
    }
    if (g == 0 && j < rows && half == 0 && rsub == 0) {
      float* dst = dy_base + (e0 + j) * a.W2;
      static_for<NY>([&](auto cc) __attribute__((always_inline)) { dst[decltype(cc)::value] = dyv[decltype(cc)::value]; });
    }
  }
  if constexpr (kMode == kAffineW)
    static_for<G::kTiles>([&](auto tc) __attribute__((always_inline)) {
      constexpr int t = decltype(tc)::value;
      const int h = 16 * t + 4 * g;
      st4(rgh, gh[t], h < a.H ? (uint32_t)(j * a.H + h) * 4u : kIdle);
    });
}

// Affine-parameter adjoints of a structure with many paths (dalpha = gw^T
// hidden, dbias = sum_e gw).  Same staged tiles as radial_weight_kernel, but
// each wave owns Plan::kWgtPaths (up to 8) consecutive paths of Plan::wgt
// (grouped by second-input entry): their dalpha tiles, 64 hidden x 16
// channels each, stay in registers, and per step the wave reads from LDS only
// the operand components its paths use (about a third at 254 paths).  8 waves
// of 8 paths: two waves per SIMD, 19% faster than 4 waves of 16 paths (one
// wave per SIMD, half the LDS reads per MFMA).
constexpr int kSWgtWaves = 8;

// The tile of this kernel: even x row stride (64-bit operand reads).
template <class Plan, int KH>
using SWTile = WTile<Plan, KH, 64 * kSWgtWaves, 2>;

template <class Plan>
constexpr int wgt_group_paths() {
  return kSWgtWaves * Plan::kWgtPaths;  // paths per block (grid z)
}

template <class Plan>
constexpr int wgt_groups() {
  return (Plan::kPaths + wgt_group_paths<Plan>() - 1) / wgt_group_paths<Plan>();
}

// Whether a path at positions [q0, q0 + n) of Plan::wgt uses entry e as its
// first input (role 0), second input (1) or output (2).
template <class Plan, int Role>
constexpr bool wgt_uses(int q0, int n, int e) {
  for (int q = q0; q < q0 + n && q < Plan::kPaths; ++q) {
    const RPath ps = Plan::paths[Plan::wgt[q]];
    if ((Role == 0 ? ps.i : Role == 1 ? ps.j : ps.k) == e) return true;
  }
  return false;
}

template <class Plan, int KH, int Q0, int NPW>
__device__ __forceinline__ void wgt_step(const float* buf, int edge, int j,
                                         f4 (&ga)[Plan::kWgtPaths][Geom<KH>::kTiles],
                                         float (&gb)[Plan::kWgtPaths]) {
  using G = Geom<KH>;
  using T = SWTile<Plan, KH>;
  const float* sx = buf;
  const float* sg = buf + T::kX;
  const float* sy = buf + 2 * T::kX;
  const float* sh = sy + T::kY;
  float xv[Plan::kComps1], gv[Plan::kComps1], yv[Plan::kComps2], hv[G::kTiles];
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
  static_for<Plan::kEntries2>([&](auto ec) __attribute__((always_inline)) {
    constexpr int e = decltype(ec)::value;
    constexpr REntry E = Plan::e2[e];
    if constexpr (wgt_uses<Plan, 1>(Q0, NPW, e))
      static_for<E.dim>([&](auto dc) __attribute__((always_inline)) {
        constexpr int d = decltype(dc)::value;
        yv[E.base + d] = sy[edge * T::kYS + E.base + d];
      });
  });
  static_for<G::kTiles>([&](auto tc) __attribute__((always_inline)) {
    hv[decltype(tc)::value] = sh[edge * T::kHS + 16 * decltype(tc)::value + j];
  });
  static_for<NPW>([&](auto qc) __attribute__((always_inline)) {
    constexpr int q = decltype(qc)::value;
    constexpr int p = Plan::wgt[Q0 + q];
    constexpr RPath ps = Plan::paths[p];
    constexpr REntry X = Plan::e1[ps.i];
    constexpr REntry Y = Plan::e2[ps.j];
    constexpr REntry O = Plan::e1[ps.k];
    // The path's weight adjoint divided by its coupling magnitude: the
    // couplings' signs are compiled, the magnitude is applied once to the
    // finished sums (wgt_body), so no coupling is read per step.
    // Per output component T = sum of the signed x y products (shared by the
    // paths of one (first, second) entry pair), gw = sum of g T.
    float gw = 0.f;
    static_for<O.dim>([&](auto occ) __attribute__((always_inline)) {
      constexpr int c = decltype(occ)::value;
      float t = 0.f;
      static_for<4>([&](auto sc) __attribute__((always_inline)) {
        constexpr int slot = c * 4 + decltype(sc)::value;
        constexpr int ia = (slot >> 1) & 1, ib = slot & 1;
        if constexpr ((ps.mask >> slot) & 1) {
          const float xy = xv[X.base + ia] * yv[Y.base + ib];
          if constexpr ((ps.neg >> slot) & 1)
            t -= xy;
          else
            t += xy;
        }
      });
      gw += gv[O.base + c] * t;
    });
    gb[q] += gw;
    static_for<G::kTiles>([&](auto tc) __attribute__((always_inline)) {
      constexpr int tt = decltype(tc)::value;
      ga[q][tt] = mfma(hv[tt], gw, ga[q][tt]);
    });
  });
}

// Direct-to-LDS staging of the affine-adjoint tiles.  buffer_load ... lds
// writes the 64 floats of one wave instruction to consecutive LDS words from
// a wave-uniform address (lane l at +4l bytes), so a tile moves from memory
// to LDS without passing through registers: the tile size costs no registers
// and there is no separate commit.  The x and g parts of an edge are 16 NC
// floats at edge * kXS (kChunks 64-float chunks, the last one masked to its
// kLast valid lanes); y is the tile's contiguous rows (masked past the tile);
// hidden is one 64-float chunk per edge (zero past a.H).  The chunks are
// dealt to the waves round-robin.  Completion is counted by vmcnt: the tile
// is complete once every wave has waited for vmcnt(0) and passed a barrier.
template <class Plan>
struct WDma {
  static constexpr int kXE = 16 * Plan::kComps1;         // x (or g) floats per edge
  static constexpr int kChunks = (kXE + 63) / 64;         // 64-float chunks per edge
  static constexpr int kLast = kXE - 64 * (kChunks - 1);  // valid lanes of the last chunk
};

// Byte offset of this lane's element of every chunk inside an edge's row (the
// same for every edge and tile of a block; kIdle for the masked lanes).
template <class Plan>
__device__ __forceinline__ void wgt_dma_cols(uint32_t (&col)[WDma<Plan>::kChunks], const Args& a,
                                             int u0, int lane) {
  static_for<WDma<Plan>::kChunks>([&](auto kc) __attribute__((always_inline)) {
    constexpr int k = decltype(kc)::value;
    const int idx = 64 * k + lane;
    col[k] = idx < WDma<Plan>::kXE ? (uint32_t)tile_x_offset<Plan>(idx, a.C, u0) * 4u : kIdle;
  });
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// One wave instruction: lane l's float at voff goes to dst[l] (dst uniform).
__device__ __forceinline__ void dma1(__amdgpu_buffer_rsrc_t r, float* dst, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)dst, 4, (int)voff, 0, 0, 0);
}

__device__ __forceinline__ void wait_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Descriptor of one edge row of `width` floats (empty when !valid: the row
// reads as zeros).  Built from uniform values, it lives in scalar registers,
// so the loads of a row need no per-lane address arithmetic.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const float* row, int width, bool valid) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(row), 0, valid ? width * 4 : 0,
                                           kRsrcFlags);
}

// Issues this wave's share of tile [t0, t0 + kWeightEdges) into buf.  lane4
// is the lane's byte offset (4 * lane).
template <class Plan, int KH, int NT>
__device__ __forceinline__ void wgt_dma(float* buf, const Args& a, const float* gout, int64_t t0,
                                        int64_t t_end, const uint32_t (&col)[WDma<Plan>::kChunks],
                                        int64_t rows_of_tile, int wave, int lane, uint32_t lane4) {
  using T = SWTile<Plan, KH>;
  using D = WDma<Plan>;
  constexpr int W = NT / 64;
  constexpr int E = Plan::kWeightEdges;
  static_assert(Geom<KH>::kHid == 64, "one hidden chunk per edge");
  const int64_t rows = t_end - t0 < E ? t_end - t0 : E;
  // x and g: (part, edge) pairs, one row descriptor each; rows past the tile
  // (and table rows outside the table) read as zeros.
  static_for<(2 * E + W - 1) / W>([&](auto ic) __attribute__((always_inline)) {
    const int pr = wave + W * decltype(ic)::value;
    if (pr < 2 * E) {
      const bool is_g = pr >= E;
      const int edge = is_g ? pr - E : pr;
      __amdgpu_buffer_rsrc_t r;
      if (is_g) {
        r = row_rsrc(gout + (t0 + edge) * a.W1, a.W1, edge < rows);
      } else if (a.xindex) {
        // Lane L of rows_of_tile holds the table row of edge L % 32.
        const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)(uint64_t)rows_of_tile, edge);
        const uint32_t hi = __builtin_amdgcn_readlane((int)((uint64_t)rows_of_tile >> 32), edge);
        const int64_t id = (int64_t)(((uint64_t)hi << 32) | lo);
        const bool ok = edge < rows && id >= 0 && id < a.x_rows;
        r = row_rsrc(a.x + (ok ? id : 0) * a.W1, a.W1, ok);
      } else {
        r = row_rsrc(a.x + (t0 + edge) * a.W1, a.W1, edge < rows);
      }
      float* dst = buf + (is_g ? T::kX : 0) + edge * T::kXS;
      static_for<D::kChunks>([&](auto kc) __attribute__((always_inline)) {
        constexpr int k = decltype(kc)::value;
        if (k + 1 < D::kChunks || lane < D::kLast) dma1(r, dst + 64 * k, col[k]);
      });
    }
  });
  // y: the tile's rows are contiguous.
  constexpr int kYC = (T::kY + 63) / 64;
  float* sy = buf + 2 * T::kX;
  const auto ry = rows_rsrc(a.y, t0, a.W2, rows);
  static_for<(kYC + W - 1) / W>([&](auto ic) __attribute__((always_inline)) {
    const int c = wave + W * decltype(ic)::value;
    if (c < kYC && 64 * c + lane < T::kY) dma1(ry, sy + 64 * c, (uint32_t)(256 * c) + lane4);
  });
  // hidden: one row of a.H floats per edge (zeros past a.H).
  float* sh = sy + T::kY;
  static_for<(E + W - 1) / W>([&](auto ic) __attribute__((always_inline)) {
    const int edge = wave + W * decltype(ic)::value;
    if (edge < E)
      dma1(row_rsrc(a.hidden + (t0 + edge) * a.H, a.H, edge < rows), sh + edge * T::kHS, lane4);
  });
}

template <class Plan, int KH, int G0>
__device__ __forceinline__ void wgt_body(float* s_mem, const Args& a, const float* gout,
                                         int64_t edges_per_slice, float* part_alpha,
                                         float* part_bias) {
  constexpr int NT = 64 * kSWgtWaves;
  using G = Geom<KH>;
  using T = SWTile<Plan, KH>;
  constexpr int P = Plan::kPaths;
  constexpr int kWeightEdges = Plan::kWeightEdges;
  float* s_tile = s_mem;  // two tiles (the couplings are compiled signs and magnitudes)

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
  const int g = lane >> 4, j = lane & 15;
  const int u0 = blockIdx.y * 16;
  const int64_t begin = (int64_t)blockIdx.x * edges_per_slice;
  const int64_t end = begin + edges_per_slice < a.n ? begin + edges_per_slice : a.n;
  const int tiles = end > begin ? (int)((end - begin + kWeightEdges - 1) / kWeightEdges) : 0;

  f4 ga[Plan::kWgtPaths][G::kTiles];
  float gb[Plan::kWgtPaths];
  static_for<Plan::kWgtPaths>([&](auto qc) __attribute__((always_inline)) {
    constexpr int q = decltype(qc)::value;
    gb[q] = 0.f;
    static_for<G::kTiles>([&](auto tc) __attribute__((always_inline)) {
      ga[q][decltype(tc)::value] = f4{0.f, 0.f, 0.f, 0.f};
    });
  });

  uint32_t col[WDma<Plan>::kChunks];
  wgt_dma_cols<Plan>(col, a, u0, lane);
  const uint32_t lane4 = 4u * (uint32_t)lane;
  if (tiles > 0)
    wgt_dma<Plan, KH, NT>(s_tile, a, gout, begin, end, col, tile_rows(a, begin, end), wave, lane,
                          lane4);
  int64_t next_rows = tile_rows(a, begin + kWeightEdges, end);
  wait_dma();
  __syncthreads();
  for (int t = 0; t < tiles; ++t) {
    // The next tile streams into the other buffer (read by every wave before
    // the last barrier) while this one is consumed.
    if (t + 1 < tiles) {
      const int64_t t1 = begin + (int64_t)(t + 1) * kWeightEdges;
      wgt_dma<Plan, KH, NT>(s_tile + ((t + 1) & 1) * T::kFloats, a, gout, t1, end, col,
                            next_rows, wave, lane, lane4);
      next_rows = tile_rows(a, t1 + kWeightEdges, end);
    }
    const float* buf = s_tile + (t & 1) * T::kFloats;
    // One dispatch on the wave per tile (per step it cost 8% at configs[4]).
    static_for<kSWgtWaves>([&](auto wc) __attribute__((always_inline)) {
      constexpr int w = decltype(wc)::value;
      constexpr int q0 = G0 * wgt_group_paths<Plan>() + w * Plan::kWgtPaths;
      constexpr int np = P - q0 < Plan::kWgtPaths ? P - q0 : Plan::kWgtPaths;
      if constexpr (np > 0) {
        if (wave == w) {
          // Not unrolled: unrolled, the steps' operand loads are hoisted and
          // the accumulators spill.
#pragma unroll 1
          for (int s = 0; s < kWeightEdges / 4; ++s) {
            wgt_step<Plan, KH, q0, np>(buf, 4 * s + g, j, ga, gb);
          }
        }
      }
    });
    wait_dma();
    __syncthreads();
  }

  const int64_t PC = (int64_t)P * a.C;
  float* pa = part_alpha + (int64_t)blockIdx.x * PC * a.H;
  float* pb = part_bias + (int64_t)blockIdx.x * PC;
  static_for<kSWgtWaves>([&](auto wc) __attribute__((always_inline)) {
    constexpr int w = decltype(wc)::value;
    constexpr int q0 = G0 * wgt_group_paths<Plan>() + w * Plan::kWgtPaths;
    constexpr int np = P - q0 < Plan::kWgtPaths ? P - q0 : Plan::kWgtPaths;
    if constexpr (np > 0) {
      if (wave == w) {
        static_for<np>([&](auto qc) __attribute__((always_inline)) {
          constexpr int q = decltype(qc)::value;
          const int64_t row = (int64_t)Plan::wgt[q0 + q] * a.C + u0 + j;
          constexpr int p = Plan::wgt[q0 + q];
          const float mag = fabsf(a.coef[p * 8 + first_slot(Plan::paths[p].mask)]);
          static_for<G::kTiles>([&](auto tc) __attribute__((always_inline)) {
            constexpr int tt = decltype(tc)::value;
            const int h = 16 * tt + 4 * g;
            if (h < a.H) *reinterpret_cast<f4*>(pa + row * a.H + h) = ga[q][tt] * mag;
          });
          float b = gb[q];
          b += __shfl_xor(b, 16);
          b += __shfl_xor(b, 32);
          if (g == 0) pb[row] = b * mag;
        });
      }
    }
  });
}

// Shared-weight gradient of the V = 1 uvu product over one edge slice and one
// channel tile: part[slice][p*C + u] = sum_e sum_slots coef y x g, the same
// per-(edge, channel) weight adjoint as the affine-adjoint kernels form,
// summed on the VALU.  Wave w owns ceil(P/8) consecutive paths of Plan::wgt
// (one accumulator per path and lane) and reads from LDS only the operand
// components they use; the dispatch on the wave is once per staged tile.  The
// lane's 4 edge rows are summed by shuffles at the end.  Grid (slices, C/16);
// the slice partials are summed in a fixed order afterwards.
template <class Plan, int KH>
__global__ __launch_bounds__(kThreads, 1) void uvu_shared_dw_kernel(Args a, const float* gout,
                                                                    int64_t edges_per_slice,
                                                                    float* part) {
  using TP = WithEdges<Plan, dw_edges<Plan, KH>()>;
  using T = WTile<TP, KH>;
  constexpr int P = Plan::kPaths;
  constexpr int kE = TP::kWeightEdges;
  constexpr int NPW = (P + kWaves - 1) / kWaves;
  constexpr int kCoefPad = (P * 8 + 3) / 4 * 4;
  // The first kCoefPad floats are unused (the couplings' signs are compiled);
  // they keep the tile size that dw_edges() chose for this layout.
  __shared__ __attribute__((aligned(16))) float s_mem[kCoefPad + 2 * T::kFloats];
  float* s_tile = s_mem + kCoefPad;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
  const int g = lane >> 4, j = lane & 15;
  const int u0 = blockIdx.y * 16;
  const int64_t begin = (int64_t)blockIdx.x * edges_per_slice;
  const int64_t end = begin + edges_per_slice < a.n ? begin + edges_per_slice : a.n;
  const int tiles = end > begin ? (int)((end - begin + kE - 1) / kE) : 0;

  float acc[NPW];
  static_for<NPW>([&](auto qc) __attribute__((always_inline)) { acc[decltype(qc)::value] = 0.f; });

  WCols<TP, KH> cols;
  weight_cols<TP, KH>(cols, a, u0);
  WPrefetch<TP, KH> pf;
  if (tiles > 0) {
    weight_fetch<TP, KH>(pf, a, gout, begin, end, cols, tile_rows(a, begin, end));
    weight_commit<TP, KH>(pf, s_tile);
  }
  int64_t next_rows = tile_rows(a, begin + kE, end);
  __syncthreads();
  for (int t = 0; t < tiles; ++t) {
    const bool more = t + 1 < tiles;
    if (more) {
      const int64_t t1 = begin + (int64_t)(t + 1) * kE;
      weight_fetch<TP, KH>(pf, a, gout, t1, end, cols, next_rows);
      next_rows = tile_rows(a, t1 + kE, end);
    }
    const float* buf = s_tile + (t & 1) * T::kFloats;
    const float* sx = buf;
    const float* sg = buf + T::kX;
    const float* sy = buf + 2 * T::kX;
    static_for<kWaves>([&](auto wc) __attribute__((always_inline)) {
      constexpr int w = decltype(wc)::value;
      constexpr int q0 = w * NPW;
      constexpr int np = P - q0 < NPW ? P - q0 : NPW;
      if constexpr (np > 0) {
        if (wave == w) {
#pragma unroll 1
          for (int s = 0; s < kE / 4; ++s) {
            const int edge = 4 * s + g;
            float xv[Plan::kComps1], gv[Plan::kComps1], yv[Plan::kComps2];
            static_for<Plan::kEntries1>([&](auto ec) __attribute__((always_inline)) {
              constexpr int e = decltype(ec)::value;
              constexpr REntry E = Plan::e1[e];
              constexpr bool use_x = wgt_uses<Plan, 0>(q0, np, e);
              constexpr bool use_g = wgt_uses<Plan, 2>(q0, np, e);
              static_for<E.dim>([&](auto dc) __attribute__((always_inline)) {
                constexpr int d = decltype(dc)::value;
                const int o = edge * T::kXS + 16 * E.base + j * E.dim + d;
                if constexpr (use_x) xv[E.base + d] = sx[o];
                if constexpr (use_g) gv[E.base + d] = sg[o];
              });
            });
            static_for<Plan::kEntries2>([&](auto ec) __attribute__((always_inline)) {
              constexpr int e = decltype(ec)::value;
              constexpr REntry E = Plan::e2[e];
              if constexpr (wgt_uses<Plan, 1>(q0, np, e))
                static_for<E.dim>([&](auto dc) __attribute__((always_inline)) {
                  constexpr int d = decltype(dc)::value;
                  yv[E.base + d] = sy[edge * T::kYS + E.base + d];
                });
            });
            // Per path: the signed x y products of its (first, second) entry
            // pair (shared by the pair's consecutive paths), summed per output
            // component into T, then acc += g . T.  The couplings' magnitudes
            // scale the finished sums.
            float z[2][2];
            static_for<np>([&](auto qc) __attribute__((always_inline)) {
              constexpr int q = decltype(qc)::value;
              constexpr int p = Plan::wgt[q0 + q];
              constexpr RPath ps = Plan::paths[p];
              constexpr REntry X = Plan::e1[ps.i];
              constexpr REntry Y = Plan::e2[ps.j];
              constexpr REntry O = Plan::e1[ps.k];
              constexpr bool first = q == 0 ||
                                     Plan::paths[Plan::wgt[q0 + (q == 0 ? 0 : q - 1)]].i != ps.i ||
                                     Plan::paths[Plan::wgt[q0 + (q == 0 ? 0 : q - 1)]].j != ps.j;
              if constexpr (first)
                static_for<X.dim * Y.dim>([&](auto zc) __attribute__((always_inline)) {
                  constexpr int ia = decltype(zc)::value / Y.dim, ib = decltype(zc)::value % Y.dim;
                  z[ia][ib] = xv[X.base + ia] * yv[Y.base + ib];
                });
              static_for<O.dim>([&](auto occ) __attribute__((always_inline)) {
                constexpr int c = decltype(occ)::value;
                float t = 0.f;
                static_for<4>([&](auto sc) __attribute__((always_inline)) {
                  constexpr int slot = c * 4 + decltype(sc)::value;
                  constexpr int ia = (slot >> 1) & 1, ib = slot & 1;
                  if constexpr ((ps.mask >> slot) & 1) {
                    if constexpr ((ps.neg >> slot) & 1)
                      t -= z[ia][ib];
                    else
                      t += z[ia][ib];
                  }
                });
                acc[q] += gv[O.base + c] * t;
              });
            });
          }
        }
      }
    });
    if (more) weight_commit<TP, KH>(pf, s_tile + ((t + 1) & 1) * T::kFloats);
    __syncthreads();
  }

  float* dst = part + (int64_t)blockIdx.x * P * a.C;
  static_for<kWaves>([&](auto wc) __attribute__((always_inline)) {
    constexpr int w = decltype(wc)::value;
    constexpr int q0 = w * NPW;
    constexpr int np = P - q0 < NPW ? P - q0 : NPW;
    if constexpr (np > 0) {
      if (wave == w) {
        static_for<np>([&](auto qc) __attribute__((always_inline)) {
          constexpr int q = decltype(qc)::value;
          constexpr int p = Plan::wgt[q0 + q];
          float v = acc[q];
          v += __shfl_xor(v, 16);
          v += __shfl_xor(v, 32);
          const float mag = fabsf(a.coef[p * 8 + first_slot(Plan::paths[p].mask)]);
          if (g == 0) dst[(int64_t)p * a.C + u0 + j] = v * mag;
        });
      }
    }
  });
}

// Grid (slices, C/16, wgt_groups<Plan>()).
template <class Plan, int KH>
__global__ __launch_bounds__(64 * kSWgtWaves, 1) void radial_weight_streamed_kernel(
    Args a, const float* gout, int64_t edges_per_slice, float* part_alpha, float* part_bias) {
  using T = SWTile<Plan, KH>;
  __shared__ __attribute__((aligned(16))) float s_mem[2 * T::kFloats];
  static_for<wgt_groups<Plan>()>([&](auto gc) __attribute__((always_inline)) {
    constexpr int grp = decltype(gc)::value;
    if (blockIdx.z == grp)
      wgt_body<Plan, KH, grp>(s_mem, a, gout, edges_per_slice, part_alpha, part_bias);
  });
}

}  // namespace radial
}  // namespace o2mi
