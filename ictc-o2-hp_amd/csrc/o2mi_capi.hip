// C ABI of the O(2) tensor-product library: plans, geometry, workspace and
// the fixed-order weight-adjoint reduction.  See include/ictc_o2_hp_amd.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "ictc_o2_hp_amd.h"
#include "o2mi_error.hpp"
#include "o2mi_tp_generic.hpp"
#include "o2mi_tp_launch.hpp"

// Defined by the generated registry (one entry per compiled plan).
const o2mi::TPKernelSet* o2mi_find_tp_set(int m_max, int full, int normalization);

struct o2mi_tp_plan {
  const o2mi::TPKernelSet* set;  // compiled kernels, or NULL (table-driven only)
  int channels;
  int m_max;
  int full;
  int normalization;
  int layout;
  int64_t width;
  int64_t weight_numel;
  int n_keys;
  int n_paths;
};

std::string& o2mi_error_slot() {
  thread_local std::string message;
  return message;
}

// Optional kernel timing: while enabled, every timed call records a HIP event
// pair around its main kernel on the call's stream.  Calls may come from any
// thread (the autograd engine runs backward on its own).
namespace {
std::mutex g_timing_mu;
bool g_timing = false;
std::vector<O2miTimed> g_timed;
std::vector<hipEvent_t> g_event_pool;

hipEvent_t take_event() {
  if (!g_event_pool.empty()) {
    hipEvent_t e = g_event_pool.back();
    g_event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}
}  // namespace

bool o2mi_timing_begin(hipStream_t s, O2miTimed* launch, int kind) {
  std::lock_guard<std::mutex> lock(g_timing_mu);
  if (!g_timing) return false;
  launch->kind = kind;
  launch->start = take_event();
  launch->stop = take_event();
  if (launch->start && launch->stop && hipEventRecord(launch->start, s) == hipSuccess)
    return true;
  // Untimed launch: return whatever events were taken to the pool.
  if (launch->start) g_event_pool.push_back(launch->start);
  if (launch->stop) g_event_pool.push_back(launch->stop);
  return false;
}

void o2mi_timing_end(hipStream_t s, O2miTimed* launch) {
  const bool recorded = hipEventRecord(launch->stop, s) == hipSuccess;
  std::lock_guard<std::mutex> lock(g_timing_mu);
  if (recorded) {
    g_timed.push_back(*launch);
  } else {
    g_event_pool.push_back(launch->start);
    g_event_pool.push_back(launch->stop);
  }
}

namespace {

int fail(int status, const std::string& message) {
  o2mi_error_slot() = message;
  return status;
}

int fail_hip(hipError_t err, const char* where) {
  o2mi_error_slot() = std::string(where) + ": " + hipGetErrorString(err);
  return O2MI_ERR_HIP;
}

constexpr int kReduceCols = 64;        // columns per reduction block (one per lane)
constexpr int kReduceWaves = 16;       // waves per reduction block
constexpr int kReduceOnePass = 2048;   // at most this many rows: one pass
constexpr int kReduceSplitRows = 1024; // rows per first-pass split above that

// out[s * ncols + col] = sum of in[r * ncols + col] over the rows of split s.
// Wave w adds rows r0 + w, r0 + w + 16, ... in increasing order (four loads in
// flight); the 16 wave sums are then combined in a fixed pairwise tree.  The
// order depends only on the row count: the sum is bitwise reproducible.
__global__ __launch_bounds__(kReduceWaves * 64) void column_sum_kernel(
    const float* __restrict__ in, int64_t nrows, int64_t ncols, int64_t rows_per_split,
    float* __restrict__ out) {
  __shared__ float part[kReduceWaves][kReduceCols];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t col = (int64_t)blockIdx.x * kReduceCols + lane;
  const int64_t r0 = (int64_t)blockIdx.y * rows_per_split;
  const int64_t r1 = min(nrows, r0 + rows_per_split);
  constexpr int W = kReduceWaves;
  float s = 0.f;
  if (col < ncols) {
    const float* p = in + col;
    int64_t r = r0 + wave;
    for (; r + 3 * W < r1; r += 4 * W) {
      const float a = p[r * ncols], b = p[(r + W) * ncols];
      const float c = p[(r + 2 * W) * ncols], d = p[(r + 3 * W) * ncols];
      s += a;
      s += b;
      s += c;
      s += d;
    }
    for (; r < r1; r += W) s += p[r * ncols];
  }
  part[wave][lane] = s;
  __syncthreads();
  for (int half = W / 2; half >= 1; half /= 2) {
    if (wave < half) part[wave][lane] += part[wave + half][lane];
    __syncthreads();
  }
  if (wave == 0 && col < ncols) out[(int64_t)blockIdx.y * ncols + col] = part[0][lane];
}

// First-pass splits of a fixed-order column sum over `rows` rows (1: one pass).
int64_t reduce_splits(int64_t rows) {
  return rows <= kReduceOnePass ? 1 : (rows + kReduceSplitRows - 1) / kReduceSplitRows;
}

__global__ __launch_bounds__(256) void fill_kernel(float* __restrict__ out, int64_t n, float v) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = v;
}

// Scratch of the allocation-free backward (o2mi_tp_backward_noalloc_f32): the
// dw partial rows and the reduction's second stage.  Every GPU the library
// runs on holds its own copy until the process ends.  In host code the name
// is only a stand-in: kernels get the address from scratch_address().
static __device__ __align__(256) float scratch[O2MI_TP_SCRATCH_BYTES / sizeof(float)];

// Device address of `scratch` on the current device, looked up once per
// device with hipGetSymbolAddress.
int scratch_address(float** out) {
  static std::mutex mu;
  static float* address[64] = {};
  int device = 0;
  const hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return fail_hip(err, "hipGetDevice");
  if (device < 0 || device >= 64) return fail(O2MI_ERR_INVALID_ARGUMENT, "device index above 63");
  std::lock_guard<std::mutex> lock(mu);
  if (!address[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return fail_hip(e, "hipGetSymbolAddress(scratch)");
    address[device] = static_cast<float*>(p);
  }
  *out = address[device];
  return O2MI_OK;
}

struct DeviceInfo {
  int cus = 0;
};

int device_cus() {
  static std::mutex mu;
  static DeviceInfo info[64];
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0) return 256;
  std::lock_guard<std::mutex> lock(mu);
  DeviceInfo& d = info[device & 63];
  if (d.cus == 0) {
    hipDeviceProp_t prop;
    d.cus = hipGetDeviceProperties(&prop, device) == hipSuccess ? prop.multiProcessorCount : 256;
    if (d.cus <= 0) d.cus = 256;
  }
  return d.cus;
}

int pick_variant(const o2mi_tp_plan* p, std::initializer_list<const void*> ptrs) {
  if (p->layout != O2MI_LAYOUT_CHANNEL_MAJOR) return o2mi::kVariantComponentMajor;
  // float2 accesses need every frequency element pair 8-byte aligned.
  const bool even_rows = p->full || (p->channels % 2 == 0);
  bool aligned = even_rows;
  for (const void* q : ptrs) {
    if (q && (reinterpret_cast<uintptr_t>(q) & 7u)) aligned = false;
  }
  return aligned ? o2mi::kVariantChannelMajorVec2 : o2mi::kVariantChannelMajor;
}

// Lanes per block, rows per block iteration and the grid for `n_rows` rows
// when at most `target_blocks` blocks should be resident, a block has
// `threads` threads and covers at most `tile` lanes of a row.  Blocks take
// row chunks round-robin (strided order, o2mi_tp.hpp row_schedule).
o2mi::TPGeom geometry(const o2mi_tp_plan* p, int64_t n_rows, int64_t target_blocks, int threads,
                      int tile, int* grid) {
  o2mi::TPGeom g{};
  g.n_rows = n_rows;
  g.channels = p->channels;
  g.width = (int)p->width;
  g.weight_numel = (int)p->weight_numel;
  g.lanes = p->full ? 2 * p->channels : p->channels;
  if (g.lanes <= tile) {
    g.tile_lanes = g.lanes;
    g.rows_per_iter = threads / g.lanes;
    g.tiles = 1;
  } else {
    g.tile_lanes = tile;
    g.rows_per_iter = threads / tile;
    g.tiles = (g.lanes + tile - 1) / tile;
  }
  const int64_t r = g.rows_per_iter;
  const int64_t iterations = std::max<int64_t>(1, (n_rows + r - 1) / r);
  const int64_t max_groups = std::max<int64_t>(1, target_blocks / g.tiles);
  g.groups = std::min(max_groups, iterations);
  *grid = (int)(g.groups * g.tiles);
  return g;
}

struct BackwardShape {
  o2mi::TPGeom geom;
  int grid;
  int variant;
  int64_t partial_rows;
  int64_t splits;  // first-pass reduction splits (1: a single pass)
  size_t bytes;
};

BackwardShape backward_shape_for(const o2mi_tp_plan* p, int64_t n_rows, int variant,
                                 int64_t target) {
  BackwardShape s{};
  s.variant = variant;
  s.geom = geometry(p, n_rows, target, o2mi::kBackwardBlock, p->set->backward_tile, &s.grid);
  s.partial_rows = (int64_t)(s.grid / s.geom.tiles) * s.geom.rows_per_iter;
  s.splits = reduce_splits(s.partial_rows);
  const int64_t floats = (s.partial_rows + (s.splits > 1 ? s.splits : 0)) * p->weight_numel;
  s.bytes = n_rows > 0 ? (size_t)floats * sizeof(float) : 0;
  return s;
}

// The occupancy-sized grid; with `max_bytes` set, the largest grid (fewest
// row groups removed) whose partial rows fit in max_bytes.  A shape that does
// not fit even with one row group comes back with bytes > max_bytes.
BackwardShape backward_shape(const o2mi_tp_plan* p, int64_t n_rows, int variant,
                             size_t max_bytes = SIZE_MAX) {
  const int64_t target = (int64_t)p->set->blocks_per_cu(variant, true) * device_cus();
  BackwardShape s = backward_shape_for(p, n_rows, variant, target);
  if (s.bytes <= max_bytes) return s;
  // Bytes grow with the number of row groups: bisect on it.
  const int64_t tiles = s.geom.tiles;
  int64_t lo = 1, hi = s.grid / tiles;  // lo may not fit; hi does not
  BackwardShape best = backward_shape_for(p, n_rows, variant, tiles);
  if (best.bytes > max_bytes) return best;
  while (hi - lo > 1) {
    const int64_t mid = lo + (hi - lo) / 2;
    BackwardShape t = backward_shape_for(p, n_rows, variant, mid * tiles);
    if (t.bytes <= max_bytes) {
      lo = mid;
      best = t;
    } else {
      hi = mid;
    }
  }
  return best;
}

hipError_t fill(float* out, int64_t n, float v, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(fill_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, out, n,
                     v);
  return hipGetLastError();
}

hipError_t column_sum(const float* in, int64_t nrows, int64_t ncols, int64_t splits, float* out,
                      hipStream_t stream) {
  const int64_t per_split = (nrows + splits - 1) / splits;
  dim3 grid((unsigned)((ncols + kReduceCols - 1) / kReduceCols), (unsigned)splits);
  hipLaunchKernelGGL(column_sum_kernel, grid, dim3(kReduceWaves * 64), 0, stream, in, nrows, ncols,
                     per_split,
                     out);
  return hipGetLastError();
}

// Keys of TensorProduct(C, m_max, parity) in row order (0e, [0o], 1..M) as
// (frequency, sign): scalars have frequency 0 and the parity sign.
struct HostKey {
  int m, sign;
};

std::vector<HostKey> host_keys(int m_max, bool full) {
  std::vector<HostKey> keys{{0, 1}};
  if (full) keys.push_back({0, -1});
  for (int m = 1; m <= m_max; ++m) keys.push_back({m, 0});
  return keys;
}

// Path count and packed weight count in units of C: every (k1, k2) and each
// output key of their product present in the row (the selection rules of
// o2_math.py:348-372), with mul(k3) weights per path.
void count_paths(int m_max, bool full, int* n_paths, int64_t* units) {
  const std::vector<HostKey> keys = host_keys(m_max, full);
  const int freq_units = full ? 2 : 1;
  *n_paths = 0;
  *units = 0;
  auto add = [&](HostKey k3) {
    const bool present = k3.m == 0 ? (k3.sign == 1 || full) : k3.m <= m_max;
    if (!present) return;
    *n_paths += 1;
    *units += k3.m == 0 ? 1 : freq_units;
  };
  for (const HostKey& a : keys) {
    for (const HostKey& b : keys) {
      if (a.m == 0 && b.m == 0) {
        add({0, a.sign * b.sign});
      } else if (a.m == 0 || b.m == 0) {
        add({a.m == 0 ? b.m : a.m, 0});
      } else if (a.m == b.m) {
        add({0, 1});
        add({0, -1});
        add({2 * a.m, 0});
      } else {
        add({a.m > b.m ? a.m - b.m : b.m - a.m, 0});
        add({a.m + b.m, 0});
      }
    }
  }
}

o2mi::generic::Geom generic_geom(const o2mi_tp_plan* p, int64_t n_rows) {
  o2mi::generic::Geom g{};
  g.n_rows = n_rows;
  g.weight_numel = p->weight_numel;
  g.channels = p->channels;
  g.width = (int)p->width;
  g.lanes = p->full ? 2 * p->channels : p->channels;
  g.full = p->full;
  g.layout = p->layout;
  g.n_keys = p->n_keys;
  g.n_paths = p->n_paths;
  return g;
}

struct TablesShape {
  o2mi::generic::WeightShape weight;
  int64_t splits;
  size_t bytes;
};

TablesShape tables_shape(const o2mi_tp_plan* p, int64_t n_rows) {
  TablesShape t{};
  t.weight = o2mi::generic::weight_shape(generic_geom(p, n_rows), device_cus());
  const int64_t rows = t.weight.groups;
  t.splits = reduce_splits(rows);
  const int64_t floats = (rows + (t.splits > 1 ? t.splits : 0)) * p->weight_numel;
  t.bytes = n_rows > 0 ? (size_t)floats * sizeof(float) : 0;
  return t;
}

// dw = fixed-order column sum of `rows` partial rows (one or two passes).
hipError_t reduce_partials(float* partial, int64_t rows, int64_t splits, int64_t pw, float* dw,
                           hipStream_t s) {
  if (splits == 1) return column_sum(partial, rows, pw, 1, dw, s);
  float* second = partial + rows * pw;
  hipError_t err = column_sum(partial, rows, pw, splits, second, s);
  if (err == hipSuccess) err = column_sum(second, splits, pw, 1, dw, s);
  return err;
}

// Shared body of the backward entry points.  `fit_grid`: shrink the grid so
// that the partial rows fit in `workspace_bytes` instead of failing.
int tp_backward(const o2mi_tp_plan* plan, const float* x, const float* y, const float* w,
                const float* g, float* dx, float* dy, float* dw, float* workspace,
                size_t workspace_bytes, bool fit_grid, int64_t n_rows, int needed,
                void* stream) {
  if (!plan) return fail(O2MI_ERR_INVALID_ARGUMENT, "plan is NULL");
  if (n_rows < 0) return fail(O2MI_ERR_INVALID_ARGUMENT, "n_rows must be non-negative");
  if (needed & ~7) return fail(O2MI_ERR_INVALID_ARGUMENT, "needed must be a mask of 1, 2, 4");
  if ((needed & 4) && !dw) return fail(O2MI_ERR_INVALID_ARGUMENT, "NULL dw for a requested gradient");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (n_rows == 0 || needed == 0) {
    // Empty inputs: dx and dy are empty (their pointers may be NULL), dw = 0.
    if (needed & 4) {
      const hipError_t err = fill(dw, plan->weight_numel, 0.f, s);
      if (err != hipSuccess) return fail_hip(err, "dw fill");
    }
    return O2MI_OK;
  }
  if (!x || !y || !w || !g) return fail(O2MI_ERR_INVALID_ARGUMENT, "NULL input pointer");
  if (((needed & 1) && !dx) || ((needed & 2) && !dy))
    return fail(O2MI_ERR_INVALID_ARGUMENT, "NULL output for a requested gradient");
  if (n_rows > (int64_t)INT32_MAX * 64)
    return fail(O2MI_ERR_INVALID_ARGUMENT, "n_rows too large");
  if (!plan->set)
    return fail(O2MI_ERR_UNSUPPORTED, "no compiled kernels for this plan: use o2mi_tp_backward_tables_f32");
  const int variant = pick_variant(plan, {x, y, g, (needed & 1) ? dx : nullptr,
                                          (needed & 2) ? dy : nullptr});
  const bool fit = fit_grid && (needed & 4);
  const BackwardShape shape = backward_shape(plan, n_rows, variant, fit ? workspace_bytes : SIZE_MAX);
  if (fit && shape.bytes > workspace_bytes)
    return fail(O2MI_ERR_WORKSPACE, "weight_numel too large for the backward scratch");
  if ((needed & 4) && (!workspace || workspace_bytes < shape.bytes))
    return fail(O2MI_ERR_WORKSPACE, "workspace smaller than o2mi_tp_backward_workspace_bytes");
  float* partial = workspace;
  O2miTimed timed;
  const bool timing = o2mi_timing_begin(s, &timed, O2MI_TIMED_TP_BACKWARD);
  hipError_t err = plan->set->backward(variant, x, y, w, g, dx, dy, partial, shape.geom,
                                       shape.grid, needed, s);
  if (timing) o2mi_timing_end(s, &timed);
  if (err != hipSuccess) return fail_hip(err, "tp backward launch");
  if (needed & 4) {
    err = reduce_partials(partial, shape.partial_rows, shape.splits, plan->weight_numel, dw, s);
    if (err != hipSuccess) return fail_hip(err, "dw reduction launch");
  }
  return O2MI_OK;
}

}  // namespace

extern "C" {

int o2mi_kernel_timing(int enable) {
  std::lock_guard<std::mutex> lock(g_timing_mu);
  g_timing = enable != 0;
  return O2MI_OK;
}

int o2mi_kernel_timing_read_kinds(double* ms, int* counts, int n_kinds) {
  std::vector<O2miTimed> done;
  {
    std::lock_guard<std::mutex> lock(g_timing_mu);
    done.swap(g_timed);
  }
  for (int k = 0; k < n_kinds; ++k) {
    if (ms) ms[k] = 0.0;
    if (counts) counts[k] = 0;
  }
  int status = O2MI_OK;
  for (const O2miTimed& t : done) {
    float elapsed = 0.f;
    if (hipEventSynchronize(t.stop) == hipSuccess &&
        hipEventElapsedTime(&elapsed, t.start, t.stop) == hipSuccess) {
      if (t.kind < n_kinds) {
        if (ms) ms[t.kind] += elapsed;
        if (counts) counts[t.kind] += 1;
      }
    } else {
      status = fail(O2MI_ERR_HIP, "kernel timing: event query failed");
    }
  }
  {
    std::lock_guard<std::mutex> lock(g_timing_mu);
    for (const O2miTimed& t : done) {
      g_event_pool.push_back(t.start);
      g_event_pool.push_back(t.stop);
    }
  }
  return status;
}

int o2mi_kernel_timing_read(double* forward_ms, int* forward_count, double* backward_ms,
                            int* backward_count) {
  double ms[2];
  int counts[2];
  const int status = o2mi_kernel_timing_read_kinds(ms, counts, 2);
  if (forward_ms) *forward_ms = ms[0];
  if (forward_count) *forward_count = counts[0];
  if (backward_ms) *backward_ms = ms[1];
  if (backward_count) *backward_count = counts[1];
  return status;
}

const char* o2mi_last_error(void) { return o2mi_error_slot().c_str(); }

const char* o2mi_version(void) { return "ictc_o2_hp_amd 0.1.0 (gfx950)"; }

int o2mi_tp_plan_create(int channels, int m_max, int parity, int normalization, int layout,
                        o2mi_tp_plan** plan) {
  if (!plan) return fail(O2MI_ERR_INVALID_ARGUMENT, "plan output pointer is NULL");
  *plan = nullptr;
  if (channels < 1) return fail(O2MI_ERR_INVALID_ARGUMENT, "channels must be positive");
  if (m_max < 0) return fail(O2MI_ERR_INVALID_ARGUMENT, "m_max must be non-negative");
  if (parity != O2MI_CANONICAL && parity != O2MI_FULL)
    return fail(O2MI_ERR_INVALID_ARGUMENT, "parity must be canonical (0) or full (1)");
  if (normalization != O2MI_COMPONENT && normalization != O2MI_NORM)
    return fail(O2MI_ERR_INVALID_ARGUMENT, "normalization must be component (0) or norm (1)");
  const bool full = parity == O2MI_FULL;
  const bool layout_ok = layout == O2MI_LAYOUT_CHANNEL_MAJOR ||
                         (layout == O2MI_LAYOUT_COMPONENT_MAJOR && !full) ||
                         (layout == O2MI_LAYOUT_COPY_COMPONENT_MAJOR && full);
  if (!layout_ok) return fail(O2MI_ERR_INVALID_ARGUMENT, "layout does not match the parity");
  // Without compiled kernels the plan is table-driven only
  // (o2mi_tp_forward_tables_f32 / o2mi_tp_backward_tables_f32).
  const o2mi::TPKernelSet* set = o2mi_find_tp_set(m_max, full ? 1 : 0, normalization);
  const int n_keys = (full ? 2 : 1) + m_max;
  if (!set && n_keys > o2mi::generic::max_keys())
    return fail(O2MI_ERR_UNSUPPORTED, "m_max beyond the table-driven kernels' limit");
  // Row width and packed weight count in units of C.
  const int width_units = (full ? 2 : 1) + m_max * (full ? 4 : 2);
  int n_paths = 0;
  int64_t units = 0;
  count_paths(m_max, full, &n_paths, &units);
  if (set && (set->table.n_paths != n_paths || set->table.n_units != units))
    return fail(O2MI_ERR_UNSUPPORTED, "compiled plan disagrees with the selection rules");
  o2mi_tp_plan* p = new (std::nothrow) o2mi_tp_plan;
  if (!p) return fail(O2MI_ERR_INVALID_ARGUMENT, "out of host memory");
  p->set = set;
  p->channels = channels;
  p->m_max = m_max;
  p->full = full ? 1 : 0;
  p->normalization = normalization;
  p->layout = layout;
  p->width = (int64_t)width_units * channels;
  p->weight_numel = units * channels;
  p->n_keys = n_keys;
  p->n_paths = n_paths;
  if (p->width * 8 >= (int64_t)INT32_MAX || p->weight_numel >= (int64_t)INT32_MAX / 4096) {
    delete p;
    return fail(O2MI_ERR_INVALID_ARGUMENT, "channels too large");
  }
  *plan = p;
  return O2MI_OK;
}

int o2mi_tp_plan_destroy(o2mi_tp_plan* plan) {
  delete plan;
  return O2MI_OK;
}

int o2mi_tp_plan_compiled(const o2mi_tp_plan* plan) { return plan ? (plan->set ? 1 : 0) : -1; }

int64_t o2mi_tp_width(const o2mi_tp_plan* plan) { return plan ? plan->width : -1; }

int64_t o2mi_tp_weight_numel(const o2mi_tp_plan* plan) { return plan ? plan->weight_numel : -1; }

int o2mi_tp_table(int m_max, int parity, int normalization, int* n_paths, int* n_terms,
                  int32_t* paths, float* magnitudes, int32_t* terms) {
  const o2mi::TPKernelSet* set = o2mi_find_tp_set(m_max, parity == O2MI_FULL ? 1 : 0, normalization);
  if (!set) return fail(O2MI_ERR_UNSUPPORTED, "no kernels compiled for this m_max/parity/normalization");
  const o2mi::TPTableView& t = set->table;
  if (n_paths) *n_paths = t.n_paths;
  if (n_terms) *n_terms = t.n_terms;
  for (int p = 0; p < t.n_paths; ++p) {
    const o2mi::PathSpec& ps = t.paths[p];
    if (paths) {
      int32_t* row = paths + 7 * p;
      row[0] = ps.k1;
      row[1] = ps.k2;
      row[2] = ps.k3;
      row[3] = ps.wunits;
      row[4] = ps.t0;
      row[5] = ps.nt;
      row[6] = t.keys[ps.k3].dim;
    }
    if (magnitudes) magnitudes[p] = ps.mag;
  }
  if (terms) {
    for (int n = 0; n < t.n_terms; ++n) {
      terms[4 * n + 0] = t.terms[n].i;
      terms[4 * n + 1] = t.terms[n].j;
      terms[4 * n + 2] = t.terms[n].k;
      terms[4 * n + 3] = t.terms[n].sign;
    }
  }
  return O2MI_OK;
}

int o2mi_tp_forward_f32(const o2mi_tp_plan* plan, const float* x, const float* y, const float* w,
                        float* out, int64_t n_rows, void* stream) {
  if (!plan) return fail(O2MI_ERR_INVALID_ARGUMENT, "plan is NULL");
  if (n_rows < 0) return fail(O2MI_ERR_INVALID_ARGUMENT, "n_rows must be non-negative");
  if (n_rows == 0) return O2MI_OK;
  if (!x || !y || !w || !out) return fail(O2MI_ERR_INVALID_ARGUMENT, "NULL tensor pointer");
  if (n_rows > (int64_t)INT32_MAX * 64)
    return fail(O2MI_ERR_INVALID_ARGUMENT, "n_rows too large");
  if (!plan->set)
    return fail(O2MI_ERR_UNSUPPORTED, "no compiled kernels for this plan: use o2mi_tp_forward_tables_f32");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int variant = pick_variant(plan, {x, y, out});
  const int64_t target = (int64_t)plan->set->blocks_per_cu(variant, false) * device_cus();
  int grid = 0;
  const o2mi::TPGeom g =
      geometry(plan, n_rows, target, plan->set->forward_block, plan->set->forward_tile, &grid);
  O2miTimed timed;
  const bool timing = o2mi_timing_begin(s, &timed, O2MI_TIMED_TP_FORWARD);
  const hipError_t err = plan->set->forward(variant, x, y, w, out, g, grid, s);
  if (timing) o2mi_timing_end(s, &timed);
  if (err != hipSuccess) return fail_hip(err, "tp forward launch");
  return O2MI_OK;
}

int o2mi_tp_launch_shape(const o2mi_tp_plan* plan, int64_t n_rows, int backward, int* grid,
                         int* blocks_per_cu, int* rows_per_iter, int* tiles) {
  if (!plan || n_rows < 0) return fail(O2MI_ERR_INVALID_ARGUMENT, "bad plan or n_rows");
  if (!plan->set) return fail(O2MI_ERR_UNSUPPORTED, "no compiled kernels for this plan");
  const int variant = plan->layout == O2MI_LAYOUT_CHANNEL_MAJOR ? o2mi::kVariantChannelMajorVec2
                                                                : o2mi::kVariantComponentMajor;
  const int per_cu = plan->set->blocks_per_cu(variant, backward != 0);
  int g = 0;
  const o2mi::TPGeom geom =
      geometry(plan, n_rows, (int64_t)per_cu * device_cus(),
               backward ? o2mi::kBackwardBlock : plan->set->forward_block,
               backward ? plan->set->backward_tile : plan->set->forward_tile, &g);
  if (grid) *grid = g;
  if (blocks_per_cu) *blocks_per_cu = per_cu;
  if (rows_per_iter) *rows_per_iter = geom.rows_per_iter;
  if (tiles) *tiles = geom.tiles;
  return O2MI_OK;
}

size_t o2mi_tp_backward_workspace_bytes(const o2mi_tp_plan* plan, int64_t n_rows) {
  if (!plan || n_rows <= 0 || !plan->set) return 0;
  // The variant only changes the occupancy query; size for the largest.
  size_t bytes = 0;
  for (int v = 0; v < o2mi::kNumVariants; ++v) {
    if ((plan->layout == O2MI_LAYOUT_CHANNEL_MAJOR) != (v != o2mi::kVariantComponentMajor)) continue;
    bytes = std::max(bytes, backward_shape(plan, n_rows, v).bytes);
  }
  return bytes;
}

int o2mi_tp_backward_f32(const o2mi_tp_plan* plan, const float* x, const float* y, const float* w,
                         const float* g, float* dx, float* dy, float* dw, void* workspace,
                         size_t workspace_bytes, int64_t n_rows, int needed, void* stream) {
  return tp_backward(plan, x, y, w, g, dx, dy, dw, static_cast<float*>(workspace),
                     workspace_bytes, false, n_rows, needed, stream);
}

int o2mi_tp_backward_noalloc_f32(const o2mi_tp_plan* plan, const float* x, const float* y,
                                 const float* w, const float* g, float* dx, float* dy, float* dw,
                                 int64_t n_rows, int needed, void* stream) {
  float* partial = nullptr;
  // Only the weight adjoint uses the scratch.  Its partial rows and second
  // stage are written in full before they are read, so nothing needs to be
  // cleared between calls.
  if ((needed & 4) && n_rows > 0) {
    const int status = scratch_address(&partial);
    if (status != O2MI_OK) return status;
  }
  return tp_backward(plan, x, y, w, g, dx, dy, dw, partial, O2MI_TP_SCRATCH_BYTES, true, n_rows,
                     needed, stream);
}

int o2mi_tp_forward_tables_f32(const o2mi_tp_plan* plan, const float* x, const float* y,
                               const float* w, const int32_t* path_info,
                               const float* path_coefficients, int n_paths, float* out,
                               int64_t n_rows, void* stream) {
  if (!plan) return fail(O2MI_ERR_INVALID_ARGUMENT, "plan is NULL");
  if (n_rows < 0) return fail(O2MI_ERR_INVALID_ARGUMENT, "n_rows must be non-negative");
  if (n_paths != plan->n_paths)
    return fail(O2MI_ERR_INVALID_ARGUMENT, "path table does not have the plan's path count");
  if (n_rows == 0) return O2MI_OK;
  if (!x || !y || !w || !out || !path_info || !path_coefficients)
    return fail(O2MI_ERR_INVALID_ARGUMENT, "NULL tensor pointer");
  if (n_rows > (int64_t)INT32_MAX * 64) return fail(O2MI_ERR_INVALID_ARGUMENT, "n_rows too large");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  O2miTimed timed;
  const bool timing = o2mi_timing_begin(s, &timed, O2MI_TIMED_TP_FORWARD);
  const hipError_t err = o2mi::generic::forward(x, y, w, out, path_info, path_coefficients,
                                                generic_geom(plan, n_rows), device_cus(), s);
  if (timing) o2mi_timing_end(s, &timed);
  if (err != hipSuccess) return fail_hip(err, "table-driven tp forward launch");
  return O2MI_OK;
}

size_t o2mi_tp_backward_tables_workspace_bytes(const o2mi_tp_plan* plan, int64_t n_rows) {
  if (!plan || n_rows <= 0) return 0;
  return tables_shape(plan, n_rows).bytes;
}

int o2mi_tp_backward_tables_f32(const o2mi_tp_plan* plan, const float* x, const float* y,
                                const float* w, const float* g, const int32_t* path_info,
                                const float* path_coefficients, int n_paths, float* dx,
                                float* dy, float* dw, void* workspace, size_t workspace_bytes,
                                int64_t n_rows, int needed, void* stream) {
  if (!plan) return fail(O2MI_ERR_INVALID_ARGUMENT, "plan is NULL");
  if (n_rows < 0) return fail(O2MI_ERR_INVALID_ARGUMENT, "n_rows must be non-negative");
  if (needed & ~7) return fail(O2MI_ERR_INVALID_ARGUMENT, "needed must be a mask of 1, 2, 4");
  if ((needed & 4) && !dw) return fail(O2MI_ERR_INVALID_ARGUMENT, "NULL dw for a requested gradient");
  if (n_paths != plan->n_paths)
    return fail(O2MI_ERR_INVALID_ARGUMENT, "path table does not have the plan's path count");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (n_rows == 0 || needed == 0) {
    if (needed & 4) {
      const hipError_t err = fill(dw, plan->weight_numel, 0.f, s);
      if (err != hipSuccess) return fail_hip(err, "dw fill");
    }
    return O2MI_OK;
  }
  if (!x || !y || !w || !g || !path_info || !path_coefficients)
    return fail(O2MI_ERR_INVALID_ARGUMENT, "NULL input pointer");
  if (((needed & 1) && !dx) || ((needed & 2) && !dy))
    return fail(O2MI_ERR_INVALID_ARGUMENT, "NULL output for a requested gradient");
  if (n_rows > (int64_t)INT32_MAX * 64) return fail(O2MI_ERR_INVALID_ARGUMENT, "n_rows too large");
  const o2mi::generic::Geom geom = generic_geom(plan, n_rows);
  const TablesShape shape = tables_shape(plan, n_rows);
  if ((needed & 4) && (!workspace || workspace_bytes < shape.bytes))
    return fail(O2MI_ERR_WORKSPACE, "workspace smaller than o2mi_tp_backward_tables_workspace_bytes");
  O2miTimed timed;
  const bool timing = o2mi_timing_begin(s, &timed, O2MI_TIMED_TP_BACKWARD);
  hipError_t err = hipSuccess;
  if (needed & 3)
    err = o2mi::generic::input_adjoint(x, y, w, g, dx, dy, path_info, path_coefficients, geom,
                                       needed, device_cus(), s);
  float* partial = static_cast<float*>(workspace);
  if (err == hipSuccess && (needed & 4))
    err = o2mi::generic::weight_adjoint(x, y, g, partial, path_info, path_coefficients, geom,
                                        shape.weight, s);
  if (timing) o2mi_timing_end(s, &timed);
  if (err != hipSuccess) return fail_hip(err, "table-driven tp backward launch");
  if (needed & 4) {
    err = reduce_partials(partial, shape.weight.groups, shape.splits, plan->weight_numel, dw, s);
    if (err != hipSuccess) return fail_hip(err, "dw reduction launch");
  }
  return O2MI_OK;
}

}  // extern "C"
