// C ABI of the fused radial affine + V=1 uvu product (RadialUvuTensorProduct).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <string>

#include "ictc_o2_hp_amd.h"
#include "o2mi_error.hpp"
#include "o2mi_radial_launch.hpp"

// Generated registry (radial_registry.hip).
const o2mi::radial::KernelSet* o2mi_find_radial_set(int m_max, int full, int m_max_in2,
                                                    int full_in2, int kh);

struct o2mi_radial_plan {
  const o2mi::radial::KernelSet* set;
  int C, H;
  int V;  // copies of the second input (shared-weight uvu plans; 1 otherwise)
  int64_t W1, W2;
};

namespace o2mi {
namespace radial {
namespace {

int fail(int status, const std::string& message) {
  o2mi_error_slot() = message;
  return status;
}

int fail_hip(hipError_t err, const char* where) {
  o2mi_error_slot() = std::string(where) + ": " + hipGetErrorString(err);
  return O2MI_ERR_HIP;
}

// out[c] = sum_s in[s * cols + c] in slice order.
__global__ __launch_bounds__(256) void slice_sum_kernel(const float* __restrict__ in, int slices,
                                                        int64_t cols, float* __restrict__ out) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= cols) return;
  float s = 0.f;
  for (int k = 0; k < slices; ++k) s += in[(int64_t)k * cols + c];
  out[c] = s;
}

__global__ __launch_bounds__(256) void zero_kernel(float* __restrict__ out, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = 0.f;
}

unsigned blocks_for(int64_t items) { return (unsigned)((items + 255) / 256); }

int device_cus() {
  static std::mutex mu;
  static int cus[64] = {0};
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0) return 256;
  std::lock_guard<std::mutex> lock(mu);
  int& c = cus[device & 63];
  if (c == 0) {
    hipDeviceProp_t prop;
    c = hipGetDeviceProperties(&prop, device) == hipSuccess ? prop.multiProcessorCount : 256;
    if (c <= 0) c = 256;
  }
  return c;
}

// Edge slices of the affine-adjoint kernel: about one block (slice x channel
// tile x path group) per CU, whole staged tiles per slice, no empty slice.
void slicing(const o2mi_radial_plan* p, int64_t n, int64_t* per_slice, int* slices) {
  const int64_t blocks_per_slice = (int64_t)(p->C / 16) * p->set->weight_groups;
  const int64_t want =
      std::max<int64_t>(1, (device_cus() + blocks_per_slice - 1) / blocks_per_slice);
  const int64_t tile = p->set->weight_edges;
  const int64_t edge_tiles = std::max<int64_t>(1, (n + tile - 1) / tile);
  const int64_t s0 = std::min(want, edge_tiles);
  const int64_t per = ((edge_tiles + s0 - 1) / s0) * tile;
  *per_slice = per;
  *slices = (int)std::max<int64_t>(1, (n + per - 1) / per);
}

bool aligned16(const void* p) { return p && (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Channels per block of the streamed kernels: all of them, unless the edge
// blocks alone would leave CUs idle; then the channel tiles are split over
// grid y (whole 16-channel tiles, no empty split).
int stream_span(const o2mi_radial_plan* p, int64_t n) {
  const int per_block = p->set->stream_edges;
  const int64_t blocks = std::max<int64_t>(1, (n + per_block - 1) / per_block);
  const int64_t cus = device_cus();
  const int tiles = p->C / 16;
  if (blocks >= cus || tiles == 1) return p->C;
  const int64_t want = std::min<int64_t>(tiles, (cus + blocks - 1) / blocks);
  return 16 * (int)((tiles + want - 1) / want);
}

int stream_splits(const o2mi_radial_plan* p, int64_t n) {
  const int span = stream_span(p, n);
  return (p->C + span - 1) / span;
}

// The per-row weight kernels' channel span: as stream_span, for their edge
// blocks and the 32 row_pairs(C) channels an edge group covers per round.
int row_span(const o2mi_radial_plan* p, int64_t n) {
  const int per_block = row_stream_edges(p->C);
  const int64_t blocks = std::max<int64_t>(1, (n + per_block - 1) / per_block);
  const int64_t cus = device_cus();
  const int round = 32 * row_pairs(p->C);
  const int tiles = (p->C + round - 1) / round;
  if (blocks >= cus || tiles == 1) return p->C;
  const int64_t want = std::min<int64_t>(tiles, (cus + blocks - 1) / blocks);
  return std::min(p->C, round * (int)((tiles + want - 1) / want));
}

int row_splits(const o2mi_radial_plan* p, int64_t n) {
  const int span = row_span(p, n);
  return (p->C + span - 1) / span;
}

// Floats of the affine-adjoint slice partials, then of the split dy / dhidden
// partials, in the backward workspace.
int64_t weight_part_floats(const o2mi_radial_plan* p, int64_t n, int needed) {
  if (!(needed & 24) || n <= 0) return 0;
  int64_t per = 0;
  int slices = 0;
  slicing(p, n, &per, &slices);
  const int64_t rows = (int64_t)p->set->paths * p->C;
  return (int64_t)slices * (rows * p->H + rows);
}

// Edge slices of the shared-weight gradient kernel: about one block (slice x
// channel tile) per CU, whole staged tiles per slice.
void dw_slicing(const o2mi_radial_plan* p, int64_t n, int64_t* per_slice, int* slices) {
  const int64_t tiles_c = p->C / 16;
  const int64_t want = std::max<int64_t>(1, (device_cus() + tiles_c - 1) / tiles_c);
  const int64_t tile = p->set->dw_edges;
  const int64_t edge_tiles = std::max<int64_t>(1, (n + tile - 1) / tile);
  const int64_t s0 = std::min(want, edge_tiles);
  const int64_t per = ((edge_tiles + s0 - 1) / s0) * tile;
  *per_slice = per;
  *slices = (int)std::max<int64_t>(1, (n + per - 1) / per);
}

int64_t split_part_floats(const o2mi_radial_plan* p, int64_t n, int needed) {
  const int splits = stream_splits(p, n);
  if (splits <= 1 || n <= 0) return 0;
  return (int64_t)splits * n * (((needed & 2) ? p->W2 : 0) + ((needed & 4) ? p->H : 0));
}

Args make_args(const o2mi_radial_plan* p, int64_t n, const float* x, const float* y,
               const float* hidden, const float* alpha, const float* bias, const float* coef) {
  Args a;
  a.n = n;
  a.C = p->C;
  a.H = p->H;
  a.W1 = (int)p->W1;
  a.W2 = (int)p->W2;
  a.V = p->V;
  a.x = x;
  a.y = y;
  a.hidden = hidden;
  a.alpha = alpha;
  a.bias = bias;
  a.coef = coef;
  a.xindex = nullptr;
  a.x_rows = n;
  a.tile_span = stream_span(p, n);
  a.part_dy = nullptr;
  a.part_gh = nullptr;
  return a;
}

// Gathered first input: x is a table of `table_rows` rows read through
// `index`; the kernels address it with one 32-bit buffer descriptor.
int gather_args(const o2mi_radial_plan* p, Args* a, int64_t table_rows, const int64_t* index) {
  if (table_rows < 0) return fail(O2MI_ERR_INVALID_ARGUMENT, "table_rows must be non-negative");
  if (table_rows * p->W1 * 4 >= ((int64_t)1 << 31))
    return fail(O2MI_ERR_UNSUPPORTED, "gathered first-input table must be below 2 GiB");
  if (!index && a->n > 0) return fail(O2MI_ERR_INVALID_ARGUMENT, "index is NULL");
  a->xindex = index;
  a->x_rows = table_rows;
  return O2MI_OK;
}

int check_inputs(const float* x, const float* y, const float* hidden, const float* alpha,
                 const float* bias, const float* coef) {
  if (!x || !y || !hidden || !alpha || !coef)
    return fail(O2MI_ERR_INVALID_ARGUMENT, "NULL input pointer");
  if (!aligned16(x) || !aligned16(hidden) || !aligned16(alpha))
    return fail(O2MI_ERR_INVALID_ARGUMENT, "x, hidden and alpha must be 16-byte aligned");
  (void)y;
  (void)bias;
  return O2MI_OK;
}

}  // namespace
}  // namespace radial
}  // namespace o2mi

using namespace o2mi::radial;

namespace {

int radial_forward(const o2mi_radial_plan* plan, const Args& a, float* out, void* stream) {
  if (a.n == 0) return O2MI_OK;
  if (int st = check_inputs(a.x, a.y, a.hidden, a.alpha, a.bias, a.coef)) return st;
  if (!aligned16(out)) return fail(O2MI_ERR_INVALID_ARGUMENT, "out must be 16-byte aligned");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  O2miTimed timed;
  const bool timing = o2mi_timing_begin(s, &timed, O2MI_TIMED_RADIAL_FORWARD);
  const hipError_t err = plan->set->forward(a, out, s);
  if (timing) o2mi_timing_end(s, &timed);
  return err == hipSuccess ? O2MI_OK : fail_hip(err, "radial forward launch");
}

int radial_backward(const o2mi_radial_plan* plan, const Args& a, const float* grad_output,
                    float* gx, float* gy, float* ghidden, float* galpha, float* gbias,
                    void* workspace, size_t workspace_bytes, int needed, void* stream) {
  const int64_t n_rows = a.n;
  const float* bias = a.bias;
  if (needed & ~31) return fail(O2MI_ERR_INVALID_ARGUMENT, "needed must be a mask of 1..16");
  if (needed & 16 && !bias)
    return fail(O2MI_ERR_INVALID_ARGUMENT, "bias gradient requested without a bias");
  if (((needed & 8) && !galpha) || ((needed & 16) && !gbias))
    return fail(O2MI_ERR_INVALID_ARGUMENT, "NULL output for a requested affine gradient");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t rows = (int64_t)plan->set->paths * plan->C;
  if (n_rows == 0) {
    // No edges: the affine adjoints are zero, the other roles are empty.
    if (needed & 8) hipLaunchKernelGGL(zero_kernel, dim3(blocks_for(rows * plan->H)), dim3(256),
                                       0, s, galpha, rows * plan->H);
    if (needed & 16) hipLaunchKernelGGL(zero_kernel, dim3(blocks_for(rows)), dim3(256), 0, s,
                                        gbias, rows);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? O2MI_OK : fail_hip(err, "radial zero fill");
  }
  if (int st = check_inputs(a.x, a.y, a.hidden, a.alpha, a.bias, a.coef)) return st;
  if (!grad_output || !aligned16(grad_output))
    return fail(O2MI_ERR_INVALID_ARGUMENT, "grad_output must be a 16-byte aligned pointer");
  if (((needed & 1) && !aligned16(gx)) || ((needed & 2) && !gy) ||
      ((needed & 4) && !aligned16(ghidden)))
    return fail(O2MI_ERR_INVALID_ARGUMENT, "NULL or misaligned output for a requested gradient");
  if ((needed & 8) && !aligned16(galpha))
    return fail(O2MI_ERR_INVALID_ARGUMENT, "galpha must be 16-byte aligned");
  const size_t need = (size_t)(weight_part_floats(plan, n_rows, needed) +
                               split_part_floats(plan, n_rows, needed)) * sizeof(float);
  if (need && (!workspace || workspace_bytes < need || !aligned16(workspace)))
    return fail(O2MI_ERR_WORKSPACE,
                "workspace smaller than o2mi_radial_backward_workspace_bytes or misaligned");
  if (needed & 7) {
    Args b = a;
    const int splits = stream_splits(plan, n_rows);
    if (splits > 1 && (needed & 6)) {
      // Split channels: dy / dhidden partials after the affine-adjoint ones.
      float* part = static_cast<float*>(workspace) + weight_part_floats(plan, n_rows, needed);
      if (needed & 2) {
        b.part_dy = part;
        part += (int64_t)splits * n_rows * plan->W2;
      }
      if (needed & 4) b.part_gh = part;
    }
    O2miTimed timed;
    const bool timing = o2mi_timing_begin(s, &timed, O2MI_TIMED_RADIAL_BACKWARD);
    hipError_t err = plan->set->backward(b, grad_output, gx, gy, ghidden, needed & 7, s);
    if (timing) o2mi_timing_end(s, &timed);
    if (err != hipSuccess) return fail_hip(err, "radial backward launch");
    if (b.part_dy)
      hipLaunchKernelGGL(slice_sum_kernel, dim3(blocks_for(n_rows * plan->W2)), dim3(256), 0, s,
                         b.part_dy, splits, n_rows * plan->W2, gy);
    if (b.part_gh)
      hipLaunchKernelGGL(slice_sum_kernel, dim3(blocks_for(n_rows * plan->H)), dim3(256), 0, s,
                         b.part_gh, splits, n_rows * plan->H, ghidden);
    err = hipGetLastError();
    if (err != hipSuccess) return fail_hip(err, "radial split sum launch");
  }
  if (needed & 24) {
    int64_t per = 0;
    int slices = 0;
    slicing(plan, n_rows, &per, &slices);
    float* part_alpha = static_cast<float*>(workspace);
    float* part_bias = part_alpha + (int64_t)slices * rows * plan->H;
    O2miTimed timed;
    const bool timing = o2mi_timing_begin(s, &timed, O2MI_TIMED_RADIAL_WEIGHT);
    hipError_t err = plan->set->weight(a, grad_output, per, slices, part_alpha, part_bias, s);
    if (timing) o2mi_timing_end(s, &timed);
    if (err != hipSuccess) return fail_hip(err, "radial weight launch");
    if (needed & 8)
      hipLaunchKernelGGL(slice_sum_kernel, dim3(blocks_for(rows * plan->H)), dim3(256), 0, s,
                         part_alpha, slices, rows * plan->H, galpha);
    if (needed & 16)
      hipLaunchKernelGGL(slice_sum_kernel, dim3(blocks_for(rows)), dim3(256), 0, s, part_bias,
                         slices, rows, gbias);
    err = hipGetLastError();
    if (err != hipSuccess) return fail_hip(err, "radial slice sum launch");
  }
  return O2MI_OK;
}

// Edge slices of the V >= 2 shared-weight gradient kernel: at most one block
// (slice x channel tile x path group) per CU — one block fills a CU, so a
// block more than the CUs would run as a second round — whole staged tiles
// per slice.
void vdw_slicing(const o2mi_radial_plan* p, int64_t n, int64_t* per_slice, int* slices) {
  const int64_t blocks_per_slice = (int64_t)(p->C / 16) * p->set->vshared->dw_groups;
  const int64_t want = std::max<int64_t>(1, device_cus() / blocks_per_slice);
  const int64_t tile = p->set->vshared->dw_edges;
  const int64_t edge_tiles = std::max<int64_t>(1, (n + tile - 1) / tile);
  const int64_t s0 = std::min(want, edge_tiles);
  const int64_t per = ((edge_tiles + s0 - 1) / s0) * tile;
  *per_slice = per;
  *slices = (int)std::max<int64_t>(1, (n + per - 1) / per);
}

void shared_slicing(const o2mi_radial_plan* p, int64_t n, int64_t* per_slice, int* slices) {
  if (p->V == 1) dw_slicing(p, n, per_slice, slices);
  else vdw_slicing(p, n, per_slice, slices);
}

// Shared-weight uvu backward workspace: the dw slice partials ([slices][P *
// C * V]), then the split dy partials.
int64_t shared_dw_floats(const o2mi_radial_plan* p, int64_t n, int needed) {
  if (!(needed & 4) || n <= 0) return 0;
  int64_t per = 0;
  int slices = 0;
  shared_slicing(p, n, &per, &slices);
  return (int64_t)slices * p->set->paths * p->C * p->V;
}

}  // namespace

extern "C" {

int o2mi_radial_plan_create(int channels, int m_max, int parity, int m_max_in2, int parity_in2,
                            int hidden, o2mi_radial_plan** plan) {
  if (!plan) return fail(O2MI_ERR_INVALID_ARGUMENT, "plan is NULL");
  *plan = nullptr;
  if (channels < 1 || m_max < 0 || m_max_in2 < 0 || hidden < 1 || (parity != 0 && parity != 1) ||
      (parity_in2 != 0 && parity_in2 != 1))
    return fail(O2MI_ERR_INVALID_ARGUMENT, "invalid radial plan arguments");
  if (channels % 16 != 0)
    return fail(O2MI_ERR_UNSUPPORTED, "fused radial kernels need channels % 16 == 0");
  if (hidden % 4 != 0 || hidden > 64)
    return fail(O2MI_ERR_UNSUPPORTED, "fused radial kernels need hidden % 4 == 0 and <= 64");
  const KernelSet* set = o2mi_find_radial_set(m_max, parity, m_max_in2, parity_in2, 16);
  if (!set)
    return fail(O2MI_ERR_UNSUPPORTED, "no fused radial kernel compiled for this structure");
  auto* p = new o2mi_radial_plan;
  p->set = set;
  p->C = channels;
  p->H = hidden;
  p->V = 1;
  p->W1 = (int64_t)channels * set->comps1;
  p->W2 = set->comps2;
  *plan = p;
  return O2MI_OK;
}

int o2mi_radial_plan_destroy(o2mi_radial_plan* plan) {
  delete plan;
  return O2MI_OK;
}

int o2mi_radial_paths(const o2mi_radial_plan* plan) { return plan ? plan->set->paths : -1; }

int o2mi_radial_forward_f32(const o2mi_radial_plan* plan, const float* x, const float* y,
                            const float* hidden, const float* alpha, const float* bias,
                            const float* coefficients, float* out, int64_t n_rows,
                            void* stream) {
  if (!plan || n_rows < 0) return fail(O2MI_ERR_INVALID_ARGUMENT, "invalid plan or n_rows");
  const Args a = make_args(plan, n_rows, x, y, hidden, alpha, bias, coefficients);
  return radial_forward(plan, a, out, stream);
}

int o2mi_radial_forward_gather_f32(const o2mi_radial_plan* plan, const float* x_table,
                                   int64_t table_rows, const int64_t* index, const float* y,
                                   const float* hidden, const float* alpha, const float* bias,
                                   const float* coefficients, float* out, int64_t n_rows,
                                   void* stream) {
  if (!plan || n_rows < 0) return fail(O2MI_ERR_INVALID_ARGUMENT, "invalid plan or n_rows");
  Args a = make_args(plan, n_rows, x_table, y, hidden, alpha, bias, coefficients);
  if (int st = gather_args(plan, &a, table_rows, index)) return st;
  return radial_forward(plan, a, out, stream);
}

size_t o2mi_radial_backward_workspace_bytes(const o2mi_radial_plan* plan, int64_t n_rows,
                                            int needed) {
  if (!plan || n_rows <= 0 || (needed & ~31)) return 0;
  return (size_t)(weight_part_floats(plan, n_rows, needed) +
                  split_part_floats(plan, n_rows, needed)) * sizeof(float);
}

int o2mi_radial_backward_f32(const o2mi_radial_plan* plan, const float* x, const float* y,
                             const float* hidden, const float* alpha, const float* bias,
                             const float* coefficients, const float* grad_output, float* gx,
                             float* gy, float* ghidden, float* galpha, float* gbias,
                             void* workspace, size_t workspace_bytes, int64_t n_rows, int needed,
                             void* stream) {
  if (!plan || n_rows < 0) return fail(O2MI_ERR_INVALID_ARGUMENT, "invalid plan or n_rows");
  const Args a = make_args(plan, n_rows, x, y, hidden, alpha, bias, coefficients);
  return radial_backward(plan, a, grad_output, gx, gy, ghidden, galpha, gbias, workspace,
                         workspace_bytes, needed, stream);
}

int o2mi_radial_backward_gather_f32(const o2mi_radial_plan* plan, const float* x_table,
                                    int64_t table_rows, const int64_t* index, const float* y,
                                    const float* hidden, const float* alpha, const float* bias,
                                    const float* coefficients, const float* grad_output,
                                    float* gx_edges, float* gy, float* ghidden, float* galpha,
                                    float* gbias, void* workspace, size_t workspace_bytes,
                                    int64_t n_rows, int needed, void* stream) {
  if (!plan || n_rows < 0) return fail(O2MI_ERR_INVALID_ARGUMENT, "invalid plan or n_rows");
  Args a = make_args(plan, n_rows, x_table, y, hidden, alpha, bias, coefficients);
  if (int st = gather_args(plan, &a, table_rows, index)) return st;
  return radial_backward(plan, a, grad_output, gx_edges, gy, ghidden, galpha, gbias, workspace,
                         workspace_bytes, needed, stream);
}

int o2mi_uvu_shared_plan_create(int channels, int channels_in2, int m_max, int parity,
                                int m_max_in2, int parity_in2, o2mi_radial_plan** plan) {
  if (!plan) return fail(O2MI_ERR_INVALID_ARGUMENT, "plan is NULL");
  *plan = nullptr;
  if (channels < 1 || channels_in2 < 1 || m_max < 0 || m_max_in2 < 0 ||
      (parity != 0 && parity != 1) || (parity_in2 != 0 && parity_in2 != 1))
    return fail(O2MI_ERR_INVALID_ARGUMENT, "invalid uvu plan arguments");
  if (channels % 16 != 0)
    return fail(O2MI_ERR_UNSUPPORTED, "shared-weight uvu kernels need channels % 16 == 0");
  if (channels_in2 > o2mi::radial::kVK)
    return fail(O2MI_ERR_UNSUPPORTED, "shared-weight uvu kernels need channels_in2 <= 8");
  const KernelSet* set = o2mi_find_radial_set(m_max, parity, m_max_in2, parity_in2, 16);
  if (!set)
    return fail(O2MI_ERR_UNSUPPORTED, "no shared-weight uvu kernel compiled for this structure");
  auto* p = new o2mi_radial_plan;
  p->set = set;
  p->C = channels;
  p->H = 0;
  p->V = channels_in2;
  p->W1 = (int64_t)channels * set->comps1;
  p->W2 = (int64_t)channels_in2 * set->comps2;
  *plan = p;
  return O2MI_OK;
}

int o2mi_uvu_shared_forward_f32(const o2mi_radial_plan* plan, const float* x, const float* y,
                                const float* weight, const float* coefficients, float* out,
                                int64_t n_rows, void* stream) {
  if (!plan || n_rows < 0) return fail(O2MI_ERR_INVALID_ARGUMENT, "invalid plan or n_rows");
  if (n_rows == 0) return O2MI_OK;
  if (!x || !y || !weight || !coefficients || !aligned16(x) || !aligned16(out))
    return fail(O2MI_ERR_INVALID_ARGUMENT, "NULL input or misaligned x / out");
  Args a = make_args(plan, n_rows, x, y, nullptr, weight, nullptr, coefficients);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  O2miTimed timed;
  const bool timing = o2mi_timing_begin(s, &timed, O2MI_TIMED_UVU_FORWARD);
  const hipError_t err = plan->V == 1 ? plan->set->shared_forward(a, out, s)
                                      : plan->set->vshared->forward(a, out, s);
  if (timing) o2mi_timing_end(s, &timed);
  return err == hipSuccess ? O2MI_OK : fail_hip(err, "shared uvu forward launch");
}

size_t o2mi_uvu_shared_backward_workspace_bytes(const o2mi_radial_plan* plan, int64_t n_rows,
                                                int needed) {
  if (!plan || n_rows <= 0 || (needed & ~7)) return 0;
  return (size_t)(shared_dw_floats(plan, n_rows, needed) +
                  split_part_floats(plan, n_rows, needed & 2)) * sizeof(float);
}

int o2mi_uvu_shared_backward_f32(const o2mi_radial_plan* plan, const float* x, const float* y,
                                 const float* weight, const float* coefficients,
                                 const float* grad_output, float* gx, float* gy, float* gweight,
                                 void* workspace, size_t workspace_bytes, int64_t n_rows,
                                 int needed, void* stream) {
  if (!plan || n_rows < 0) return fail(O2MI_ERR_INVALID_ARGUMENT, "invalid plan or n_rows");
  if (needed & ~7) return fail(O2MI_ERR_INVALID_ARGUMENT, "needed must be a mask of 1, 2, 4");
  if ((needed & 4) && !gweight)
    return fail(O2MI_ERR_INVALID_ARGUMENT, "NULL weight gradient for a requested role");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t wn = (int64_t)plan->set->paths * plan->C * plan->V;
  if (n_rows == 0) {
    if (needed & 4)
      hipLaunchKernelGGL(zero_kernel, dim3(blocks_for(wn)), dim3(256), 0, s, gweight, wn);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? O2MI_OK : fail_hip(err, "shared uvu zero fill");
  }
  if (!x || !y || !weight || !coefficients || !aligned16(x))
    return fail(O2MI_ERR_INVALID_ARGUMENT, "NULL input or misaligned x");
  if (!grad_output || !aligned16(grad_output))
    return fail(O2MI_ERR_INVALID_ARGUMENT, "grad_output must be a 16-byte aligned pointer");
  if (((needed & 1) && !aligned16(gx)) || ((needed & 2) && !gy))
    return fail(O2MI_ERR_INVALID_ARGUMENT, "NULL or misaligned output for a requested gradient");
  const int64_t dw_floats = shared_dw_floats(plan, n_rows, needed);
  const size_t need = (size_t)(dw_floats + split_part_floats(plan, n_rows, needed & 2)) *
                      sizeof(float);
  if (need && (!workspace || workspace_bytes < need || !aligned16(workspace)))
    return fail(O2MI_ERR_WORKSPACE,
                "workspace smaller than o2mi_uvu_shared_backward_workspace_bytes or misaligned");
  Args a = make_args(plan, n_rows, x, y, nullptr, weight, nullptr, coefficients);
  O2miTimed timed;
  const bool timing = o2mi_timing_begin(s, &timed, O2MI_TIMED_UVU_BACKWARD);
  if (needed & 3) {
    const int splits = stream_splits(plan, n_rows);
    if (splits > 1 && (needed & 2))
      a.part_dy = static_cast<float*>(workspace) + dw_floats;
    hipError_t err =
        plan->V == 1 ? plan->set->shared_backward(a, grad_output, gx, gy, needed & 3, s)
                     : plan->set->vshared->backward(a, grad_output, gx, gy, needed & 3, s);
    if (err != hipSuccess) return fail_hip(err, "shared uvu backward launch");
    if (a.part_dy)
      hipLaunchKernelGGL(slice_sum_kernel, dim3(blocks_for(n_rows * plan->W2)), dim3(256), 0, s,
                         a.part_dy, splits, n_rows * plan->W2, gy);
  }
  if (needed & 4) {
    int64_t per = 0;
    int slices = 0;
    shared_slicing(plan, n_rows, &per, &slices);
    float* part = static_cast<float*>(workspace);
    hipError_t err = plan->V == 1 ? plan->set->shared_dw(a, grad_output, per, slices, part, s)
                                  : plan->set->vshared->dw(a, grad_output, per, slices, part, s);
    if (err != hipSuccess) return fail_hip(err, "shared uvu weight-gradient launch");
    hipLaunchKernelGGL(slice_sum_kernel, dim3(blocks_for(wn)), dim3(256), 0, s, part, slices, wn,
                       gweight);
  }
  if (timing) o2mi_timing_end(s, &timed);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? O2MI_OK : fail_hip(err, "shared uvu launch");
}

int o2mi_uvu_rows_forward_f32(const o2mi_radial_plan* plan, const float* x, const float* y,
                              const float* weight, const float* coefficients, float* out,
                              int64_t n_rows, void* stream) {
  if (!plan || n_rows < 0) return fail(O2MI_ERR_INVALID_ARGUMENT, "invalid plan or n_rows");
  if (plan->V != 1)
    return fail(O2MI_ERR_UNSUPPORTED, "per-row weight kernels need a plan with channels_in2 == 1");
  if (n_rows == 0) return O2MI_OK;
  if (!x || !y || !weight || !coefficients || !aligned16(x) || !aligned16(out) ||
      !aligned16(weight))
    return fail(O2MI_ERR_INVALID_ARGUMENT, "NULL input or misaligned x / weight / out");
  Args a = make_args(plan, n_rows, x, y, nullptr, weight, nullptr, coefficients);
  a.tile_span = row_span(plan, n_rows);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  O2miTimed timed;
  const bool timing = o2mi_timing_begin(s, &timed, O2MI_TIMED_UVU_FORWARD);
  const hipError_t err = plan->set->row_forward(a, out, s);
  if (timing) o2mi_timing_end(s, &timed);
  return err == hipSuccess ? O2MI_OK : fail_hip(err, "per-row uvu forward launch");
}

size_t o2mi_uvu_rows_backward_workspace_bytes(const o2mi_radial_plan* plan, int64_t n_rows,
                                              int needed) {
  if (!plan || n_rows <= 0 || (needed & ~7) || !(needed & 2)) return 0;
  const int splits = row_splits(plan, n_rows);
  return splits > 1 ? (size_t)splits * n_rows * plan->W2 * sizeof(float) : 0;
}

int o2mi_uvu_rows_backward_f32(const o2mi_radial_plan* plan, const float* x, const float* y,
                               const float* weight, const float* coefficients,
                               const float* grad_output, float* gx, float* gy, float* gweight,
                               void* workspace, size_t workspace_bytes, int64_t n_rows,
                               int needed, void* stream) {
  if (!plan || n_rows < 0) return fail(O2MI_ERR_INVALID_ARGUMENT, "invalid plan or n_rows");
  if (plan->V != 1)
    return fail(O2MI_ERR_UNSUPPORTED, "per-row weight kernels need a plan with channels_in2 == 1");
  if (needed & ~7) return fail(O2MI_ERR_INVALID_ARGUMENT, "needed must be a mask of 1, 2, 4");
  if (n_rows == 0 || needed == 0) return O2MI_OK;
  if (!x || !y || !weight || !coefficients || !aligned16(x) || !aligned16(weight))
    return fail(O2MI_ERR_INVALID_ARGUMENT, "NULL input or misaligned x / weight");
  if (!grad_output || !aligned16(grad_output))
    return fail(O2MI_ERR_INVALID_ARGUMENT, "grad_output must be a 16-byte aligned pointer");
  if (((needed & 1) && !aligned16(gx)) || ((needed & 2) && !gy) ||
      ((needed & 4) && !aligned16(gweight)))
    return fail(O2MI_ERR_INVALID_ARGUMENT, "NULL or misaligned output for a requested gradient");
  const size_t need = o2mi_uvu_rows_backward_workspace_bytes(plan, n_rows, needed);
  if (need && (!workspace || workspace_bytes < need || !aligned16(workspace)))
    return fail(O2MI_ERR_WORKSPACE,
                "workspace smaller than o2mi_uvu_rows_backward_workspace_bytes or misaligned");
  Args a = make_args(plan, n_rows, x, y, nullptr, weight, nullptr, coefficients);
  a.tile_span = row_span(plan, n_rows);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int splits = row_splits(plan, n_rows);
  if (splits > 1 && (needed & 2)) a.part_dy = static_cast<float*>(workspace);
  O2miTimed timed;
  const bool timing = o2mi_timing_begin(s, &timed, O2MI_TIMED_UVU_BACKWARD);
  hipError_t err = plan->set->row_backward(a, grad_output, gx, gy, gweight, needed, s);
  if (err != hipSuccess) return fail_hip(err, "per-row uvu backward launch");
  if (a.part_dy)
    hipLaunchKernelGGL(slice_sum_kernel, dim3(blocks_for(n_rows * plan->W2)), dim3(256), 0, s,
                       a.part_dy, splits, n_rows * plan->W2, gy);
  if (timing) o2mi_timing_end(s, &timed);
  err = hipGetLastError();
  return err == hipSuccess ? O2MI_OK : fail_hip(err, "per-row uvu launch");
}

}  // extern "C"
