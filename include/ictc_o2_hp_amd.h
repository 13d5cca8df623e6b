/*
 * ictc_o2_hp_amd.h -- C ABI of the MI355X (gfx950) O(2) tensor-product kernels.
 *
 * Plain C: raw device pointers, row counts, a plan handle, a caller-provided
 * workspace and a hipStream_t (passed as void*).  The library never allocates
 * device memory and never synchronises the stream; every call is
 * asynchronous on `stream`.  Every entry point returns O2MI_OK (0) or a
 * negative status; o2mi_last_error() describes the most recent failure of the
 * calling thread.
 *
 * Each declaration names the reference interface it replaces
 * (Parity-LRX/ICTC-O2-HP, src/ictc_o2_hp/...).
 */
#ifndef ICTC_O2_HP_AMD_H
#define ICTC_O2_HP_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum o2mi_status {
  O2MI_OK = 0,
  O2MI_ERR_INVALID_ARGUMENT = -1, /* bad pointer, size, shape or flag */
  O2MI_ERR_UNSUPPORTED = -2,      /* no kernel compiled for this plan */
  O2MI_ERR_WORKSPACE = -3,        /* workspace missing or too small */
  O2MI_ERR_HIP = -4,              /* a HIP runtime call failed */
};

enum o2mi_parity { O2MI_CANONICAL = 0, O2MI_FULL = 1 };
enum o2mi_normalization { O2MI_COMPONENT = 0, O2MI_NORM = 1 };
/* Flat row layouts of triton_o2.py:99-121: 0 = channel-major
 * [copy, channel, component]; 1 = canonical component-major
 * [component, channel]; 2 = full component-major [copy, component, channel]. */
enum o2mi_layout { O2MI_LAYOUT_CHANNEL_MAJOR = 0, O2MI_LAYOUT_COMPONENT_MAJOR = 1,
                   O2MI_LAYOUT_COPY_COMPONENT_MAJOR = 2 };
/* Gradient roles of a backward call (bit mask). */
enum o2mi_needed { O2MI_NEED_X = 1, O2MI_NEED_Y = 2, O2MI_NEED_W = 4 };

typedef struct o2mi_tp_plan o2mi_tp_plan;

/* Status text of the calling thread's last failure ("" if none). */
const char *o2mi_last_error(void);

/* Library version string. */
const char *o2mi_version(void);

/* Create an immutable plan for TensorProduct(channels, m_max, parity,
 * normalization) with flat layout `layout`.  Replaces the per-module
 * metadata registration of triton_o2.py:1098-1132 (_METADATA / metadata_id)
 * and the layout override of triton_o2.py:1226-1234.  A plan may be shared
 * by threads.  Plans with m_max <= 8 have compiled kernels
 * (o2mi_tp_forward_f32 / o2mi_tp_backward_f32); larger m_max (up to 46 full,
 * 47 canonical) give table-driven plans, which only the *_tables_* entry
 * points run (the compiled ones return O2MI_ERR_UNSUPPORTED for them). */
int o2mi_tp_plan_create(int channels, int m_max, int parity, int normalization,
                        int layout, o2mi_tp_plan **plan);
int o2mi_tp_plan_destroy(o2mi_tp_plan *plan);

/* 1 if the plan has compiled kernels (o2mi_tp_forward_f32 and
 * o2mi_tp_backward_f32 run it), 0 if it is table-driven only, -1 for NULL.
 * No counterpart in the reference (its kernels are JIT-specialised). */
int o2mi_tp_plan_compiled(const o2mi_tp_plan *plan);

/* Row width W and packed weight count P_w of the plan
 * (representation_dimension and weight.numel(), native_o2.py:137-143). */
int64_t o2mi_tp_width(const o2mi_tp_plan *plan);
int64_t o2mi_tp_weight_numel(const o2mi_tp_plan *plan);

/* Compiled path table of (m_max, parity, normalization), for verification
 * against the host-side plan.  With `paths`/`terms` NULL only the counts are
 * returned.  paths[7*p..] = k1, k2, k3, weight_units, first_term, n_terms,
 * out_dim; magnitudes[p] = common |coefficient|; terms[4*t..] = i, j, k, sign.
 * Host-only: needs no GPU. */
int o2mi_tp_table(int m_max, int parity, int normalization, int *n_paths,
                  int *n_terms, int32_t *paths, float *magnitudes, int32_t *terms);

/* out[N, W] = TP(x, y; w).  Replaces the o2_forward op
 * (triton_o2.py:786-875): x, y, out are contiguous f32 [N, W]; w is the packed
 * f32 weight [P_w].  n_rows may be 0. */
int o2mi_tp_forward_f32(const o2mi_tp_plan *plan, const float *x, const float *y,
                        const float *w, float *out, int64_t n_rows, void *stream);

/* Launch shape the library picks on the current device for n_rows rows of a
 * forward (backward = 0) or backward (1) call: grid blocks, resident blocks per
 * CU assumed, rows per block iteration and blocks per row (channel tiles).
 * No counterpart in the reference (its grids are fixed per op). */
int o2mi_tp_launch_shape(const o2mi_tp_plan *plan, int64_t n_rows, int backward, int *grid,
                         int *blocks_per_cu, int *rows_per_iter, int *tiles);

/* Bytes of workspace o2mi_tp_backward_f32 needs for n_rows rows. */
size_t o2mi_tp_backward_workspace_bytes(const o2mi_tp_plan *plan, int64_t n_rows);

/* (dx, dy, dw) = VJP of the forward at cotangent g.  Replaces the o2_backward
 * op (triton_o2.py:878-966): the input adjoint of :452-568 and the
 * deterministic weight adjoint + fixed-order reduction of :688-780, fused
 * into one pass over x, y, g.  Roles not set in `needed` are not written
 * (their pointers may be NULL).  n_rows == 0 writes dw = 0.  dw is a
 * fixed-order fp32 sum: bitwise reproducible for a given n_rows. */
int o2mi_tp_backward_f32(const o2mi_tp_plan *plan, const float *x, const float *y,
                         const float *w, const float *g, float *dx, float *dy,
                         float *dw, void *workspace, size_t workspace_bytes,
                         int64_t n_rows, int needed, void *stream);

/* Table-driven forward for any plan, including plans without compiled
 * kernels (m_max >= 9; o2mi_tp_plan_create accepts m_max up to 46 in full
 * parity, 47 in canonical).  Replaces the o2_forward op (triton_o2.py:786-875)
 * for plans the reference JIT-specialises (triton_o2.py:1098-1132): the path
 * table is the op's own device metadata, path_info int32 [n_paths, 25] and
 * path_coefficients f32 [n_paths, 4] as built by runtime_weight.py:14-29
 * (weight_metadata), with n_paths the plan's path count.  Same layouts and
 * results as o2mi_tp_forward_f32. */
int o2mi_tp_forward_tables_f32(const o2mi_tp_plan *plan, const float *x, const float *y,
                               const float *w, const int32_t *path_info,
                               const float *path_coefficients, int n_paths, float *out,
                               int64_t n_rows, void *stream);

/* Bytes of workspace o2mi_tp_backward_tables_f32 needs for n_rows rows. */
size_t o2mi_tp_backward_tables_workspace_bytes(const o2mi_tp_plan *plan, int64_t n_rows);

/* Table-driven VJP for any plan: the o2_backward op (triton_o2.py:878-966)
 * with the runtime-table weight adjoint of runtime_weight.py:54-91.  dx, dy
 * and the dw partial rows are separate passes; dw is a fixed-order sum
 * (bitwise reproducible).  Arguments as o2mi_tp_backward_f32 plus the path
 * table of o2mi_tp_forward_tables_f32. */
int o2mi_tp_backward_tables_f32(const o2mi_tp_plan *plan, const float *x, const float *y,
                                const float *w, const float *g, const int32_t *path_info,
                                const float *path_coefficients, int n_paths, float *dx,
                                float *dy, float *dw, void *workspace, size_t workspace_bytes,
                                int64_t n_rows, int needed, void *stream);

/* Bytes of the library-owned device scratch of o2mi_tp_backward_noalloc_f32
 * (one array per GPU, held until the process ends). */
#define O2MI_TP_SCRATCH_BYTES ((size_t)64 << 20)

/* o2mi_tp_backward_f32 without a workspace argument and without any device
 * allocation: the dw partial rows live in a library-owned device array of
 * O2MI_TP_SCRATCH_BYTES per GPU.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Results equal
 * o2mi_tp_backward_f32's (bitwise whenever that call's workspace would fit in
 * the scratch; otherwise the grid is reduced to fit and dw is a different
 * fixed-order sum, equal within fp32 rounding).  Returns O2MI_ERR_WORKSPACE
 * when even one block's partial rows exceed the scratch (weight_numel too
 * large).  Every call on a GPU shares that GPU's array: calls that overlap on
 * one GPU (several streams or threads) race and must be serialised by the
 * caller. */
int o2mi_tp_backward_noalloc_f32(const o2mi_tp_plan *plan, const float *x, const float *y,
                                 const float *w, const float *g, float *dx, float *dy,
                                 float *dw, int64_t n_rows, int needed, void *stream);

/* ---- uvu product (UvuTensorProduct) ---------------------------------------
 * One problem description per call; the tables are device arrays the caller
 * owns (the module buffers _path_info, _coefficients, _first_order,
 * _second_order of uvu_o2.py:218-226, built as in uvu_triton.py:39-67). */
typedef struct o2mi_uvu_problem {
  int64_t n_rows;
  int32_t channels;       /* C: channels per entry of the first input and output */
  int32_t channels_in2;   /* V: channels per entry of the second input */
  int32_t n_paths;        /* P */
  int32_t n_out_entries;  /* entries of the first input (= output entries) */
  int32_t n_in2_entries;  /* entries of the second input */
  int32_t width1;         /* floats per row of x and out */
  int32_t width2;         /* floats per row of y */
  int32_t shared_weights; /* 1: w is [P*C*V]; 0: w is [n_rows, P*C*V] */
  const int32_t *info;         /* [P + 2*n_out_entries + n_in2_entries][7] records */
  const float *coefficients;   /* [P][2][2][2]: out, in1, in2 components */
  const int32_t *first_order;  /* [P] paths sorted by first entry */
  const int32_t *second_order; /* [P] paths sorted by second entry */
} o2mi_uvu_problem;

/* out = uvu(x, y; w).  Replaces the uvu forward / forward_into ops
 * (uvu_triton.py:235-284). */
int o2mi_uvu_forward_f32(const o2mi_uvu_problem *problem, const float *x, const float *y,
                         const float *w, float *out, void *stream);

/* Workspace of o2mi_uvu_backward_f32 (non-zero only for shared weights with
 * the weight role requested). */
size_t o2mi_uvu_backward_workspace_bytes(const o2mi_uvu_problem *problem, int needed);

/* (gx, gy, gw) for the roles in `needed` (1 x, 2 y, 4 w).  Replaces the uvu
 * backward / backward_into ops (uvu_triton.py:287-414).  gw is [P*C*V] for
 * shared weights (a fixed-order sum over rows) or [n_rows, P*C*V]. */
int o2mi_uvu_backward_f32(const o2mi_uvu_problem *problem, const float *x, const float *y,
                          const float *w, const float *g, float *gx, float *gy, float *gw,
                          int needed, void *workspace, size_t workspace_bytes, void *stream);

/* ---- radial affine fused with a V=1 uvu product (RadialUvuTensorProduct) --
 * out = uvu(x, y; W) with per-edge weights W = hidden @ alpha^T + bias
 * generated inside the kernel (radial_uvu.py:10-66, radial_streamed.py:37-57).
 * Layouts: x, out, g, dx [N, C*K1] as the uvu first input ([copy, channel,
 * component] entries); y, dy [N, K2] (V = 1); hidden, dhidden [N, H];
 * alpha, dalpha [P*C, H] (torch.nn.Linear.weight); bias, dbias [P*C];
 * coefficients [P][2][2][2] (the tp module's _coefficients).  x, out, g, dx,
 * hidden, dhidden, alpha, dalpha and the workspace must be 16-byte aligned. */
typedef struct o2mi_radial_plan o2mi_radial_plan;

/* Plan for a uvu structure (m_max, parity, m_max_in2, parity_in2), C channels
 * and hidden width H.  O2MI_ERR_UNSUPPORTED when no fused kernel exists for
 * it (C % 16 != 0, H % 4 != 0, H > 64, m_max > 6 or m_max_in2 != m_max);
 * callers then compose the affine map and the uvu product.  Replaces the
 * block policy of radial_streamed.py:17-34. */
int o2mi_radial_plan_create(int channels, int m_max, int parity, int m_max_in2,
                            int parity_in2, int hidden, o2mi_radial_plan **plan);
int o2mi_radial_plan_destroy(o2mi_radial_plan *plan);

/* Number of paths P of the plan's structure. */
int o2mi_radial_paths(const o2mi_radial_plan *plan);

/* out = tp(x, y, hidden @ alpha^T + bias); bias may be NULL.  Replaces the
 * radial_stream_forward op (radial_streamed.py:81-99). */
int o2mi_radial_forward_f32(const o2mi_radial_plan *plan, const float *x, const float *y,
                            const float *hidden, const float *alpha, const float *bias,
                            const float *coefficients, float *out, int64_t n_rows,
                            void *stream);

/* o2mi_radial_forward_f32 with a gathered first input: edge e reads row
 * index[e] of x_table ([table_rows, W1], 16-byte aligned, below 2 GiB; an
 * index outside [0, table_rows) reads a zero row).  Equals the reference's
 * composition tp(x_table[index], y, radial_out(hidden)) (radial_uvu.py:50-52)
 * without materialising the gathered rows; the node -> edge gather of a
 * message-passing layer, which the reference leaves outside its radial chain
 * (docs/RADIAL.md:97-99).  O2MI_ERR_UNSUPPORTED for a larger table. */
int o2mi_radial_forward_gather_f32(const o2mi_radial_plan *plan, const float *x_table,
                                   int64_t table_rows, const int64_t *index, const float *y,
                                   const float *hidden, const float *alpha, const float *bias,
                                   const float *coefficients, float *out, int64_t n_rows,
                                   void *stream);

/* Workspace of o2mi_radial_backward_f32 (non-zero when dalpha or dbias is
 * requested). */
size_t o2mi_radial_backward_workspace_bytes(const o2mi_radial_plan *plan, int64_t n_rows,
                                            int needed);

/* Adjoints at cotangent g for the roles in `needed`: 1 x, 2 y, 4 hidden,
 * 8 alpha, 16 bias (the mask of radial_streamed.py:109-139).  dalpha and dbias
 * are fixed-order fp32 sums over edges; n_rows == 0 writes them as zero. */
int o2mi_radial_backward_f32(const o2mi_radial_plan *plan, const float *x, const float *y,
                             const float *hidden, const float *alpha, const float *bias,
                             const float *coefficients, const float *grad_output, float *dx,
                             float *dy, float *dhidden, float *dalpha, float *dbias,
                             void *workspace, size_t workspace_bytes, int64_t n_rows,
                             int needed, void *stream);

/* o2mi_radial_backward_f32 with the gathered first input of
 * o2mi_radial_forward_gather_f32.  dx_edges ([n_rows, W1]) receives the
 * adjoint of each edge's gathered row; o2mi_rows_segment_sum_f32 reduces it
 * onto the table rows.  Workspace as o2mi_radial_backward_workspace_bytes. */
int o2mi_radial_backward_gather_f32(const o2mi_radial_plan *plan, const float *x_table,
                                    int64_t table_rows, const int64_t *index, const float *y,
                                    const float *hidden, const float *alpha, const float *bias,
                                    const float *coefficients, const float *grad_output,
                                    float *dx_edges, float *dy, float *dhidden, float *dalpha,
                                    float *dbias, void *workspace, size_t workspace_bytes,
                                    int64_t n_rows, int needed, void *stream);

/* ---- uvu product with shared weights, 1 <= V <= 8 ---------------------------
 * UvuTensorProduct(C, V, m, parity=..., parity_in2=..., shared_weights=True),
 * the reference's default weight mode: out[k, u] += sum over paths (i, j, k)
 * of CG_p(x[i, u], sum_v w[p, u, v] y[j, v]) (uvu_o2.py:50-73).  Layouts as
 * the uvu calls above (uvu_o2.py:27-41): x [n][C * components], y [n][V *
 * components] (entry-major, [copy][component] inside an entry), weights
 * [P*C*V] in [path, channel, copy] order.  Plans exist for the same
 * structures as the radial plans (C % 16 == 0, m_max = m_max_in2 <= 6) and
 * channels_in2 = V <= 8 (O2MI_ERR_UNSUPPORTED otherwise: use the
 * o2mi_uvu_* calls); destroy with o2mi_radial_plan_destroy. */
int o2mi_uvu_shared_plan_create(int channels, int channels_in2, int m_max, int parity,
                                int m_max_in2, int parity_in2, o2mi_radial_plan **plan);

/* out = uvu(x, y; w).  Replaces the uvu forward op for this mode
 * (uvu_triton.py:235-284). */
int o2mi_uvu_shared_forward_f32(const o2mi_radial_plan *plan, const float *x, const float *y,
                                const float *weight, const float *coefficients, float *out,
                                int64_t n_rows, void *stream);

/* Workspace of o2mi_uvu_shared_backward_f32 (the weight gradient's edge-slice
 * partials, and the dy partials when few rows split the channels). */
size_t o2mi_uvu_shared_backward_workspace_bytes(const o2mi_radial_plan *plan, int64_t n_rows,
                                                int needed);

/* (gx, gy, gweight) for the roles in `needed` (1 x, 2 y, 4 weight): the uvu
 * backward op for this mode (uvu_triton.py:287-414).  gweight [P*C] is a
 * fixed-order fp32 sum over rows (zero for n_rows == 0). */
int o2mi_uvu_shared_backward_f32(const o2mi_radial_plan *plan, const float *x, const float *y,
                                 const float *weight, const float *coefficients,
                                 const float *grad_output, float *gx, float *gy, float *gweight,
                                 void *workspace, size_t workspace_bytes, int64_t n_rows,
                                 int needed, void *stream);

/* ---- V = 1 uvu product with per-row weights -------------------------------
 * UvuTensorProduct(C, 1, m, ..., shared_weights=False) with external weights
 * [n][P*C] (uvu_single.py's kernels and uvu_triton.py:235-414 in the
 * reference).  Takes a plan from o2mi_uvu_shared_plan_create with
 * channels_in2 == 1 (O2MI_ERR_UNSUPPORTED otherwise); layouts as above.  x,
 * weight, out, gx, gweight 16-byte aligned. */
int o2mi_uvu_rows_forward_f32(const o2mi_radial_plan *plan, const float *x, const float *y,
                              const float *weight, const float *coefficients, float *out,
                              int64_t n_rows, void *stream);

/* Workspace of o2mi_uvu_rows_backward_f32 (split dy partials when few rows
 * split the channels; 0 otherwise). */
size_t o2mi_uvu_rows_backward_workspace_bytes(const o2mi_radial_plan *plan, int64_t n_rows,
                                              int needed);

/* (gx, gy, gweight [n][P*C]) for the roles in `needed` (1 x, 2 y, 4 weight). */
int o2mi_uvu_rows_backward_f32(const o2mi_radial_plan *plan, const float *x, const float *y,
                               const float *weight, const float *coefficients,
                               const float *grad_output, float *gx, float *gy, float *gweight,
                               void *workspace, size_t workspace_bytes, int64_t n_rows,
                               int needed, void *stream);

/* ---- row gather and deterministic row segment sums -------------------------
 * The node <-> edge data movement of a message-passing layer around the
 * radial product.  No counterpart in the reference, which gathers with
 * torch indexing and scatters with atomic index_add outside its chain
 * (docs/RADIAL.md:97-99). */

/* dst[e, :] = src[index[e], :] for e < n_rows ([n_rows, width] f32); an
 * index outside [0, src_rows) writes a zero row. */
int o2mi_rows_gather_f32(const float *src, int64_t src_rows, const int64_t *index,
                         int64_t n_rows, int64_t width, float *dst, void *stream);

/* dst[s, :] = sum of rows[order[k], :] for k in [offsets[s], offsets[s+1]),
 * added in increasing k (s < n_segments; offsets has n_segments + 1 entries;
 * runs are clamped to [0, n_rows) and entries of `order` outside [0, n_rows)
 * are skipped).  With `order` a stable sort of the edges by index and
 * `offsets` each table row's run, this is the adjoint of o2mi_rows_gather_f32
 * in a fixed summation order (bitwise reproducible). */
int o2mi_rows_segment_sum_f32(const float *rows, int64_t n_rows, int64_t width,
                              const int64_t *order, const int64_t *offsets, int64_t n_segments,
                              float *dst, void *stream);

/* Kernel timing for measurement harnesses (no counterpart in the reference):
 * while enabled, every forward/backward call records a HIP event pair around
 * its main kernel on the call's stream.  o2mi_kernel_timing_read waits for
 * the recorded events and returns the summed milliseconds and counts since the
 * previous read. */
int o2mi_kernel_timing(int enable);
int o2mi_kernel_timing_read(double *forward_ms, int *forward_count, double *backward_ms,
                            int *backward_count);
/* Same, per kind: 0 TP forward, 1 TP backward, 2 radial forward, 3 radial
 * input adjoints (dx, dy, dhidden), 4 radial affine adjoints (dalpha, dbias),
 * 5 uvu forward (per-row-weight and shared-weight V = 1 kernels), 6 uvu
 * backward (the same).
 * ms[k] and counts[k] for k < n_kinds. */
int o2mi_kernel_timing_read_kinds(double *ms, int *counts, int n_kinds);

#ifdef __cplusplus
}
#endif

#endif /* ICTC_O2_HP_AMD_H */
