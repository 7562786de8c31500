/* gm_hip.h -- the C ABI of libgmhip.so, the MI355X (gfx950) kernels of
 * gm-attention's fused hot path.
 *
 * Every entry point takes raw device pointers, element counts and a
 * hipStream_t (passed as void*), launches asynchronously on that stream and
 * returns GM_OK (0) or an error code; gm_last_error() holds the message of the
 * calling thread's last failure.  Nothing here allocates, frees or
 * synchronises: outputs and workspaces are the caller's.  Tensors are
 * contiguous, row-major, in the element type the suffix names (_f32: float,
 * _f64: double); index arrays are int64.
 *
 * Descriptor tables (`desc`) are HOST memory: they are a few dozen integers
 * fixed per layer, read at launch to pick the kernel specialisation.  All other
 * pointers are device memory.
 *
 * Flat node layout (the reference's SO2FeatureField.to_flat on the heads'
 * direct sum): frequency 0 first, then each frequency n >= 1 as (copies, 2)
 * real/imaginary pairs; within a frequency the heads' copies are head-major.
 *
 * Reference interfaces each entry point replaces are cited per function
 * (paths relative to masonfaldet/gm-attention's src/gm_attention/nn/).
 */
#ifndef GM_HIP_H
#define GM_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  GM_OK = 0,
  GM_ERR_ARGUMENT = 1, /* a shape, bound or pointer check failed */
  GM_ERR_LAUNCH = 2,   /* the HIP runtime rejected a launch */
  GM_ERR_UNSUPPORTED = 3
};

/* Attention descriptor: one row per frequency, GM_ATTN_DESC int64 columns
 * (n, a_n per head, flat offset, coefficient offset, dim) -- the layout of
 * fused_attention.Plan.rows (fused_attention.py:74-114, fused/attention.h:57-63). */
#define GM_ATTN_DESC 5
#define GM_ATTN_MAX_F 8
#define GM_ATTN_MAX_H 16
#define GM_ATTN_MAX_D 1024

/* Factored descriptor: one row per coefficient block, GM_FACT_DESC int32 columns
 * (kind, z_offset, b_m, angular, transport, power, out_offset, take_real) --
 * fused_factored.Block.row (fused_factored.py:80-99, fused/factored.h:74-83). */
#define GM_FACT_DESC 8
#define GM_FACT_MAX_K 20
#define GM_FACT_MAX_OUT 128
#define GM_FACT_MAX_BM 32
#define GM_FACT_MAX_C 320
#define GM_FACT_MAX_BLOCKS 64
#define GM_FACT_MAX_SEG 4

/* The calling thread's last error message ("" when none). */
const char* gm_last_error(void);

/* ABI version of this library: bump when a signature changes. */
int gm_abi_version(void);

/* Host-side diagnostic, no counterpart in the reference: the logical block
 * each hardware block b < nb runs under the kernels' XCD assignments, written
 * to out[b] (HOST memory).  kind 0: contiguous eighths (xcd_block); 1: chunks
 * dealt round-robin (xcd_spread_block); 2: contiguous unless some eighth of
 * the items holds more than 5/4 of an eighth of the CSR entries
 * (xcd_balanced_block over HOST ptr (n_items + 1), per items a block).
 * Touches no GPU. */
int gm_xcd_block_map(int64_t nb, int kind, const int64_t* ptr, int64_t n_items, int per, int64_t* out);

/* ---------------- scores and neighbourhood softmax ----------------
 *
 * alpha[e, h] = softmax over target i's edges e of
 *   scale * sum_n Re<q_i,n,h , tau_n(e) k_j,n,h> + bias[e],
 * restricted to the edges with inside[e] != 0 (others get 0).
 *
 * Replaces gm_fused_attention.softmax_forward(q, k, transport, bias, inside,
 * desc, row_ptr, source, H, scale, deg_max) (fused/attention_cpu.cpp:197-219,
 * bound at :258-260; called from fused_attention.py:383).
 *   q, k       (n_nodes, D)          transport (n_edges, orders, 2)
 *   bias       (n_edges,)            inside    (n_edges,) uint8
 *   desc       HOST (F, 5) int64     row_ptr   (n_nodes + 1,)    source (n_edges,)
 *   alpha      (n_edges, H) out
 * deg_max is accepted for signature parity; the kernels need no bound on it. */
int gm_softmax_forward_f32(const float* q, const float* k, const float* transport, const float* bias,
                           const uint8_t* inside, const int64_t* desc, const int64_t* row_ptr, const int64_t* source,
                           int64_t n_nodes, int64_t n_edges, int64_t D, int64_t orders, int64_t F, int64_t H,
                           double scale, int64_t deg_max, float* alpha, void* stream);
int gm_softmax_forward_f64(const double* q, const double* k, const double* transport, const double* bias,
                           const uint8_t* inside, const int64_t* desc, const int64_t* row_ptr, const int64_t* source,
                           int64_t n_nodes, int64_t n_edges, int64_t D, int64_t orders, int64_t F, int64_t H,
                           double scale, int64_t deg_max, double* alpha, void* stream);

/* bfloat16 rows for q and k (widened exactly in the kernels), every other
 * tensor float32: the arithmetic of the _f32 entry points, alpha, dq and dk
 * float32.  Build-specific, no counterpart in the reference's op (whose
 * tensors share one dtype); the attention layer reaches them for bfloat16
 * rows.  Heads a power of two up to 16 whose segments are whole chunks of four
 * reals, rows 8-byte aligned (else GM_ERR_ARGUMENT). */
int gm_softmax_forward_bf16(const uint16_t* q, const uint16_t* k, const float* transport, const float* bias,
                            const uint8_t* inside, const int64_t* desc, const int64_t* row_ptr, const int64_t* source,
                            int64_t n_nodes, int64_t n_edges, int64_t D, int64_t orders, int64_t F, int64_t H,
                            double scale, int64_t deg_max, float* alpha, void* stream);
int gm_softmax_backward_bf16(const float* dalpha, const uint16_t* q, const uint16_t* k, const float* transport,
                             const float* bias, const uint8_t* inside, const int64_t* desc, const int64_t* row_ptr,
                             const int64_t* source, const float* alpha, int64_t n_nodes, int64_t n_edges, int64_t D,
                             int64_t orders, int64_t F, int64_t H, double scale, int64_t deg_max,
                             const int64_t* src_ptr, const int64_t* src_order, const int32_t* target_s,
                             const int32_t* inv, const float* transport_s, float* ds, float* dq, float* dk,
                             void* stream);

/* The softmax adjoint and the scores' backward: dq (n_nodes, D) written, dk
 * (n_nodes, D) written (every row, zero where a node is nobody's source).
 *
 * Replaces gm_fused_attention.softmax_backward(dalpha, q, k, transport, bias,
 * inside, desc, row_ptr, source, alpha, H, scale, deg_max)
 * (fused/attention_cpu.cpp:222-252; called from fused_attention.py:395).
 * Unlike the reference (atomic adds on dk, attention_cuda.cu:20-28) the key
 * gradient is gathered per source, so it is deterministic; that pass reads
 * the edges grouped by source, its per-edge inputs as streams in that order:
 *   src_ptr     (n_nodes + 1,)        group offsets into src_order
 *   src_order   (n_edges,)            edge ids sorted by source (stable)
 *   target_s    (n_edges,) int32      target of edge src_order[g], at g
 *   inv         (n_edges,) int32      inverse of src_order (edge e sits at inv[e])
 *   transport_s (n_edges, orders, 2)  transport row of edge src_order[g], at g
 *   ds          (n_edges, H)          workspace of the element type
 * (n_nodes and n_edges below 2^31).  bias and inside are accepted for
 * signature parity and not read. */
int gm_softmax_backward_f32(const float* dalpha, const float* q, const float* k, const float* transport,
                            const float* bias, const uint8_t* inside, const int64_t* desc, const int64_t* row_ptr,
                            const int64_t* source, const float* alpha, int64_t n_nodes, int64_t n_edges, int64_t D,
                            int64_t orders, int64_t F, int64_t H, double scale, int64_t deg_max,
                            const int64_t* src_ptr, const int64_t* src_order, const int32_t* target_s,
                            const int32_t* inv, const float* transport_s, float* ds, float* dq, float* dk, void* stream);
int gm_softmax_backward_f64(const double* dalpha, const double* q, const double* k, const double* transport,
                            const double* bias, const uint8_t* inside, const int64_t* desc, const int64_t* row_ptr,
                            const int64_t* source, const double* alpha, int64_t n_nodes, int64_t n_edges, int64_t D,
                            int64_t orders, int64_t F, int64_t H, double scale, int64_t deg_max,
                            const int64_t* src_ptr, const int64_t* src_order, const int32_t* target_s,
                            const int32_t* inv, const double* transport_s, double* ds, double* dq, double* dk, void* stream);

/* ---------------- depthwise steerable convolution ----------------
 *
 * out_i = sum_e weights[e] C_e(tau v_j): per scalar copy a, rc[e, a] v_j,a;
 * per complex copy of frequency n, A z + (r/c)^{2n} e^{2 i n phi} B conj(z)
 * with z = tau_n(e) v_j and (A, B) read from cc[e, coff + 2a], cc[e, coff + 2a_n + 2a].
 *
 * Replaces gm_fused_attention.conv_forward(v, rc, cc, transport, angular, rho,
 * weights, desc, row_ptr, source, A0, W) (fused/attention_cpu.cpp:94-115;
 * called from fused_attention.py:339).
 *   v (n_nodes, D); rc (n_edges, A0); cc (n_edges, W); transport, angular
 *   (n_edges, orders, 2); rho, weights (n_edges,); out (n_nodes, D). */
int gm_conv_forward_f32(const float* v, const float* rc, const float* cc, const float* transport, const float* angular,
                        const float* rho, const float* weights, const int64_t* desc, const int64_t* row_ptr,
                        const int64_t* source, int64_t n_nodes, int64_t n_edges, int64_t D, int64_t orders, int64_t F,
                        int64_t A0, int64_t W, float* out, void* stream);
int gm_conv_forward_f64(const double* v, const double* rc, const double* cc, const double* transport,
                        const double* angular, const double* rho, const double* weights, const int64_t* desc,
                        const int64_t* row_ptr, const int64_t* source, int64_t n_nodes, int64_t n_edges, int64_t D,
                        int64_t orders, int64_t F, int64_t A0, int64_t W, double* out, void* stream);

/* (dv, drc, dcc) from the output gradient g (n_nodes, D).
 * Replaces gm_fused_attention.conv_backward(g, v, rc, cc, transport, angular,
 * rho, weights, desc, row_ptr, source, A0, W) (fused/attention_cpu.cpp:118-145;
 * called from fused_attention.py:351).  One pass per source node (no atomics:
 * the reference adds dv atomically, attention_cuda.cu:157-170); src_ptr,
 * src_order and target as for gm_softmax_backward_*.  dv, drc, dcc written whole. */
int gm_conv_backward_f32(const float* g, const float* v, const float* rc, const float* cc, const float* transport,
                         const float* angular, const float* rho, const float* weights, const int64_t* desc,
                         const int64_t* row_ptr, const int64_t* source, int64_t n_nodes, int64_t n_edges, int64_t D,
                         int64_t orders, int64_t F, int64_t A0, int64_t W, const int64_t* src_ptr,
                         const int64_t* src_order, const int64_t* target, float* dv, float* drc, float* dcc,
                         void* stream);
int gm_conv_backward_f64(const double* g, const double* v, const double* rc, const double* cc,
                         const double* transport, const double* angular, const double* rho, const double* weights,
                         const int64_t* desc, const int64_t* row_ptr, const int64_t* source, int64_t n_nodes,
                         int64_t n_edges, int64_t D, int64_t orders, int64_t F, int64_t A0, int64_t W,
                         const int64_t* src_ptr, const int64_t* src_order, const int64_t* target, double* dv,
                         double* drc, double* dcc, void* stream);

/* ---------------- depthwise convolution with in-walk radial heads ----------------
 *
 * The depthwise layer's aggregation with its radial trunk and readout heads
 * evaluated inside the walk from rho = d / cutoff: h = SiLU(W1 b(rho) + b1)
 * over the Gaussian basis b_k = exp(-((rho^2 - c_k) / width)^2 / 2) (nb = 4, 6
 * or 8 functions, centers HOST), then per 16-row tile of the packed readout R
 * the coefficient rows R[:, :16] h + R[:, 16], fed to the same message as
 * gm_conv_forward_*.  Replaces the reference's per-edge stacked_coefficients
 * (nn/depthwise.py:206-238) followed by gm_fused_attention.conv_forward
 * (fused/attention_cpu.cpp:94-115) as nn/convolution.py:432-441 chains them.
 *   rf (18, 4, 64): R[:, :16] in MFMA A-operand order; rbias (18 * 16): R[:, 16];
 *   w1 (16, nb), b1 (16) or NULL; ns scalar tiles (a0 = 4..16 ns, multiple of 4),
 *   nc complex tiles of four copies each (tile_n[m] in {1, 2}, tile_col[m] its
 *   first flat column; HOST int32 arrays); the tiles cover the flat width D. */
int64_t gm_conv_radial_partial_row(void);
int64_t gm_conv_radial_backward_groups(int64_t nc);
/* Rows (of gm_conv_radial_partial_row() floats) of the backward's workspace. */
int64_t gm_conv_radial_workspace_rows(int64_t n_blocks);
int gm_conv_radial_forward_f32(const float* v, const float* rf, const float* rbias, const float* w1, const float* b1,
                               const float* centers, int64_t nb, double width, const float* transport,
                               const float* angular, const float* rho, const float* weights, const int64_t* row_ptr,
                               const int64_t* source, int64_t n_nodes, int64_t n_edges, int64_t D, int64_t orders,
                               int64_t a0, int64_t ns, int64_t nc, const int32_t* tile_n, const int32_t* tile_col,
                               float* out, void* stream);
/* dv (n_nodes, D) and grad = (dR in lane order (18 * 256), dR's bias column
 * (18 * 16), dW1 (16 x 8, row-major, first nb columns live), db1 (16)),
 * parameter gradients reduced over n_blocks (a multiple of 8 in 8..65536)
 * persistent workgroups in a fixed order through `partial`
 * (gm_conv_radial_workspace_rows(n_blocks) rows).  src_ptr, src_order, target
 * as for gm_softmax_backward_*; rb (18, 4, 64): R[:, :16] in B-operand order.
 * Replaces the readout and trunk gradients of the reference's torch autograd
 * through stacked_coefficients plus gm_fused_attention.conv_backward
 * (fused/attention_cpu.cpp:118-145). */
int gm_conv_radial_backward_f32(const float* g, const float* v, const float* rf, const float* rbias, const float* rb,
                                const float* w1, const float* b1, const float* centers, int64_t nb, double width,
                                const float* transport, const float* angular, const float* rho, const float* weights,
                                const int64_t* src_ptr, const int64_t* src_order, const int64_t* target,
                                int64_t n_nodes, int64_t n_edges, int64_t D, int64_t orders, int64_t a0, int64_t ns,
                                int64_t nc, const int32_t* tile_n, const int32_t* tile_col, int64_t n_blocks,
                                float* partial, float* dv, float* grad, void* stream);

/* ---------------- neighbourhoods, CSR and per-edge geometry ----------------
 *
 * Paths in this section are relative to src/gm_attention/.
 * targets (n_targets, 3) and sources (n_sources, 3) are float64 unit vectors,
 * | |p|^2 - 1 | <= 1e-14 (the self graph passes one node set twice).  Target i and source j are
 * neighbours iff atan2(|p_i x q_j|, clamp(<p_i, q_j>, -1, 1)) <= limit, each
 * product rounded on its own (limit = r + 1e-10 under the whole-shell rule).
 *
 * Replaces _compute_radius_edges (discretization/edge_geometry.py:656-715: KD-tree ball
 * query and lexsort), the exact filter of compute_edge_geometry (:381-387) and
 * _build_row_ptr (:622-653): step one writes row_ptr (n_targets + 1); the
 * caller reads E = row_ptr[n_targets], sizes edge_index (2, E) and calls step
 * two, which writes targets in row 0 and sources in row 1, target-major,
 * source-minor.  workspace: gm_radius_workspace_doubles(n_targets, n_sources)
 * doubles, kept between the two steps. */
int64_t gm_radius_workspace_doubles(int64_t n_targets, int64_t n_sources);
int gm_radius_row_ptr_f64(const double* targets, int64_t n_targets, const double* sources, int64_t n_sources,
                          double limit, double* workspace, int64_t* row_ptr, void* stream);
int gm_radius_edges_f64(const double* targets, int64_t n_targets, const double* sources, int64_t n_sources,
                        double limit, const double* workspace, const int64_t* row_ptr, int64_t n_edges,
                        int64_t* edge_index, void* stream);

/* The membership distance of each edge, float64 (_geodesic_distances,
 * discretization/edge_geometry.py:492-503).  An index out of range yields NaN. */
int gm_geodesic_distances_f64(const double* targets, const double* sources, const int64_t* edge_index,
                              int64_t n_edges, int64_t n_targets, int64_t n_sources, double* distances, void* stream);

/* The per-edge tables of edge_geometry_from_index
 * (discretization/edge_geometry.py:506-619):
 * log_coordinates (E, 2) = F_i^T (d / sin d)(q - <p, q> p); distances (E);
 * polar_angles = atan2 of the log coordinates; transport_angles = atan2 of
 * column 0 of F_i^T R F_j with R = I + K + K^2 / (1 + <q, p>), K = [q x p]_x
 * (:718-771, :574-585); tangent_quadrature (E) = w_j d / sin d (:588-591);
 * angular_phases and transport_phases (E, max_frequency + 1, 2) = (cos, sin)
 * of k times the angle (phase_powers, representations/so2.py:167-213).
 * Frames (n, 3, 2) hold e1, e2 as columns.  An index out of range yields a
 * row of NaN. */
int gm_edge_tables_f64(const double* targets, const double* target_frames, const double* sources,
                       const double* source_frames, const double* source_quadrature, const int64_t* edge_index,
                       int64_t n_edges, int64_t n_targets, int64_t n_sources, int64_t max_frequency,
                       double* log_coordinates, double* distances, double* polar_angles, double* transport_angles,
                       double* tangent_quadrature, double* angular_phases, double* transport_phases, void* stream);

/* ---------------- transformer block pointwise operators ----------------
 *
 * Flat node rows of width D: frequency 0 in [0, a0), then the nf nonzero
 * frequencies' copies as (re, im) pairs at [offsets[f], offsets[f] + 2 mults[f])
 * (HOST arrays, contiguous after frequency 0, D <= 1024).  Suffixes: _f32
 * (float rows, float parameters), _f64 (double, double), _bf16 (bfloat16 rows
 * as uint16_t, float parameters and float arithmetic).
 *
 * Merged equivariant layer normalization; replaces SO2LayerNorm.forward
 * (nn/normalization.py:150-190): mu = mean x0, v0 = mean (x0 - mu)^2,
 * vn = mean_a |x_n,a|^2 / 2, d = sqrt(mean_present v + eps),
 * y = gamma (x - mu [frequency 0]) / d + beta [frequency 0].  gamma (D) is
 * per coordinate (a copy's gain repeated for re and im), beta (a0) or NULL.
 * Writes y and per node mean and inv_d = 1 / d for the backward. */
int gm_layer_norm_forward_f32(const float* x, const float* gamma, const float* beta, int64_t n_nodes, int64_t D,
                              int64_t a0, int64_t nf, const int64_t* offsets, const int64_t* mults, double eps,
                              float* y, float* mean, float* inv_d, void* stream);
int gm_layer_norm_forward_f64(const double* x, const double* gamma, const double* beta, int64_t n_nodes, int64_t D,
                              int64_t a0, int64_t nf, const int64_t* offsets, const int64_t* mults, double eps,
                              double* y, double* mean, double* inv_d, void* stream);
int gm_layer_norm_forward_bf16(const uint16_t* x, const float* gamma, const float* beta, int64_t n_nodes, int64_t D,
                               int64_t a0, int64_t nf, const int64_t* offsets, const int64_t* mults, double eps,
                               uint16_t* y, float* mean, float* inv_d, void* stream);
/* dx (n_nodes, D) and dparams (D + a0) = (dgamma per coordinate, dbeta), the
 * parameter gradients summed over the nodes in a fixed order through
 * `partial` (gm_layer_norm_partial_rows(n_nodes) rows of D + a0). */
int64_t gm_layer_norm_partial_rows(int64_t n_nodes);
int gm_layer_norm_backward_f32(const float* gy, const float* x, const float* gamma, const float* mean,
                               const float* inv_d, int64_t n_nodes, int64_t D, int64_t a0, int64_t nf,
                               const int64_t* offsets, const int64_t* mults, float* dx, float* partial, float* dparams,
                               void* stream);
int gm_layer_norm_backward_f64(const double* gy, const double* x, const double* gamma, const double* mean,
                               const double* inv_d, int64_t n_nodes, int64_t D, int64_t a0, int64_t nf,
                               const int64_t* offsets, const int64_t* mults, double* dx, double* partial,
                               double* dparams, void* stream);
int gm_layer_norm_backward_bf16(const uint16_t* gy, const uint16_t* x, const float* gamma, const float* mean,
                                const float* inv_d, int64_t n_nodes, int64_t D, int64_t a0, int64_t nf,
                                const int64_t* offsets, const int64_t* mults, uint16_t* dx, float* partial,
                                float* dparams, void* stream);

/* Scalar-gated nonlinearity; replaces SO2ScalarGatedNonlinearity.forward after
 * its gate Linear layers (nn/nonlinearities.py:140-166): y0 = SiLU(h0), and
 * copy a of the f-th nonzero frequency times act(pre[node, g_f + a]) on both
 * coordinates, act = SiLU or, with double_sigmoid, 2 sigmoid; pre (n_nodes, G)
 * holds the gates' pre-activations, frequency-major (g_f = sum of the earlier
 * multiplicities).  Backward: dh = the direct part (SiLU'(h0) gy0, act gy_n)
 * and dpre = act'(pre) <gy_n, h_n>; the gate Linear's own gradient is the
 * caller's. */
int gm_gate_forward_f32(const float* h, const float* pre, int64_t n_nodes, int64_t D, int64_t a0, int64_t nf,
                        const int64_t* offsets, const int64_t* mults, int64_t double_sigmoid, float* y, void* stream);
int gm_gate_forward_f64(const double* h, const double* pre, int64_t n_nodes, int64_t D, int64_t a0, int64_t nf,
                        const int64_t* offsets, const int64_t* mults, int64_t double_sigmoid, double* y, void* stream);
int gm_gate_forward_bf16(const uint16_t* h, const uint16_t* pre, int64_t n_nodes, int64_t D, int64_t a0, int64_t nf,
                         const int64_t* offsets, const int64_t* mults, int64_t double_sigmoid, uint16_t* y,
                         void* stream);
int gm_gate_backward_f32(const float* gy, const float* h, const float* pre, int64_t n_nodes, int64_t D, int64_t a0,
                         int64_t nf, const int64_t* offsets, const int64_t* mults, int64_t double_sigmoid, float* dh,
                         float* dpre, void* stream);
int gm_gate_backward_f64(const double* gy, const double* h, const double* pre, int64_t n_nodes, int64_t D, int64_t a0,
                         int64_t nf, const int64_t* offsets, const int64_t* mults, int64_t double_sigmoid, double* dh,
                         double* dpre, void* stream);
int gm_gate_backward_bf16(const uint16_t* gy, const uint16_t* h, const uint16_t* pre, int64_t n_nodes, int64_t D,
                          int64_t a0, int64_t nf, const int64_t* offsets, const int64_t* mults, int64_t double_sigmoid,
                          uint16_t* dh, uint16_t* dpre, void* stream);

/* Fused feed-forward of the transformer block; replaces the norm2 -> linear1 ->
 * activation -> linear2 -> residual sequence of SO2TransformerBlock.forward
 * (nn/blocks.py:326-349, with nn/normalization.py:117-178,
 * nn/nonlinearities.py:140-166 and nn/linear.py:130-190) for bfloat16 rows of a
 * field with frequencies 0, 1, 2 of A = 32 copies each, widened to B = 64 or
 * 128 copies each, the dropout inactive: out = x + linear2(act(linear1(norm(x)))).
 * Weights are the layers' flat-matrix blocks per frequency f in bfloat16:
 * w1t[f] = M1_f^T (Dh_f, D_f) and w2t[f] = M2_f^T (D_f, Dh_f), row-major, with
 * D_f = A, 2A, 2A and Dh_f = B, 2B, 2B; wg (2B, B) the gates' nn.Linear weights
 * stacked frequency-major; gamma (5A) per flat coordinate, beta (A), b1 (B),
 * bg (2B), b2 (A) float32 or null.  The forward saves mean and inv_d per node.
 * The backward takes the blocks' other orientation too (w1n[f] = M1_f,
 * w2n[f] = M2_f, wgt = wg^T), writes dx = dz + the branch's input gradient and
 * the factors of the parameter gradients: xhat (N x 5A), outs[f] and dhidden[f]
 * (N x Dh_f), dpre (N x 2B) in bfloat16, hidden0 (N x B) float32, and per
 * 16-node tile one row of (dgamma | dbeta) partials (gm_ffn_partial_rows(N)
 * rows of 6A). */
int64_t gm_ffn_partial_rows(int64_t N);
int gm_ffn_forward_bf16(const uint16_t* x, int64_t N, int64_t A, int64_t B, double eps, int double_sigmoid,
                        const float* gamma, const float* beta, const uint16_t* const* w1t, const float* b1,
                        const uint16_t* wg, const float* bg, const uint16_t* const* w2t, const float* b2,
                        uint16_t* out, float* mean, float* inv_d, void* stream);
int gm_ffn_backward_bf16(const uint16_t* dz, const uint16_t* x, int64_t N, int64_t A, int64_t B, double eps,
                         int double_sigmoid, const float* gamma, const float* beta, const uint16_t* const* w1t,
                         const uint16_t* const* w1n, const float* b1, const uint16_t* wg, const uint16_t* wgt,
                         const float* bg, const uint16_t* const* w2t, const uint16_t* const* w2n, const float* mean,
                         const float* inv_d, uint16_t* dx, uint16_t* xhat, float* hidden0, uint16_t* const* outs,
                         uint16_t* const* dhidden, uint16_t* dpre, float* partial, void* stream);

/* ---------------- factored steerable kernel ----------------
 *
 * Per edge e = (i <- j) with h~ = (1, h(e)): every block b's combination
 * u_b = sum_t h~_t Z_t,b(j) of the source's packed mixes, times the block's
 * factor e^{i ang phi} e^{i tr gamma} (rho_e)^power, summed per output slot
 * (rows onto frequency 0 take the real part) into the edge's row.
 *   h (n_edges, K - 1); zc (n_nodes, K, wc, 2); zr (n_nodes, K, wr);
 *   angular, transport (n_edges, n_f, 2); rho (n_edges,);
 *   desc HOST (n_blocks, 8) int32 (GM_FACT_DESC columns);
 *   order (n_edges,) the edges sorted stably by source; group_ptr (n_groups + 1,)
 *   each source's run in that order; group_source (n_groups,) the sources.
 * The blocks must pack zc contiguously, cover zr with one real block, and
 * list the blocks of one output slot consecutively (fused_factored.plan's
 * order).
 *
 * Replaces gm_factored.forward(h, zc, zr, angular, transport, rho, desc,
 * source, order, group_ptr, group_source, d_out, max_bm)
 * (fused/factored_cpu.cpp:77-109; called from fused_factored.py:260, 281).
 * out (n_edges, d_out) written. */
int gm_factored_forward_f32(const float* h, const float* zc, const float* zr, const float* angular,
                            const float* transport, const float* rho, const int32_t* desc, const int64_t* order,
                            const int64_t* group_ptr, const int64_t* group_source, int64_t n_nodes, int64_t n_edges,
                            int64_t n_groups, int64_t K, int64_t wc, int64_t wr, int64_t n_f, int64_t n_blocks,
                            int64_t d_out, int64_t max_bm, float* out, void* stream);
int gm_factored_forward_f64(const double* h, const double* zc, const double* zr, const double* angular,
                            const double* transport, const double* rho, const int32_t* desc, const int64_t* order,
                            const int64_t* group_ptr, const int64_t* group_source, int64_t n_nodes, int64_t n_edges,
                            int64_t n_groups, int64_t K, int64_t wc, int64_t wr, int64_t n_f, int64_t n_blocks,
                            int64_t d_out, int64_t max_bm, double* out, void* stream);

/* out (n_targets, d_out) = each target's weighted sum of its rows over
 * [row_ptr[i], row_ptr[i + 1]).
 * Replaces gm_factored.aggregate(rows, weights, row_ptr)
 * (fused/factored_cpu.cpp:113-138; called from fused_factored.py:283). */
int gm_factored_aggregate_f32(const float* rows, const float* weights, const int64_t* row_ptr, int64_t n_targets,
                              int64_t n_edges, int64_t d_out, float* out, void* stream);
int gm_factored_aggregate_f64(const double* rows, const double* weights, const int64_t* row_ptr, int64_t n_targets,
                              int64_t n_edges, int64_t d_out, double* out, void* stream);

/* The backward: dh (n_edges, K - 1) written; dzc, dzr written for every
 * group source (the caller zeroes them first: a node without edges keeps 0).
 * With target == NULL, g is the rows' gradient (n_edges, d_out) and weights,
 * rows and dweights are ignored (gm_factored.backward, factored_cpu.cpp:198-207).
 * With target (n_edges,), g is the targets' gradient (n_targets, d_out), the
 * edge's gradient is weights[e] g[target[e]], and dweights[e] = <g[target[e]],
 * rows[e]> is written (gm_factored.backward_aggregated, factored_cpu.cpp:210-219;
 * called from fused_factored.py:268, 297).  No atomics: dZ(j) is summed per
 * source group in a fixed order. */
int gm_factored_backward_f32(const float* g, const int64_t* target, const float* weights, const float* rows,
                             const float* h, const float* zc, const float* zr, const float* angular,
                             const float* transport, const float* rho, const int32_t* desc, const int64_t* order,
                             const int64_t* group_ptr, const int64_t* group_source, int64_t n_nodes, int64_t n_edges,
                             int64_t n_groups, int64_t K, int64_t wc, int64_t wr, int64_t n_f, int64_t n_blocks,
                             int64_t d_out, float* dh, float* dzc, float* dzr, float* dweights, void* stream);
int gm_factored_backward_f64(const double* g, const int64_t* target, const double* weights, const double* rows,
                             const double* h, const double* zc, const double* zr, const double* angular,
                             const double* transport, const double* rho, const int32_t* desc, const int64_t* order,
                             const int64_t* group_ptr, const int64_t* group_source, int64_t n_nodes, int64_t n_edges,
                             int64_t n_groups, int64_t K, int64_t wc, int64_t wr, int64_t n_f, int64_t n_blocks,
                             int64_t d_out, double* dh, double* dzc, double* dzr, double* dweights, void* stream);

/* The same forward and backward with the node mixes as up to GM_FACT_MAX_SEG
 * runs of packed columns: run r covers columns [c_r, c_r + width[r]) (runs in
 * column order, tiling [0, 2 wc + wr), none straddling the boundary 2 wc), and
 * column c of node j at mix t is z[r][j * node_stride[r] + t * t_stride[r] +
 * (c - c_r)]; the backward writes dZ to dz[r] at the same places (the caller
 * zeroes them first).  The arrays are HOST memory; the runs are device memory.
 * With this layout the node mixes of every head and input frequency come from
 * one matrix product per input frequency and are read where they were
 * written, with no packing copy.  No counterpart in the reference: zc / zr
 * of gm_factored.forward / backward_aggregated are the two-run case
 * (fused_factored.py:247-299); its batched attention packs every head's
 * node products with a concatenation instead (fused_factored.py:156-180). */
int gm_factored_forward_seg_f32(const float* h, const float* const* z, const int64_t* node_stride,
                                const int64_t* t_stride, const int64_t* width, int64_t n_runs, const float* angular,
                                const float* transport, const float* rho, const int32_t* desc, const int64_t* order,
                                const int64_t* group_ptr, const int64_t* group_source, int64_t n_nodes,
                                int64_t n_edges, int64_t n_groups, int64_t K, int64_t wc, int64_t wr, int64_t n_f,
                                int64_t n_blocks, int64_t d_out, int64_t max_bm, float* out, void* stream);
int gm_factored_forward_seg_f64(const double* h, const double* const* z, const int64_t* node_stride,
                                const int64_t* t_stride, const int64_t* width, int64_t n_runs, const double* angular,
                                const double* transport, const double* rho, const int32_t* desc, const int64_t* order,
                                const int64_t* group_ptr, const int64_t* group_source, int64_t n_nodes,
                                int64_t n_edges, int64_t n_groups, int64_t K, int64_t wc, int64_t wr, int64_t n_f,
                                int64_t n_blocks, int64_t d_out, int64_t max_bm, double* out, void* stream);
int gm_factored_backward_seg_f32(const float* g, const int64_t* target, const float* weights, const float* rows,
                                 const float* h, const float* const* z, float* const* dz, const int64_t* node_stride,
                                 const int64_t* t_stride, const int64_t* width, int64_t n_runs, const float* angular,
                                 const float* transport, const float* rho, const int32_t* desc, const int64_t* order,
                                 const int64_t* group_ptr, const int64_t* group_source, int64_t n_nodes,
                                 int64_t n_edges, int64_t n_groups, int64_t K, int64_t wc, int64_t wr, int64_t n_f,
                                 int64_t n_blocks, int64_t d_out, float* dh, float* dweights, void* stream);
int gm_factored_backward_seg_f64(const double* g, const int64_t* target, const double* weights, const double* rows,
                                 const double* h, const double* const* z, double* const* dz,
                                 const int64_t* node_stride, const int64_t* t_stride, const int64_t* width,
                                 int64_t n_runs, const double* angular, const double* transport, const double* rho,
                                 const int32_t* desc, const int64_t* order, const int64_t* group_ptr,
                                 const int64_t* group_source, int64_t n_nodes, int64_t n_edges, int64_t n_groups,
                                 int64_t K, int64_t wc, int64_t wr, int64_t n_f, int64_t n_blocks, int64_t d_out,
                                 double* dh, double* dweights, void* stream);

/* The same forward and backward (fp32, K = 17, at most 128 packed columns)
 * with every per-edge stream in the order of the source grouping: row g of
 * h_g (n_edges, 16), phase_g (n_edges, 8, 2) -- the angular orders 0..pa-1
 * then the transport orders 0..pt-1 as re/im pairs, pa + pt <= 8 --, rho_g,
 * target_g, weights_g, rows_g (n_edges, d_out), dh_g and dweights_g belongs to
 * the g-th edge of the grouping (order[g] in the others' terms).  A tile's
 * loads are then contiguous and issued before the previous tile finishes.
 * The mixes come as runs (see gm_factored_forward_seg_*).  zw_g
 * (n_edges, 4), or NULL, holds per edge (in the same order) r e^{i phi} and
 * e^{i gamma} (r = rho, phi and gamma the angular and transport angles, the
 * order-1 entries of the phase tables); given it, plans with four copies per
 * frequency and head form every block factor (r e^{i phi})^a (e^{i gamma})^s
 * from it by products instead of reading phase_g.  group_order
 * (n_groups,), or NULL, lists the groups in launch order: largest first
 * keeps the long pole groups off the end of the launch.  No counterpart in
 * the reference, whose kernels index every per-edge table through the
 * grouping (factored_cuda.cu:70-89, 133-248); the results equal those of
 * gm_factored_forward_seg / backward_seg on the permuted streams.
 *
 * The fused trunk: with trunk_w (16, trunk_nb) non-NULL, the lane-owned
 * kernels evaluate h from rho_g themselves -- h_t = SiLU(sum_k W1[t, k] b_k +
 * b1[t]) over the Gaussian basis b_k = exp(-((rho^2 - c_k) / width)^2 / 2),
 * trunk_centers (HOST, trunk_nb <= 8) the c_k, trunk_b (16) or NULL -- and h_g
 * may be NULL (the reference's separate trunk, nn/kernels.py:191-231,
 * 605-607, then never writes h).  Plans that take the generic grouped kernels
 * are rejected under it (gm_factored_lane_tables reports which).  dh_g is
 * still written by the backward. * accumulate != 0: dh_g and dweights_g are added to (the shares of one head's
 * output copies, run one launch each, read the same trunk features and weights)
 * instead of written.
 */
int gm_factored_forward_grouped_f32(const float* h_g, const float* const* z, const int64_t* node_stride,
                                    const int64_t* t_stride, const int64_t* width, int64_t n_runs,
                                    const float* phase_g, const float* rho_g, const float* zw_g,
                                    const int32_t* desc, const int64_t* group_ptr, const int64_t* group_source,
                                    const int64_t* group_order, int64_t n_nodes, int64_t n_edges, int64_t n_groups,
                                    int64_t K, int64_t wc, int64_t wr, int64_t pa, int64_t pt, int64_t n_blocks,
                                    int64_t d_out, const float* trunk_w, const float* trunk_b,
                                    const float* trunk_centers, int64_t trunk_nb, double trunk_width, float* rows_g,
                                    void* stream);
int gm_factored_backward_grouped_f32(const float* g, const int64_t* target_g, const float* weights_g,
                                     const float* rows_g, const float* h_g, const float* const* z, float* const* dz,
                                     const int64_t* node_stride, const int64_t* t_stride, const int64_t* width,
                                     int64_t n_runs, const float* phase_g, const float* rho_g, const float* zw_g,
                                     const int32_t* desc, const int64_t* group_ptr, const int64_t* group_source,
                                     const int64_t* group_order, int64_t n_nodes, int64_t n_edges, int64_t n_groups,
                                     int64_t K, int64_t wc, int64_t wr, int64_t pa, int64_t pt, int64_t n_blocks,
                                     int64_t d_out, const float* trunk_w, const float* trunk_b,
                                     const float* trunk_centers, int64_t trunk_nb, double trunk_width,
                                     int64_t accumulate, float* dh_g, float* dweights_g, void* stream);

/* gm_factored_backward_grouped with the gradient rows g[target * g_ld ..
 * + d_out) read in place from a wider array (one head's columns of the
 * heads' (n_targets, H, d_out) gradient: g_ld = H d_out, even, rows 8-byte
 * aligned).  Build-specific, no counterpart in the reference; the entry
 * above is this one with g_ld = d_out. */
int gm_factored_backward_grouped_ld_f32(const float* g, int64_t g_ld, const int64_t* target_g, const float* weights_g,
                                        const float* rows_g, const float* h_g, const float* const* z,
                                        float* const* dz, const int64_t* node_stride, const int64_t* t_stride,
                                        const int64_t* width, int64_t n_runs, const float* phase_g,
                                        const float* rho_g, const float* zw_g, const int32_t* desc,
                                        const int64_t* group_ptr, const int64_t* group_source,
                                        const int64_t* group_order, int64_t n_nodes, int64_t n_edges,
                                        int64_t n_groups, int64_t K, int64_t wc, int64_t wr, int64_t pa, int64_t pt,
                                        int64_t n_blocks, int64_t d_out, const float* trunk_w, const float* trunk_b,
                                        const float* trunk_centers, int64_t trunk_nb, double trunk_width,
                                        int64_t accumulate, float* dh_g, float* dweights_g, void* stream);

/* The grouped forward and backward with the per-edge streams h_g, rows_g and
 * dh_g in bfloat16 (rounded to nearest even on store, widened exactly on
 * load; every product and sum in float32, the gradients g and the weights
 * float32): the value kernels of a bfloat16 transformer block, whose
 * reference keeps these streams in the rows' dtype (nn/blocks.py:326-349
 * over the factored path, fused_factored.py:247-299).  Plans whose lane
 * slots are one of the compiled-in tables only (gm_factored_lanes_fixed), the
 * trunk read (no fused trunk).  Arguments otherwise as the float32 entries. */
int gm_factored_forward_grouped_bf16(const uint16_t* h_g, const float* const* z, const int64_t* node_stride,
                                     const int64_t* t_stride, const int64_t* width, int64_t n_runs,
                                     const float* phase_g, const float* rho_g, const float* zw_g,
                                     const int32_t* desc, const int64_t* group_ptr, const int64_t* group_source,
                                     const int64_t* group_order, int64_t n_nodes, int64_t n_edges, int64_t n_groups,
                                     int64_t K, int64_t wc, int64_t wr, int64_t pa, int64_t pt, int64_t n_blocks,
                                     int64_t d_out, uint16_t* rows_g, void* stream);
int gm_factored_backward_grouped_ld_bf16(const float* g, int64_t g_ld, const int64_t* target_g,
                                         const float* weights_g, const uint16_t* rows_g, const uint16_t* h_g,
                                         const float* const* z, float* const* dz, const int64_t* node_stride,
                                         const int64_t* t_stride, const int64_t* width, int64_t n_runs,
                                         const float* phase_g, const float* rho_g, const float* zw_g,
                                         const int32_t* desc, const int64_t* group_ptr, const int64_t* group_source,
                                         const int64_t* group_order, int64_t n_nodes, int64_t n_edges,
                                         int64_t n_groups, int64_t K, int64_t wc, int64_t wr, int64_t pa, int64_t pt,
                                         int64_t n_blocks, int64_t d_out, int64_t accumulate, uint16_t* dh_g,
                                         float* dweights_g, void* stream);

/* gm_factored_aggregate with edge e's row at rows[inv[e]] (rows kept in the
 * grouping's order; inv is the grouping's inverse permutation). */
int gm_factored_aggregate_gather_f32(const float* rows, const int64_t* inv, const float* weights,
                                     const int64_t* row_ptr, int64_t n_targets, int64_t n_edges, int64_t d_out,
                                     float* out, void* stream);

/* ---------------- radial trunk ----------------
 *
 * Every head's radial trunk over the edges in one pass: with r = rho[e] and
 * s = r^2, the basis b_k = exp(-((s - centers[k]) / width)^2 / 2) (k < B) and
 * h[head, e, t] = SiLU(sum_k weight[head, t, k] b_k + bias[head, t]) (t < T).
 * T = 16 and B in {4, 6, 8} (the reference's default trunk (16,) over
 * n_radial_basis functions); fp32; h (H, E, T) written.
 * Replaces, for all H heads at once, SO2SteerableKernel._trunk_hidden
 * (nn/kernels.py:605-607): _GaussianRadialBasis (:191-231) then
 * apply_radial_trunk's Linear + SiLU (:108-117). */
int gm_radial_trunk_forward_f32(const float* rho, const float* weight, const float* bias, const float* centers,
                                int64_t n_edges, int64_t H, int64_t T, int64_t B, double width, float* h,
                                void* stream);

/* The trunk's parameter gradients from dh (H, E, T): dparams (H, T * B + T) =
 * per head dweight (T, B) then dbias (T), summed over the edges in a fixed
 * order through `partial`, a workspace of gm_radial_trunk_partials(n_edges)
 * * H * (T * B + T) floats.  Replaces the weight and bias gradients of the
 * reference's split_k_linear (nn/kernels.py:49-105) for the trunk layer. */
int64_t gm_radial_trunk_partials(int64_t n_edges);
int gm_radial_trunk_backward_f32(const float* dh, const float* rho, const float* weight, const float* bias,
                                 const float* centers, int64_t n_edges, int64_t H, int64_t T, int64_t B, double width,
                                 float* partial, float* dparams, void* stream);

/* The same trunk with its features h, and in the backward their gradients dh,
 * stored in bfloat16 (round to nearest even on store, widened exactly on
 * load; float32 arithmetic): the trunk of a bfloat16 transformer block, whose
 * per-edge streams the reference's block keeps in the rows' dtype
 * (nn/blocks.py:326-349 over nn/kernels.py:605-607).  h and dh 8-byte aligned. */
int gm_radial_trunk_forward_bf16(const float* rho, const float* weight, const float* bias, const float* centers,
                                 int64_t n_edges, int64_t H, int64_t T, int64_t B, double width, uint16_t* h,
                                 void* stream);
int gm_radial_trunk_backward_bf16(const uint16_t* dh, const float* rho, const float* weight, const float* bias,
                                  const float* centers, int64_t n_edges, int64_t H, int64_t T, int64_t B, double width,
                                  float* partial, float* dparams, void* stream);

/* ---------------- node mixes (the factored kernel's channel mixing) ----------------
 *
 * Every head's node mixes for one input frequency n as one real product over
 * the nodes: mix (N, C) = v (N, w) M (w, C), v the node field's frequency-n
 * reals (row stride ldv, columns contiguous: a column slice of the flat rows),
 * M the heads' mixing matrix (each block's complex product and input
 * conjugation as reals; C = H K C_n), 1 <= w <= 128, fp32, on MFMA.
 * Replaces the reference's node_products, one complex einsum("ja,bat->jtb")
 * per node vector over _block_weights (nn/kernels.py:575-603, :506-536),
 * for all heads of a layer at once. */
int gm_node_mix_forward_f32(const float* v, int64_t ldv, const float* M, int64_t N, int64_t w, int64_t C, float* out,
                            void* stream);

/* Its input gradient dv (N, w) = dmix (N, C) M^T, written into dv (row stride
 * lddv, only its w columns touched); C a multiple of 4, dmix and M 16-byte
 * aligned.  The reference takes it from autograd through the einsum. */
int gm_node_mix_backward_input_f32(const float* dmix, const float* M, int64_t N, int64_t w, int64_t C, float* dv,
                                   int64_t lddv, void* stream);

/* Its weight gradient dM (w, C) = v^T dmix, summed over row ranges into
 * `partial` (a workspace of gm_node_mix_weight_partials(N, w, C) floats) and
 * then over the ranges in a fixed order: deterministic.  C a multiple of 4. */
int64_t gm_node_mix_weight_partials(int64_t N, int64_t w, int64_t C);
int gm_node_mix_backward_weight_f32(const float* v, int64_t ldv, const float* dmix, int64_t N, int64_t w, int64_t C,
                                    float* partial, float* dM, void* stream);

/* The forward and the weight gradient for bfloat16 node vectors (the rows of
 * a bfloat16 field, widened exactly while staged; w <= 64), M, dmix, out and
 * dM float32: the products of the float32 entry points on the widened values.
 * Build-specific, no counterpart in the reference's op (whose tensors share
 * one dtype); the layers reach them for bfloat16 rows.  The input gradient of
 * a bfloat16 field is gm_node_mix_backward_input_f32's float32 dv. */
int gm_node_mix_forward_bf16(const uint16_t* v, int64_t ldv, const float* M, int64_t N, int64_t w, int64_t C,
                             float* out, void* stream);
int gm_node_mix_backward_weight_bf16(const uint16_t* v, int64_t ldv, const float* dmix, int64_t N, int64_t w,
                                     int64_t C, float* partial, float* dM, void* stream);
/* The weight gradient with bfloat16 mix gradients (widened exactly): v bfloat16
 * (w <= 64) or float32 (w <= 128), dmix (N, C) bfloat16, 8-byte aligned; the
 * partials workspace as gm_node_mix_weight_partials(N, w, C).  The reference
 * has no such entry: they take the fused feed-forward's parameter gradients,
 * x^T g over the nodes (SO2Linear and the gates' nn.Linear, nn/linear.py:130-190,
 * nn/nonlinearities.py:140-166), from the factors its backward writes.  They
 * need the split products (GM_SPLIT_PRODUCTS unset or 1). */
int gm_node_mix_backward_weight_bf16_bf16(const uint16_t* v, int64_t ldv, const uint16_t* dmix, int64_t N, int64_t w,
                                          int64_t C, float* partial, float* dM, void* stream);
int gm_node_mix_backward_weight_f32_bf16(const float* v, int64_t ldv, const uint16_t* dmix, int64_t N, int64_t w,
                                         int64_t C, float* partial, float* dM, void* stream);

/* gm_node_mix_backward_weight_f32 without a workspace argument and without
 * allocating: no counterpart in the reference; for callers that cannot
 * allocate device memory (code under graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The partials live in a 32 MiB
 * (2^23-float) device array of the library, one per GPU, held until the
 * process ends; every call on a GPU uses that GPU's array.  Calls on one GPU
 * are ordered by an event per GPU (created with the array's lookup on the
 * first call): each call's stream waits for the previous call's kernels, on
 * whatever stream or host thread it came from, and the call records the event
 * after its own.  Under stream capture that ordering is not applied: replays
 * of a captured call must not overlap other calls on the same GPU.  Fails
 * with GM_ERR_ARGUMENT when 4 w C (the fp32 kernel of w > 64 under
 * GM_SPLIT_PRODUCTS=0: w C) exceeds 2^23.  Sums in
 * a different split order than the workspace form (same bar, not bitwise). */
int gm_node_mix_backward_weight_noalloc_f32(const float* v, int64_t ldv, const float* dmix, int64_t N, int64_t w,
                                            int64_t C, float* dM, void* stream);

/* Every head's aggregate at once: out[i, h, :] = sum over target i's edges e
 * (CSR order) of alpha[e, h / split] rows[h, inv[e], :].  rows (H, n_edges,
 * d_out) holds each row head's rows in the grouping's order (inv[e] = edge
 * e's position there), alpha (n_edges, H / split) and out (n_targets, H,
 * d_out); H d_out <= 1024.  split > 1 serves a layer whose heads' value rows
 * are computed in split pieces of output copies sharing one attention weight.
 * Serves the heads of one layer at once where the reference aggregates each
 * head on its own (fused/factored_cpu.cpp:110-130 `aggregate`, called from
 * fused_factored.py:273-299 FactoredAggregate); the per-head sums are the
 * same, in the same edge order. */
int gm_factored_aggregate_heads_f32(const float* rows, const int64_t* inv, const float* alpha, const int64_t* row_ptr,
                                    int64_t n_targets, int64_t n_edges, int64_t H, int64_t d_out, int64_t split,
                                    float* out, void* stream);

/* The same aggregate over bfloat16 rows (widened exactly as read; float32
 * sums and output): the rows of gm_factored_forward_grouped_bf16.  d_out a
 * multiple of 4, rows 8-byte and out 16-byte aligned. */
int gm_factored_aggregate_heads_bf16(const uint16_t* rows, const int64_t* inv, const float* alpha,
                                     const int64_t* row_ptr, int64_t n_targets, int64_t n_edges, int64_t H,
                                     int64_t d_out, int64_t split, float* out, void* stream);

/* A row gather fused with a transpose, and its inverse:
 *   gm_gather_transpose_f32:  dst_t[h, g] = src[perm[g], h]   src (n, width), dst_t (width, n)
 *   gm_scatter_transpose_f32: dst[perm[g], h] = src_t[h, g]   src_t (width, n), dst (n, width)
 * perm a permutation of 0..n-1, width <= 64.  Moves per-edge, per-head
 * tables (attention weights and their gradients) between edge order and the
 * grouping's order; no counterpart in the reference. */
int gm_gather_transpose_f32(const float* src, const int64_t* perm, int64_t n, int64_t width, float* dst_t,
                            void* stream);
int gm_scatter_transpose_f32(const float* src_t, const int64_t* perm, int64_t n, int64_t width, float* dst,
                             void* stream);

/* The lane-owned output tables the grouped factored kernels use for a plan
 * (host only; nothing runs on the GPU).  When every block comes in
 * multiplicities of four with radial power equal to its angular order, lane
 * q of an edge's four lanes owns the copies q (mod 4) of every block; its
 * slots are its (block, copy) pairs, the blocks of one output consecutive.
 * On return *n_slots is the slot count (0: the plan takes the generic grouped
 * kernels), slot[16] the per-slot words (bits 0-6 output base, 7 active,
 * 8 real block, 9 scalar output, 10 last slot of its output, 11-13 angular
 * entry, 14 its conjugate, 15-17 transport entry, 18 its conjugate) and
 * slotcol[128] the packed column of slot column 16 (s / 2) + 4 q + 2 (s % 2)
 * + part (0xFF: padding).  desc as for gm_factored_forward_grouped_f32.  No
 * counterpart in the reference: it exposes this build's kernel layout for
 * tests and tools. */
int gm_factored_lane_tables(const int32_t* desc, int64_t n_blocks, int64_t wc, int64_t wr, int64_t d_out, int64_t pa,
                            int64_t pt, int32_t* n_slots, uint32_t* slot, uint8_t* slotcol);

/* *fixed = 1 when a plan's lane slots are one of the compiled-in tables (the
 * kernels that also serve the bfloat16 streams; GM_FACTORED_STATIC=0 declines
 * them), else 0.  Host only; no counterpart in the reference. */
int gm_factored_lanes_fixed(const int32_t* desc, int64_t n_blocks, int64_t wc, int64_t wr, int64_t d_out, int64_t pa,
                            int64_t pt, int32_t* fixed);

/* ---------------- steerable kernel pair terms (per-edge readout) ----------------
 *
 * One (n, m, role) term of the general kernel's per-edge readout:
 *   out(e) += post(e) s(e) f( sum_a M_ba(e) uu_a(e) ),  uu = pre(e) u~(e),
 *   M_ba(e) = sum_t W[(b a) row, t] hidden(e, t) + bias[(b a) row],
 * f = Re under GM_PAIRS_OUT_REAL (then out(e) += s(e) Re(...), post unused),
 * u~ = conj(u) under GM_PAIRS_CONJ_U, a real u promoted under GM_PAIRS_U_REAL;
 * under GM_PAIRS_MATRIX_COMPLEX entry idx = b * a + a' is the row pair
 * (2 idx, 2 idx + 1) = (re, im), else the single real row idx.
 *
 * Replaces gm_pairs.forward(hidden, weight, bias, u, pre, post, scale, out,
 * a, b, flags) (fused/pairs_cpu.cpp:88-111, the per-term launch of
 * fused_pairs.py:176-185).
 *   hidden (n_edges, trunk)     weight (width, trunk)   bias (width) or NULL
 *   u      (n_edges, a[, 2])    pre, post (n_edges, 2) or NULL   scale (n_edges) or NULL
 *   out    (n_edges, b[, 2])    accumulated
 * width = (MATRIX_COMPLEX ? 2 : 1) a b;  1 <= a, b, trunk <= 16.
 *
 * gm_pairs_backward replaces gm_pairs.backward(hidden, weight, bias, u, pre,
 * post, scale, grad_out, grad_u, grad_hidden, grad_k, a, b, flags)
 * (fused/pairs_cpu.cpp:113-136; fused_pairs.py:209-218): accumulates
 * grad_u (n_edges, a[, 2]) and grad_hidden (n_edges, trunk), and writes this
 * term's coefficient gradient row r of edge e at grad_k[r * grad_k_stride + e]
 * (grad_k_stride >= n_edges).  Terms launched in stream order accumulate
 * without races (each lane owns its edge's rows). */
#define GM_PAIRS_MATRIX_COMPLEX 1
#define GM_PAIRS_U_REAL 2
#define GM_PAIRS_CONJ_U 4
#define GM_PAIRS_OUT_REAL 8
int gm_pairs_forward_f32(const float* hidden, const float* weight, const float* bias, const float* u,
                         const float* pre, const float* post, const float* scale, float* out, int64_t n_edges,
                         int64_t a, int64_t b, int64_t trunk, int64_t flags, void* stream);
int gm_pairs_forward_f64(const double* hidden, const double* weight, const double* bias, const double* u,
                         const double* pre, const double* post, const double* scale, double* out, int64_t n_edges,
                         int64_t a, int64_t b, int64_t trunk, int64_t flags, void* stream);
int gm_pairs_backward_f32(const float* hidden, const float* weight, const float* bias, const float* u,
                          const float* pre, const float* post, const float* scale, const float* grad_out,
                          float* grad_u, float* grad_hidden, float* grad_k, int64_t grad_k_stride, int64_t n_edges,
                          int64_t a, int64_t b, int64_t trunk, int64_t flags, void* stream);
int gm_pairs_backward_f64(const double* hidden, const double* weight, const double* bias, const double* u,
                          const double* pre, const double* post, const double* scale, const double* grad_out,
                          double* grad_u, double* grad_hidden, double* grad_k, int64_t grad_k_stride,
                          int64_t n_edges, int64_t a, int64_t b, int64_t trunk, int64_t flags, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GM_HIP_H */
