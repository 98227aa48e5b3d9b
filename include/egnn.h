/* C-ABI of the MI355X-native fused EGNN/MPNN message-passing layer.
 *
 * Plain C, plain pointers and sizes, no torch types.  All device pointers are
 * HIP device memory owned by the caller; `stream` is a hipStream_t passed as
 * void*.  Every call is asynchronous on `stream` except egnn_schedule_build,
 * which synchronises once to report CSR validation errors.
 *
 * Reference interfaces replaced (SatxaFortuny/PyMolecular):
 *   egnn_fwd            <- egnn_forward_kernel_node_parallel[grid](...)
 *                          models/EGNN/forward_kernel.py:14-43 (launch grid
 *                          (num_nodes,), forward_kernel.py:47-49)
 *   egnn_bwd            <- egnn_backward_kernel_node_parallel[grid](...)
 *                          models/EGNN/backward_kernel.py:14-50, launched by
 *                          launch_triton, test_mem.py:7-35
 *   egnn_node_fwd/bwd   <- the node MLP of E_GCL.node_model (egnn_clean.py:60-70)
 *                          and EGNN_Triton_Layer (layer.py:97-101), torch
 *                          modules in the reference
 *   egnn_schedule_build <- no reference counterpart: the reference runs one
 *                          program per CSR row (forward_kernel.py:47,
 *                          test_mem.py:22); this builds the degree-aware edge
 *                          tiling, the split-row list and the source-sorted
 *                          (CSC) permutation once per graph.
 *
 * Semantics (pytorch_baseline.py:18-48 with the optional biases of
 * egnn_clean.py:22-37): CSR row i is the destination, col[e] the source j,
 *   delta = x_i - x_j, r2 = |delta|^2
 *   m  = SiLU(SiLU(h_i W_n1 + h_j W_n2 + r2 w_d + e W_e + b1) W_hl + b2)
 *   phi = SiLU(m W1_mov + bx1) . w2_mov
 *   out_msg[i] = sum_j m_ij ;  out_mov[i] = sum_j delta_ij phi_ij  (/ max(deg_i,1) if mean_agg)
 * Weights are row-major (in, out) as in layer.py:24-33: w1_msg is the packed
 * (2F + g + FE, H) matrix [W_n1 | W_n2 | w_d | W_e] (g = 1 EGNN, 0 MPNN: no w_d
 * row, no phi_x, no coordinate output).  Outputs are overwritten (never
 * accumulated into) and weight gradients go to separate buffers.
 */
#ifndef PYMOLECULAR_AMD_EGNN_H
#define PYMOLECULAR_AMD_EGNN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define EGNN_OK 0
#define EGNN_ERR_NULL 1        /* a required pointer is NULL */
#define EGNN_ERR_DIMS 2        /* unsupported or inconsistent dimensions */
#define EGNN_ERR_STRIDE 3      /* a row stride is too small or not a multiple of the vector width */
#define EGNN_ERR_ALIGN 4       /* h, grad_h, edge_feat, out_msg, grad_out_msg or workspace not 16-byte aligned */
#define EGNN_ERR_WORKSPACE 5   /* workspace or schedule buffer too small */
#define EGNN_ERR_CSR 6         /* rowptr not monotone / not [0..E], or a col index out of [0, N) */
#define EGNN_ERR_HIP 7         /* a HIP runtime call or kernel launch failed */
#define EGNN_ERR_SCRATCH 8     /* the call needs more than egnn_fwd_static's fixed scratch */

/* activation / weight dtype of h, edge_feat, weights, out_msg and grads
 * (coordinates, out_mov and grad_coord are always fp32) */
#define EGNN_F32 0
#define EGNN_BF16 1

typedef struct EgnnDims {
  int64_t N;           /* nodes */
  int64_t E;           /* CSR edges */
  int32_t F;           /* node feature width (F_NODE); multiple of 16, <= 512 */
  int32_t FE;          /* edge feature width (F_EDGE); multiple of 8, 0..480 */
  int32_t H;           /* phi_e hidden (HIDDEN_FEATURES): 64, 128 or 256 */
  int32_t O;           /* message width (OUT_FEATURES): equal to H, or 32 when H = 64 */
  int32_t M;           /* phi_x hidden (HID_FEAT_MOV_MLP): equal to O */
  int32_t equivariant; /* 1 = EGNN (r2 input, phi_x, coordinate output), 0 = MPNN */
  int32_t mean_agg;    /* 1: out_mov divided by max(in-degree, 1) (egnn_clean.py:11,78) */
  int32_t dtype;       /* EGNN_F32 or EGNN_BF16 */
  int32_t weight_layout; /* EGNN_WEIGHTS_PACKED: w1_msg (2F+g+F_E, H), w2_msg (H, O), w1_mov (O, M), the
                            (in, out) layout of layer.py:24-28; EGNN_WEIGHTS_LINEAR: the same matrices
                            transposed, as torch.nn.Linear stores them (egnn_clean.py:24-40): w1_msg
                            (H, 2F+g+F_E), w2_msg (O, H), w1_mov (M, O).  Weight gradients are written
                            in the same layout. */
  int32_t flags;       /* 0, or an OR of:
                          EGNN_FLAG_ACCUMULATE_GRAD_H: egnn_bwd adds its grad_h to the values already in
                          that buffer instead of overwriting them (a layer whose h also feeds the node
                          update passes the node update's gradient of h there);
                          EGNN_FLAG_COORD_RESIDUAL (equivariant only): the layer's coordinate output is
                          x' = x + agg_x (egnn_clean.py:97, coord += agg): egnn_fwd writes coord + agg_x
                          into out_mov, and egnn_bwd writes grad_out_mov + (d agg_x / d coord)^T
                          grad_out_mov into grad_coord, the whole gradient of x' with respect to x;
                          EGNN_FLAG_PROBE_IDENTITY: an instrument, not the layer: egnn_fwd / egnn_bwd
                          run the layer's edge-parallel kernels with the MLP replaced by identity
                          (message P_i + Q_j + W_u e without SiLU or W_hl; dL/dpre1 = grad_out_msg of
                          the row) and keep their gathers, tile schedule, Gh stores and row / source
                          sums, so that the data movement of the gather / segment-sum portion can be
                          timed alone.  bf16 MPNN at H = 128 within those kernels' limits only
                          (EGNN_ERR_DIMS otherwise: it never times another kernel); the outputs are
                          not the layer's */
} EgnnDims;

#define EGNN_WEIGHTS_PACKED 0
#define EGNN_WEIGHTS_LINEAR 1
#define EGNN_FLAG_ACCUMULATE_GRAD_H 1
#define EGNN_FLAG_COORD_RESIDUAL 2
#define EGNN_FLAG_PROBE_IDENTITY 4

/* Row strides in elements; the inner dimension is always contiguous. */
typedef struct EgnnStrides {
  int64_t h;           /* h (rows 16-byte aligned)                      */
  int64_t coord;       /* coord and grad_coord (>= 3)                   */
  int64_t edge;        /* edge_feat                                     */
  int64_t msg;         /* out_msg and grad_out_msg                      */
  int64_t mov;         /* out_mov and grad_out_mov (>= 3)               */
  int64_t grad_h;      /* grad_h; 0: the same as h                      */
} EgnnStrides;

/* Version of this ABI (bumped on any signature change). */
int32_t egnn_abi_version(void);

/* Human-readable text for a status code (static storage). */
const char* egnn_status_string(int32_t status);

/* Schedule buffer bytes (device memory) for a graph of N nodes and E edges. */
size_t egnn_schedule_bytes(int64_t N, int64_t E);
/* Temporary device bytes needed while building the schedule. */
size_t egnn_schedule_tmp_bytes(int64_t N, int64_t E);

/* Validate the CSR (rowptr[0]=0, non-decreasing, rowptr[N]=E, 0<=col<N) and
 * build the schedule into `sched` (egnn_schedule_bytes bytes): the per-edge
 * row ids, the list of rows that cross a 32-edge tile or are empty, the
 * stable source-sorted permutation of the edges, and for every 32-edge tile
 * the runs of one row inside it (span and destination of each, for the
 * per-tile row sums).  Bit-exact and deterministic.
 * Synchronises `stream` once to read the validation flag. */
int32_t egnn_schedule_build(const int32_t* rowptr, const int32_t* col, int64_t N, int64_t E,
                            void* sched, size_t sched_bytes, void* tmp, size_t tmp_bytes,
                            void* stream);

/* Workspace bytes for egnn_fwd / egnn_bwd with these dimensions. */
size_t egnn_fwd_workspace_bytes(const EgnnDims* dims);
size_t egnn_bwd_workspace_bytes(const EgnnDims* dims);

/* Bytes of the optional node_proj buffer: the per-node projections
 * [h W_n1 + b1 | h W_n2] (N x 2H, activation dtype, internal column order).
 * The first phi_e layer is linear in h_i and h_j, so these are computed once
 * per node instead of once per edge (forward_kernel.py:207 recomputes h_i W_n1
 * for every edge).  egnn_fwd fills the buffer when it is given one; egnn_bwd
 * given the same buffer (with h, w1_msg and b1 unchanged) reuses it instead of
 * recomputing; NULL means computed internally. */
size_t egnn_node_proj_bytes(const EgnnDims* dims);

/* Fused forward.  b1/b2/bx1 may be NULL (no bias); edge_ids may be NULL
 * (identity, datasets_loaders.py:11); edge_feat may be NULL when FE = 0 or E = 0.
 * For MPNN (equivariant = 0) coord, w1_mov, w2_mov, bx1 and out_mov are
 * ignored and may be NULL.  Writes out_msg (N, O) and out_mov (N, 3). */
int32_t egnn_fwd(const EgnnDims* dims, const EgnnStrides* strides,
                 const void* h, const float* coord, const void* edge_feat,
                 const int32_t* rowptr, const int32_t* col, const int32_t* edge_ids,
                 const void* w1_msg, const void* w2_msg, const void* w1_mov, const void* w2_mov,
                 const void* b1, const void* b2, const void* bx1,
                 void* out_msg, float* out_mov, void* node_proj,
                 const void* sched, void* workspace, size_t workspace_bytes, void* stream);

/* Allocation-free forward.  No counterpart in the reference: for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops
 * that forbid hipMalloc).  The same computation and kernels as egnn_fwd, with
 * the workspace in a fixed device array inside the library instead of caller
 * memory: EGNN_FWD_STATIC_SCRATCH_BYTES per GPU, part of the library's device
 * code object: resident from when that object is loaded on a GPU (the library's
 * first kernel launch or symbol lookup there, whichever entry point makes it)
 * until the process ends.  Calls whose egnn_fwd_workspace_bytes exceed it
 * return EGNN_ERR_SCRATCH before touching the device.  The caller still provides
 * inputs, outputs and the schedule (built once, beforehand).  It calls no
 * allocator.  All calls on one GPU share the array: calls that overlap on one
 * GPU (several streams or host threads) race.  The stream must belong to the
 * current device. */
#define EGNN_FWD_STATIC_SCRATCH_BYTES ((size_t)128 << 20)
int32_t egnn_fwd_static(const EgnnDims* dims, const EgnnStrides* strides,
                        const void* h, const float* coord, const void* edge_feat,
                        const int32_t* rowptr, const int32_t* col, const int32_t* edge_ids,
                        const void* w1_msg, const void* w2_msg, const void* w1_mov, const void* w2_mov,
                        const void* b1, const void* b2, const void* bx1,
                        void* out_msg, float* out_mov, void* node_proj,
                        const void* sched, void* stream);

/* Fused backward by recomputation.  Takes the forward inputs plus the
 * incoming gradients grad_out_msg (N, O) and grad_out_mov (N, 3), and writes
 * grad_h (N, F), grad_coord (N, 3), grad_w1_msg (packed, like w1_msg),
 * grad_w2_msg (H, O), grad_w1_mov (O, M), grad_w2_mov (M), and grad_b1/b2/bx1
 * when non-NULL.  No edge-feature gradient (the reference computes none).
 * Deterministic: fixed-order reductions only, no floating-point atomics. */
int32_t egnn_bwd(const EgnnDims* dims, const EgnnStrides* strides,
                 const void* h, const float* coord, const void* edge_feat,
                 const int32_t* rowptr, const int32_t* col, const int32_t* edge_ids,
                 const void* w1_msg, const void* w2_msg, const void* w1_mov, const void* w2_mov,
                 const void* b1, const void* b2, const void* bx1,
                 const void* grad_out_msg, const float* grad_out_mov,
                 void* grad_h, float* grad_coord,
                 void* grad_w1_msg, void* grad_w2_msg, void* grad_w1_mov, void* grad_w2_mov,
                 void* grad_b1, void* grad_b2, void* grad_bx1, const void* node_proj,
                 const void* sched, void* workspace, size_t workspace_bytes, void* stream);

/* ---- node update (the per-node epilogue of a layer) ------------------------
 * Replaces the host-side node MLP of E_GCL.node_model (egnn_clean.py:60-70)
 * and of EGNN_Triton_Layer.forward (layer.py:97-101):
 *   z = [x1 | x2] W1^T + b1,  a = SiLU(z),  out = a W2^T + b2 (+ x1 if residual)
 * x1 = h (N, K1), x2 = aggregated messages (N, K2), optionally with node
 * attributes appended by the caller.  W1 (Hn, K1 + K2) and W2 (Fo, Hn) are in
 * torch.nn.Linear layout (out, in); b1 (Hn) and b2 (Fo) may be NULL.
 * K1, K2, Hn and Fo are multiples of 8; Fo == K1 when residual.  Activations,
 * weights and gradients share one dtype (EGNN_F32 or EGNN_BF16), with fp32
 * accumulation.  Row strides (ld*) are in elements, rows 16-byte aligned. */
typedef struct EgnnNodeDims {
  int64_t N;
  int32_t K1, K2, Hn, Fo;
  int32_t residual;
  int32_t dtype;
} EgnnNodeDims;

/* Workspace bytes for egnn_node_bwd. */
size_t egnn_node_bwd_workspace_bytes(const EgnnNodeDims* dims);

/* 1 if egnn_node_fwd / egnn_node_bwd need the activation buffer `act` for these
 * dims, 0 if it may be NULL (bf16, K1 = Hn = Fo = 128, K2 in {0, 128}, N >= 65536:
 * the backward then reads SiLU of the saved `pre` on load, the same bf16 values
 * the forward would have stored), minus an EGNN_ERR_* code for invalid dims.
 * No counterpart in the reference, which keeps every activation of its
 * torch node_mlp for autograd (egnn_clean.py:60-70). */
int32_t egnn_node_act_required(const EgnnNodeDims* dims);

/* Forward.  Writes out (N, Fo, row stride ldo) and the pre-activation `pre`
 * and activation `act` (both (N, Hn) contiguous) that egnn_node_bwd reads;
 * `act` may be NULL when egnn_node_act_required(dims) is 0 (not written). */
int32_t egnn_node_fwd(const EgnnNodeDims* dims, const void* x1, int64_t ld1, const void* x2, int64_t ld2,
                      const void* w1, const void* b1, const void* w2, const void* b2,
                      void* pre, void* act, void* out, int64_t ldo, void* stream);

/* Backward.  Writes grad_x (N, K1 + K2) contiguous: columns [0, K1) are dL/dx1
 * (including the residual term), [K1, K1 + K2) dL/dx2; grad_w1 (Hn, K1 + K2),
 * grad_w2 (Fo, Hn), and grad_b1 / grad_b2 when non-NULL.  `act` may be NULL
 * when egnn_node_act_required(dims) is 0; the results are the same either way.
 * Weight gradients are split-K partial products summed in a fixed order
 * (deterministic). */
int32_t egnn_node_bwd(const EgnnNodeDims* dims, const void* x1, int64_t ld1, const void* x2, int64_t ld2,
                      const void* w1, const void* w2, const void* pre, const void* act,
                      const void* grad_out, int64_t ldgo, void* grad_x,
                      void* grad_w1, void* grad_b1, void* grad_w2, void* grad_b2,
                      void* workspace, size_t workspace_bytes, void* stream);

/* ---- dense-layer weight gradient ---------------------------------------------
 * No kernel counterpart in the reference: the weight gradient of a plain
 * torch.nn.Linear over all nodes, as used by the stack's embedding_in /
 * embedding_out (egnn_clean.py:127-128, 139-145), where K = number of nodes is
 * far larger than the weight.  grad_w (Nout, Kin) in nn.Linear layout and
 * grad_b (Nout, may be NULL) = column sums of dy; deterministic split-K sums.
 * x (N, Kin) and dy (N, Nout) row-major with row strides ldx, lddy (any
 * widths).  One dtype for all tensors (EGNN_F32 / EGNN_BF16). */
/* Forward of the same layer: y (N, Nout, row stride ldy) = x w^T + b, with
 * w (Nout, Kin) in nn.Linear layout and b (Nout) possibly NULL; replaces the
 * torch.nn.Linear calls of embedding_in / embedding_out (egnn_clean.py:139,
 * 145).  Kin, Nout, ldx and ldy are multiples of 8 (16-byte bf16 rows; the
 * Python wrapper pads other widths with zero columns), fp32 accumulation. */
int32_t egnn_dense_fwd(int32_t dtype, int64_t N, int32_t Kin, int32_t Nout, const void* x, int64_t ldx,
                       const void* w, const void* b, void* y, int64_t ldy, void* stream);
/* Input gradient of the same layer: dx (N, Kin, row stride lddx) = dy w, with
 * dy (N, Nout, row stride lddy) and w (Nout, Kin) in nn.Linear layout read as
 * it is (no transposed copy): torch.nn.Linear's grad_input.  Widths and row
 * strides as for egnn_dense_fwd. */
int32_t egnn_dense_dgrad(int32_t dtype, int64_t N, int32_t Kin, int32_t Nout, const void* dy, int64_t lddy,
                         const void* w, void* dx, int64_t lddx, void* stream);
size_t egnn_dense_wgrad_workspace_bytes(int64_t N, int32_t Kin, int32_t Nout);
int32_t egnn_dense_wgrad(int32_t dtype, int64_t N, int32_t Kin, int32_t Nout, const void* x, int64_t ldx,
                         const void* dy, int64_t lddy, void* grad_w, void* grad_b, void* workspace,
                         size_t workspace_bytes, void* stream);

/* ---- instrumentation (no reference counterpart) ---------------------------
 * egnn_profile_enable(class_mask): the kernel launches of the classes whose bit
 * (1 << class) is set in class_mask, made by egnn_fwd / egnn_bwd / egnn_node_* /
 * egnn_dense_*, are bracketed by HIP events recorded on the caller's stream;
 * 0 turns recording off, EGNN_PROFILE_ALL records every class.  Every call clears
 * the previous records.  egnn_profile_read synchronises on those events and
 * returns the summed device time and the launch count of one class.  Off by
 * default.  Not thread-safe; for benchmarks only. */
#define EGNN_PROFILE_ALL 0x1FF
#define EGNN_K_FWD_EDGE 0     /* fused forward edge kernel             */
#define EGNN_K_FWD_FIXUP 1    /* forward split/empty-row fix-up         */
#define EGNN_K_BWD_EDGE 2     /* fused backward edge kernel            */
#define EGNN_K_NODE_GEMM 3    /* per-node projection GEMMs (P|Q, dh)   */
#define EGNN_K_WGRAD 4        /* node-side weight-gradient GEMMs + sums */
#define EGNN_K_NODE_REDUCE 5  /* CSR/CSC node gradient reduction       */
#define EGNN_K_PREP 6         /* weight-fragment preparation           */
#define EGNN_K_NODE_UPDATE 7  /* node update GEMMs (egnn_node_fwd/bwd) */
#define EGNN_K_EDGE_WGRAD 8   /* weight-gradient products over per-edge
                                 factors the backward edge kernel stored
                                 (H = 256 and one-wave-per-tile paths)  */
#define EGNN_K_COUNT 9
int32_t egnn_profile_enable(int32_t class_mask);
int32_t egnn_profile_read(int32_t kernel_class, double* total_ms, int64_t* launches);

/* ---- graph construction (the step before the layer) ------------------------
 * kNN and radius graphs inside segments (protein chains, catalyst systems) as
 * CSR: row i lists the sources j of node i's edges in ascending order.  They
 * replace the host builders of the workload generator (no reference function:
 * the reference draws random CSR graphs, datasets_loaders.py:3-39).
 * pos [N][3] fp64 (8-byte aligned); seg_ptr [n_seg + 1] device int32, from 0 to N,
 * nondecreasing, with no segment larger than max_seg (<= 2048).  The squared
 * distance is ((dx*dx + dy*dy) + dz*dz) in fp64, d = pos_i - pos_j, each operation
 * rounded on its own; the candidates of node i are the other nodes of its segment
 * in (squared distance, index) order.  egnn_knn_graph keeps the first min(k, n - 1)
 * (k <= 64); egnn_radius_graph the first max_nb (<= 64) with squared distance
 * <= cutoff * cutoff.  rowptr [N + 1] and col [col_capacity >= N * k (max_nb)] are
 * written; *n_edges receives E = rowptr[N].  tmp: egnn_graph_tmp_bytes(N) bytes.
 * Each call synchronises the stream once (for the edge count and the segment check:
 * EGNN_ERR_DIMS when a segment is malformed or larger than max_seg). */
size_t egnn_graph_tmp_bytes(int64_t N);
int32_t egnn_knn_graph(const double* pos, int64_t N, const int32_t* seg_ptr, int32_t n_seg, int32_t max_seg,
                       int32_t k, int32_t* rowptr, int32_t* col, int64_t col_capacity, void* tmp, size_t tmp_bytes,
                       int64_t* n_edges, void* stream);
int32_t egnn_radius_graph(const double* pos, int64_t N, const int32_t* seg_ptr, int32_t n_seg, int32_t max_seg,
                          double cutoff, int32_t max_nb, int32_t* rowptr, int32_t* col, int64_t col_capacity,
                          void* tmp, size_t tmp_bytes, int64_t* n_edges, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PYMOLECULAR_AMD_EGNN_H */
