/*
 * molnex C ABI — MI355X (gfx950) kernels for MolNex's equivariant message-passing
 * hot path.  Plain pointers and sizes only: every tensor argument is a device
 * pointer to contiguous row-major memory, every call is enqueued on the given
 * HIP stream, returns an MNX_* status and never allocates memory the caller
 * sees.  Scratch memory comes in through `workspace` (size from the matching
 * *_workspace_bytes query).  mnx_last_error() gives the message of the last
 * failing call on this thread.
 *
 * The reference exposes this path as torch custom ops (TORCH_LIBRARY(molix),
 * src/molix/op/src/molix_library.cpp:16-43) plus the cuequivariance-backed
 * modules of molrep; each entry point below names the reference interface it
 * replaces.
 */
#ifndef MOLNEX_H
#define MOLNEX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* mnx_stream_t; /* == hipStream_t */

#define MNX_OK 0
#define MNX_ERR_INVALID 1     /* bad argument (shape, size, null pointer) */
#define MNX_ERR_UNSUPPORTED 2 /* configuration without a compiled kernel */
#define MNX_ERR_HIP 3         /* HIP runtime error */
#define MNX_ERR_WORKSPACE 4   /* workspace smaller than the query returned */

const char* mnx_last_error(void);
int mnx_abi_version(void);

/* ------------------------------------------------------------------------ */
/* Neighbor list (cell list).                                                */
/*                                                                            */
/* Replaces torch.ops.molix.get_neighbor_pairs                                */
/* (molix_library.cpp:22-26; CPU get_neighbor_pairs.cpp:28-77, CUDA           */
/* get_neighbor_pairs.cu:29-79,104-151) and the pair enumeration behind       */
/* molix.data.tasks.NeighborList (src/molix/data/tasks/neighbor_list.py:67-103).
 * Pair predicate and geometry are the reference CPU path's, bit for bit:     */
/*   d = pos[i] - pos[j]; for k = 2,1,0: d -= rint(d[k] / box[k][k]) * box[k] */
/*   dist = sqrt(fma(d2, d2, fma(d1, d1, d0 * d0)));                          */
/*   keep if dist <= cutoff && dist > 0.                                      */
/* box: device pointer to a 3x3 row-major lower-triangular cell (rows a, b, c */
/* as in the reference), or NULL for open boundaries.                          */
/* ------------------------------------------------------------------------ */

#define MNX_NLIST_HALF 0 /* unordered pairs, i > j (reference half list) */
#define MNX_NLIST_FULL 1 /* ordered pairs, i != j */

#define MNX_NLIST_COMPACT 0    /* pairs sorted by (i, j) at slots 0..total-1 */
#define MNX_NLIST_TRIANGULAR 1 /* HALF only: pair (i, j) at slot i*(i-1)/2 + j
                                  (reference max_num_pairs == -1 layout) */

size_t mnx_nlist_workspace_bytes(int64_t num_atoms);

/* Stage 1: bin atoms into cells and count pairs.  Writes the total pair count
 * to *d_total (device int64).  The workspace keeps the bins for stage 2. */
int mnx_nlist_count_f32(const float* pos, int64_t num_atoms, double cutoff, const float* box,
                        int32_t mode, void* workspace, size_t workspace_bytes, int64_t* d_total,
                        mnx_stream_t stream);
int mnx_nlist_count_f64(const double* pos, int64_t num_atoms, double cutoff, const double* box,
                        int32_t mode, void* workspace, size_t workspace_bytes, int64_t* d_total,
                        mnx_stream_t stream);

/* Stage 2: write pairs sorted by (i, j) into slots [0, capacity); slots past
 * the pair count get i = j = -1 and NaN geometry (the reference padding).
 * idx_i / idx_j: int32 [capacity]; deltas (d above) [capacity][3];
 * distances [capacity]; shifts [capacity][3] = image offset added to pos[j]
 * (d = pos[i] - (pos[j] + shift)).  Any output pointer may be NULL. */
int mnx_nlist_emit_f32(const float* pos, int64_t num_atoms, double cutoff, const float* box,
                       int32_t mode, int32_t layout, const void* workspace, size_t workspace_bytes,
                       int64_t capacity, int32_t* idx_i, int32_t* idx_j, float* deltas,
                       float* distances, float* shifts, mnx_stream_t stream);
int mnx_nlist_emit_f64(const double* pos, int64_t num_atoms, double cutoff, const double* box,
                       int32_t mode, int32_t layout, const void* workspace, size_t workspace_bytes,
                       int64_t capacity, int32_t* idx_i, int32_t* idx_j, double* deltas,
                       double* distances, double* shifts, mnx_stream_t stream);

/* Reverse-mode of get_neighbor_pairs w.r.t. positions (get_neighbor_pairs.cu:81-102):
 * grad_pos[i] += g_d + d/dist * g_dist, grad_pos[j] -= the same, over valid slots
 * (idx_i >= 0).  grad_pos must be zeroed by the caller. */
int mnx_nlist_backward_f32(const int32_t* idx_i, const int32_t* idx_j, const float* deltas,
                           const float* distances, const float* grad_deltas,
                           const float* grad_distances, int64_t num_slots, int64_t num_atoms,
                           float* grad_pos, mnx_stream_t stream);
int mnx_nlist_backward_f64(const int32_t* idx_i, const int32_t* idx_j, const double* deltas,
                           const double* distances, const double* grad_deltas,
                           const double* grad_distances, int64_t num_slots, int64_t num_atoms,
                           double* grad_pos, mnx_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Receiver CSR of an edge list (the gather/scatter index behind ConvTP's     */
/* indices_1 / indices_out, tensor_product.py:101-111).                       */
/* edge_index: int64 [E][2], column 0 = sender, column 1 = receiver.          */
/* row_ptr: int32 [N+1]; perm: int32 [E] = edge ids grouped by receiver, in   */
/* ascending edge id within a receiver (deterministic); senders_sorted: int32 */
/* [E] = sender of perm[k].  Edges with an index outside [0, N) are left out  */
/* and counted in *d_invalid (device int32, may be NULL); the kernels below   */
/* then leave their grad_Y / grad_w rows untouched, so callers must reject    */
/* such edge lists.                                                           */
/* ------------------------------------------------------------------------ */
size_t mnx_csr_workspace_bytes(int64_t num_nodes, int64_t num_edges);
int mnx_csr_build(const int64_t* edge_index, int64_t num_edges, int64_t num_nodes, int32_t* row_ptr,
                  int32_t* perm, int32_t* senders_sorted, int32_t* d_invalid, void* workspace,
                  size_t workspace_bytes, mnx_stream_t stream);

/* The same CSR build without a workspace and without any allocation: no
 * counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Its scratch (about 17 MB: per-receiver counters, scan
 * tiles, flags) is one static device array per GPU, held until the process
 * ends and cleared by fill kernels on every call; num_nodes above
 * MNX_CSR_NOALLOC_MAX_NODES is rejected with MNX_ERR_INVALID.  All calls on
 * one GPU share that array: calls that overlap on one GPU (concurrent
 * streams or host threads) race and must be serialised by the caller. */
#define MNX_CSR_NOALLOC_MAX_NODES 2097152
int mnx_csr_build_noalloc(const int64_t* edge_index, int64_t num_edges, int64_t num_nodes, int32_t* row_ptr,
                          int32_t* perm, int32_t* senders_sorted, int32_t* d_invalid, mnx_stream_t stream);

/* Reverse edges of a directed edge list, for work that depends on an edge only
 * through per-edge features shared by the two directions of an undirected
 * pair (the radial MLP of src/molrep/interaction/radial_mlp.py:38-93 evaluated
 * per edge for ConvTP, tensor_product.py:72-79,101-111, sees only the
 * distance).  rev[e] (int32 [E]) = the one edge e2 != e with edge_index[e2] =
 * (edge_index[e][1], edge_index[e][0]) whose feats row [num_feats] equals
 * feats[e] bit for bit; -1 if there is none or more than one, each such edge
 * counted in d_bad[0] (device int32 [2], both words cleared by the caller;
 * d_bad[1] is scratch).  row_ptr / perm / senders_sorted: the receiver CSR of
 * edge_index (mnx_csr_build).  Binary search per edge when every receiver
 * segment lists its senders in ascending order (checked on the device), a
 * scan of the segment otherwise. */
int mnx_edge_reverse(const int64_t* edge_index, int64_t num_edges, int64_t num_nodes, const int32_t* row_ptr,
                     const int32_t* perm, const int32_t* senders_sorted, const float* feats, int32_t num_feats,
                     int32_t* rev, int32_t* d_bad, mnx_stream_t stream);

/* The pairs themselves (num_edges even): after mnx_edge_reverse, the lead of
 * each pair is its lower edge id; pair P (in ascending lead order) has
 * lead[P] (int64 [E/2]) and pairs[P] = (lead, partner) (int32 [E/2][2]), and
 * wrow[e] (int32 [E]) is the pair of edge e.  d_bad[0] (device int32 [2],
 * both words cleared by the caller) counts edges without a partner or whose
 * partner does not point back; when it is non-zero the outputs are not a
 * pairing (every write stays inside them).  Workspace:
 * mnx_edge_pairs_workspace_bytes. */
/* d_bad[0] (device int32, cleared by the caller) += the number of pairs
 * (int32 [num_pairs][2], mnx_edge_pairs) whose two edges' feats rows differ in
 * any bit: a pairing built once per edge list, checked again for new features. */
int mnx_edge_pairs_verify(const int32_t* pairs, int64_t num_pairs, const float* feats, int32_t num_feats,
                          int32_t* d_bad, mnx_stream_t stream);

/* Rows of F floats by index (the radial features of each pair's lead edge,
 * feeding the radial MLP of radial_mlp.py:38-93 once per pair):
 * dst[i] = src[idx[i]] (gather) and dst[idx[i]] = src[i] (its adjoint for
 * distinct indices; rows not indexed are left as they are); idx int64 [n]. */
int mnx_gather_rows_f32(const float* src, const int64_t* idx, int64_t n, int32_t F, float* dst,
                        mnx_stream_t stream);
int mnx_scatter_rows_f32(const float* src, const int64_t* idx, int64_t n, int32_t F, float* dst,
                         mnx_stream_t stream);
/* dst[i] = src[pairs[i][0]] + src[pairs[i][1]] for rows of F floats (F a multiple of 4, src and  */
/* dst 16-byte aligned): the per-pair sum of per-edge rows (the output layer's input gradient     */
/* of a pair from its two edges').  No counterpart in the reference (its MLP runs per edge).     */
int mnx_pair_sum_rows_f32(const float* src, const int32_t* pairs, int64_t num_pairs, int32_t F, float* dst,
                          mnx_stream_t stream);

size_t mnx_edge_pairs_workspace_bytes(int64_t num_edges);
int mnx_edge_pairs(const int64_t* edge_index, int64_t num_edges, int64_t num_nodes, const int32_t* row_ptr,
                   const int32_t* perm, const int32_t* senders_sorted, const float* feats, int32_t num_feats,
                   int32_t* wrow, int64_t* lead, int32_t* pairs, int32_t* d_bad, void* workspace,
                   size_t workspace_bytes, mnx_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Segment sums over a CSR (row_ptr / perm from mnx_csr_build of the rows'    */
/* segment ids): replaces the scatter_add_ of molix.F.scatter_sum / batch_add */
/* (src/molix/F/scatter.py:13-51) and MessageAggregation's neighbour sum      */
/* (src/molrep/interaction/aggregation.py:93-117):                            */
/*   out[n][:] = sum_{k in [row_ptr[n], row_ptr[n+1])} w[perm[k]] values[perm[k]][:] */
/* values [num_rows][dim], weights [num_rows] or NULL (all ones), out          */
/* [num_segments][dim] (overwritten; no atomics, a fixed summation order).    */
/* ------------------------------------------------------------------------ */
int mnx_segment_sum_f32(const float* values, int64_t num_rows, int32_t dim, const int32_t* row_ptr,
                        const int32_t* perm, const float* weights, int64_t num_segments, float* out,
                        mnx_stream_t stream);
/* Its gradients: grad_values[r][:] = w[r] grad_out[index[r]][:] and grad_weights[r] =
 * <values[r], grad_out[index[r]]> (either output may be NULL; rows whose index lies outside
 * [0, num_segments) get zeros).  index: int64 [num_rows]. */
int mnx_segment_sum_bwd_f32(const float* grad_out, const int64_t* index, const float* weights, const float* values,
                            int64_t num_rows, int32_t dim, int64_t num_segments, float* grad_values,
                            float* grad_weights, mnx_stream_t stream);

/* Nodes grouped by class (a stable counting sort; no atomics, no host sync):
 * order [num_nodes] = node ids, classes ascending (classes outside
 * [0, num_classes) last, as class num_classes), ascending node id within a
 * class; class_start [num_classes + 2] = where each class begins in order.
 * The grouping that cuet.Linear(weight_classes=S, method="indexed_linear")
 * (src/molrep/interaction/element_update.py:101-109) and the per-element
 * weights of cuet.SymmetricContraction (symmetric_contraction.py:100-109)
 * need; replaces the torch.argsort of node elements. */
#define MNX_CLASS_GROUPS_MAX_CLASSES 4096
size_t mnx_class_groups_workspace_bytes(int64_t num_nodes, int32_t num_classes);
int mnx_class_groups(const int64_t* classes, int64_t num_nodes, int32_t num_classes, int32_t* order,
                     int32_t* class_start, void* workspace, size_t workspace_bytes, mnx_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Real spherical harmonics, component normalisation, l <= 3, input vectors   */
/* normalised inside (replaces cuet.SphericalHarmonics(ls, normalize=True),   */
/* src/molrep/embedding/angular.py:89,104).  Output [n][(l_max+1)^2].         */
/* ------------------------------------------------------------------------ */
int mnx_sh_fwd_f32(const float* vec, int64_t n, int32_t l_max, float* out, mnx_stream_t stream);
/* grad_vec[n][3] = d<grad_out, Y(vec)>/d vec (overwritten). */
int mnx_sh_bwd_f32(const float* vec, const float* grad_out, int64_t n, int32_t l_max,
                   float* grad_vec, mnx_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Channelwise tensor product fused with gather/scatter (replaces             */
/* cuet.ChannelWiseTensorProduct(..., layout=ir_mul, shared_weights=False,    */
/* internal_weights=False) called with indices_1 / indices_out / size_out,    */
/* src/molrep/interaction/tensor_product.py:72-79,104-111).                   */
/*                                                                            */
/*   out[r] = sum_{e: recv(e)=r} TP(x[send(e)], Y[e]; w[e])                   */
/*                                                                            */
/* A configuration is the set of l's in irreps_in1 (uniform multiplicity C,   */
/* natural parity), in irreps_in2 (the harmonics) and in the output filter,   */
/* each given as a bit mask over l = 0..3.  mnx_tp_config returns its id or   */
/* -1 when no kernel was compiled for it.  Layouts (ir_mul):                  */
/*   x   [N][sum_l1 (2l1+1) * C]        Y [E][sum_l2 (2l2+1)]                 */
/*   w   [E][num_paths * C]  (path-major)  out [N][sum_paths (2l3+1) * C]     */
/* ------------------------------------------------------------------------ */
int mnx_tp_config(int32_t in_mask, int32_t sh_mask, int32_t out_mask);
/* info[0] = num_paths, info[1] = x comps per channel, info[2] = Y comps,
 * info[3] = out comps per channel. */
int mnx_tp_config_info(int32_t config, int32_t* info);

int mnx_tp_fwd_f32(int32_t config, int32_t channels, const float* x, const float* Y,
                   const float* w, const int32_t* row_ptr, const int32_t* perm,
                   const int32_t* senders_sorted, int64_t num_nodes, int64_t num_edges, float* out,
                   mnx_stream_t stream);

/* Gradients of <grad_out, out> w.r.t. x, Y and w.  grad_x is accumulated with
 * atomics and must be zeroed by the caller; grad_Y and grad_w are overwritten.
 * Any of grad_x / grad_Y / grad_w may be NULL when not needed. */
size_t mnx_tp_bwd_workspace_bytes(int32_t config, int32_t channels, int64_t num_edges);
int mnx_tp_bwd_f32(int32_t config, int32_t channels, const float* x, const float* Y,
                   const float* w, const float* grad_out, const int32_t* row_ptr,
                   const int32_t* perm, const int32_t* senders_sorted, int64_t num_nodes,
                   int64_t num_edges, float* grad_x, float* grad_Y, float* grad_w,
                   void* workspace, size_t workspace_bytes, mnx_stream_t stream);

/* The same gradients, walked by sender, without atomics (bitwise reproducible):
 * the CSR of edge_index[:, 0] (mnx_csr_build on the column-swapped edge list:
 * s_row_ptr [N+1], s_perm = edge ids, s_receivers = their receivers).  grad_x,
 * grad_Y and grad_w are overwritten (no zeroing needed).  Same results as
 * mnx_tp_bwd_f32 up to fp32 summation order; slower on large graphs (weight rows
 * are visited in sender order).  Replaces the same reference call (ConvTP
 * backward, tensor_product.py:101-111). */
int mnx_tp_bwd_sender_f32(int32_t config, int32_t channels, const float* x, const float* Y,
                          const float* w, const float* grad_out, const int32_t* s_row_ptr,
                          const int32_t* s_perm, const int32_t* s_receivers, int64_t num_nodes,
                          int64_t num_edges, float* grad_x, float* grad_Y, float* grad_w,
                          mnx_stream_t stream);

/* The backward one path group at a time (groups = paths sharing the l of irreps_in1;
 * mnx_tp_group_paths fills bounds[0..ngroups] with their path ranges and returns ngroups): group
 * `group`'s kernel of mnx_tp_bwd_rows_f32, writing grad_w for the group's columns
 * [bounds[g] * C, bounds[g + 1] * C) and accumulating grad_x; its grad_Y partials go to the
 * workspace (mnx_tp_bwd_workspace_bytes; NULL: no grad_Y), summed by mnx_tp_bwd_reduce_gy_f32
 * once every group has run.  Lets a caller start consuming one group's grad_w (on another stream)
 * while the next group runs. */
int mnx_tp_group_paths(int32_t config, int32_t* bounds);
int mnx_tp_bwd_group_rows_f32(int32_t config, int32_t channels, int32_t group, const float* x, const float* Y,
                              const float* w, const int32_t* wrow, const float* grad_out, const int32_t* row_ptr,
                              const int32_t* perm, const int32_t* senders_sorted, int64_t num_nodes,
                              int64_t num_edges, float* grad_x, float* grad_w, void* workspace,
                              size_t workspace_bytes, mnx_stream_t stream);
int mnx_tp_bwd_reduce_gy_f32(int32_t config, int32_t channels, int64_t num_edges, const void* workspace,
                             size_t workspace_bytes, float* grad_Y, mnx_stream_t stream);

/* The three calls above with the per-edge weights taken from row wrow[e] of w
 * (int32 [E], any number of rows) instead of row e: edges whose weights are
 * equal share one row, e.g. the two directions of an undirected pair, whose
 * radial MLP inputs (the distance) are the same (the weights the reference
 * computes per directed edge, radial_mlp.py:76-82, fed to ConvTP,
 * tensor_product.py:72-79,101-111).  grad_w is still per directed edge
 * ([E][num_paths*C]); summing it over the edges of a row is the caller's. */
int mnx_tp_fwd_rows_f32(int32_t config, int32_t channels, const float* x, const float* Y,
                        const float* w, const int32_t* wrow, const int32_t* row_ptr,
                        const int32_t* perm, const int32_t* senders_sorted, int64_t num_nodes,
                        int64_t num_edges, float* out, mnx_stream_t stream);
int mnx_tp_bwd_rows_f32(int32_t config, int32_t channels, const float* x, const float* Y,
                        const float* w, const int32_t* wrow, const float* grad_out,
                        const int32_t* row_ptr, const int32_t* perm, const int32_t* senders_sorted,
                        int64_t num_nodes, int64_t num_edges, float* grad_x, float* grad_Y,
                        float* grad_w, void* workspace, size_t workspace_bytes, mnx_stream_t stream);
int mnx_tp_bwd_sender_rows_f32(int32_t config, int32_t channels, const float* x, const float* Y,
                               const float* w, const int32_t* wrow, const float* grad_out,
                               const int32_t* s_row_ptr, const int32_t* s_perm,
                               const int32_t* s_receivers, int64_t num_nodes, int64_t num_edges,
                               float* grad_x, float* grad_Y, float* grad_w, mnx_stream_t stream);


/* ------------------------------------------------------------------------ */
/* Particle-mesh Ewald (replaces torch.ops.molix.pme_reciprocal and           */
/* pme_direct: molix_library.cpp:29-41, CPU pme_cpu.cpp:95-458, CUDA          */
/* pme_cuda.cu:106-523).  box: device 3x3 lower-triangular cell.  The caller  */
/* runs the 3-D real FFTs (rocFFT) between the stages:                        */
/*   spread -> rfftn -> convolve (energy)   and   irfftn(norm=forward) -> gather */
/* Spline orders 3..8 (the reference CUDA path: 4, 5).                        */
/* ------------------------------------------------------------------------ */
/* grid[gx][gy][gz] (overwritten) = sum_atoms q sqrt(coulomb) B(x) B(y) B(z)  (pme_cpu.cpp:240-256).
 * Computed as a gather over 8^3-point mesh bricks with atoms binned by brick: no atomics, every
 * point written once, a fixed summation order (deterministic). */
size_t mnx_pme_spread_workspace_bytes(int64_t num_atoms, int32_t gx, int32_t gy, int32_t gz);
int mnx_pme_spread_f32(const float* pos, const float* charges, const float* box, int64_t num_atoms,
                       int32_t gx, int32_t gy, int32_t gz, int32_t order, double coulomb, float* grid,
                       void* workspace, size_t workspace_bytes, mnx_stream_t stream);
int mnx_pme_spread_f64(const double* pos, const double* charges, const double* box, int64_t num_atoms,
                       int32_t gx, int32_t gy, int32_t gz, int32_t order, double coulomb, double* grid,
                       void* workspace, size_t workspace_bytes, mnx_stream_t stream);
/* In place on the half spectrum cgrid[gx][gy][gz/2+1] (interleaved re, im):
 * G *= exp(-pi^2 m^2/alpha^2) / (pi V m^2 xm ym zm), m = 0 term zeroed;
 * *energy = 1/2 sum scale |G|^2 eterm before the multiply (pme_cpu.cpp:263-294, 378). */
size_t mnx_pme_convolve_workspace_bytes(int32_t gx, int32_t gy, int32_t gz);
int mnx_pme_convolve_f32(float* cgrid, const float* box, int32_t gx, int32_t gy, int32_t gz, double alpha,
                         const float* xmoduli, const float* ymoduli, const float* zmoduli,
                         float* energy, void* workspace, size_t workspace_bytes, mnx_stream_t stream);
int mnx_pme_convolve_f64(double* cgrid, const double* box, int32_t gx, int32_t gy, int32_t gz,
                         double alpha, const double* xmoduli, const double* ymoduli,
                         const double* zmoduli, double* energy, void* workspace,
                         size_t workspace_bytes, mnx_stream_t stream);
/* From the back-transformed grid: dE/dpos [n][3] and dE/dq [n] (pme_cpu.cpp:311-343). */
int mnx_pme_gather_f32(const float* pos, const float* charges, const float* box, int64_t num_atoms,
                       const float* grid, int32_t gx, int32_t gy, int32_t gz, int32_t order,
                       double coulomb, float* dpos, float* dq, mnx_stream_t stream);
int mnx_pme_gather_f64(const double* pos, const double* charges, const double* box, int64_t num_atoms,
                       const double* grid, int32_t gx, int32_t gy, int32_t gz, int32_t order,
                       double coulomb, double* dpos, double* dq, mnx_stream_t stream);
/* Real-space sum over a pair list neighbors[2][num_pairs] (i = -1 padding skipped) minus the
 * erf term of excluded pairs; exclusions[n][max_excl] descending, -1 padded (pme_cpu.cpp:95-164).
 * *energy, dpos [n][3], dq [n] are overwritten; dpos and dq may both be NULL (energy only, no
 * atomics).  The reference computes both in its forward (pme_cpu.cpp:168-205); the torch op
 * here computes the energy in the forward and the derivatives in the backward. */
size_t mnx_pme_direct_workspace_bytes(int64_t num_atoms, int64_t num_pairs);
int mnx_pme_direct_f32(const float* pos, const float* charges, int64_t num_atoms, const int32_t* neighbors,
                       int64_t num_pairs, const float* deltas, const float* distances,
                       const int32_t* exclusions, int32_t max_excl, double alpha, double coulomb,
                       float* energy, float* dpos, float* dq, void* workspace, size_t workspace_bytes,
                       mnx_stream_t stream);
int mnx_pme_direct_f64(const double* pos, const double* charges, int64_t num_atoms,
                       const int32_t* neighbors, int64_t num_pairs, const double* deltas,
                       const double* distances, const int32_t* exclusions, int32_t max_excl,
                       double alpha, double coulomb, double* energy, double* dpos, double* dq,
                       void* workspace, size_t workspace_bytes, mnx_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Symmetric contraction of scalar channels, as the reference configures it  */
/* (cuet.SymmetricContraction("{D}x0e" -> "{D}x0e", original_mace=True),     */
/* src/molrep/interaction/symmetric_contraction.py:90-109):                  */
/*   out[n][c] = sum_{k=1..nu} W[types[n]][k-1][c] x[n][c]^k                 */
/* W [S][nu][D], S <= 16, nu <= 4.  grad_W is accumulated (zero it first).   */
/* ------------------------------------------------------------------------ */
int mnx_sc_scalar_fwd_f32(const float* x, const int64_t* types, const float* W, int64_t num_nodes,
                          int32_t channels, int32_t num_elements, int32_t degree, float* out,
                          mnx_stream_t stream);
int mnx_sc_scalar_bwd_f32(const float* x, const int64_t* types, const float* W, const float* grad_out,
                          int64_t num_nodes, int32_t channels, int32_t num_elements, int32_t degree,
                          float* grad_x, float* grad_W, mnx_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Equivariant symmetric contraction (the MACE product basis that the        */
/* reference reaches through cuet.SymmetricContraction,                      */
/* src/molrep/interaction/symmetric_contraction.py:94-109, here for irreps   */
/* in = C x (0e+1o+..+l_in), out = C x (0e [+1o]), correlation 1..3):        */
/*   out[n][L,M][c] = sum_{nu,k} W[types[n]][p(L,nu,k)][c]                   */
/*                    sum_{i1..inu} U_{L,nu,k}[M][i1..inu] A[n][i1][c]..     */
/* with the basis U of the library (symmetrised coupling chains,             */
/* Gram-Schmidt in a fixed order).  ir_mul layouts: A [N][(l_in+1)^2][C],    */
/* out [N][(L_out+1)^2][C]; W [S][paths][C].  Nodes with types outside       */
/* [0, S) give zero output and zero grad_A.                                  */
/* mnx_sc_config returns the config id (or -1); info = {dim_in, dim_out,     */
/* paths, coefficients}.  Backward: order is a permutation of [0, N) that    */
/* groups nodes by element (NULL = identity; only the number of atomics      */
/* depends on it); grad_W is accumulated (zero it first); either gradient    */
/* pointer may be NULL.                                                      */
/* ------------------------------------------------------------------------ */
int mnx_sc_config(int32_t l_in, int32_t l_out, int32_t correlation);
int mnx_sc_config_info(int32_t config, int32_t* info);
int mnx_sc_fwd_f32(int32_t config, const float* A, const int64_t* types, const float* W,
                   int64_t num_nodes, int32_t channels, int32_t num_elements, float* out,
                   mnx_stream_t stream);
int mnx_sc_bwd_f32(int32_t config, const float* A, const int64_t* types, const float* W,
                   const float* grad_out, const int32_t* order, int64_t num_nodes,
                   int32_t channels, int32_t num_elements, float* grad_A, float* grad_W,
                   mnx_stream_t stream);
/* Second order of the contraction (force-matching training): with seeds   */
/* seed_A [N][ni*C] and seed_W [S][paths][C] (either may be NULL: zero) on   */
/* the first-order gradients of <grad_out, B>, the gradients of              */
/* L2 = <seed_A, grad_A> + <seed_W, grad_W> with respect to grad_out         */
/* (d_grad_out [N][no*C], overwritten), A (d_A, overwritten) and W (d_W,     */
/* accumulated: zero it first); NULL outputs are skipped.  order as for     */
/* mnx_sc_bwd_f32.  No counterpart in the reference's ops (cuequivariance    */
/* provides it for symmetric_contraction.py:94-109).                        */
int mnx_sc_bwd2_f32(int32_t config, const float* A, const int64_t* types, const float* W, const float* grad_out,
                    const float* seed_A, const float* seed_W, const int32_t* order, int64_t N, int32_t C,
                    int32_t S, float* d_grad_out, float* d_A, float* d_W, mnx_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Equivariant (ir_mul) block linear, one output irrep block per call        */
/* (replaces the cuet.Linear of src/molrep/interaction/linear.py:43-105):    */
/*   out[n*out_stride + out_off + i*out_comp + p] = sum_k A_k * w[k][p]       */
/* for nodes n < R, components i < d, columns p < N, where k runs over the   */
/* nseg input segments in order, segment s contributing seg_len[s] values    */
/* a[n*a_stride + seg_col[s] + i*seg_comp[s] + 0..seg_len[s]-1].  The K x N  */
/* weights (K = sum seg_len, pre-scaled by the caller) come in the kernel's  */
/* fragment order: with T = N >= 128 ? 4 : ceil(N/32) tiles, element         */
/* [y][chunk][q][t][lane][i] (y < ceil(N/32T), chunk < ceil(K/64), q < 4,    */
/* t < T, lane < 64, i < 8) holds W[64 chunk + 16q + 8(lane/32) + i]         */
/* [32T y + 32t + lane%32], zero outside K x N; mnx_block_linear_frag_floats */
/* gives its length.  Products are fp32-accurate (three-way bf16 splits of   */
/* both operands, six partial products accumulated in fp32 on the matrix    */
/* cores).  nseg = 0 writes zeros.  seg_len multiples of 8;                  */
/* a_stride, seg_col, seg_comp multiples of 4; a and w 16-byte aligned; at   */
/* most 8 segments.  Segment arrays are host memory.                        */
/* ------------------------------------------------------------------------ */
int64_t mnx_block_linear_frag_floats(int32_t K, int32_t N);
int mnx_block_linear_f32(const float* a, int64_t a_stride, int32_t nseg, const int64_t* seg_col,
                         const int32_t* seg_comp, const int32_t* seg_len, const float* w, int32_t N,
                         int64_t R, int32_t d, float* out, int64_t out_stride, int64_t out_off,
                         int32_t out_comp, mnx_stream_t stream);
/* The same block linear with one weight set per node class: the indexed     */
/* linear of ElementUpdate (cuet.Linear(weight_classes=S,                     */
/* method="indexed_linear"), src/molrep/interaction/element_update.py:        */
/* 101-109,147-158).  Node n uses the weights of its class; the caller passes */
/* the nodes grouped by class, order [R] (int32 node ids, classes ascending,  */
/* ascending node id within a class, nodes whose class lies outside [0, S)    */
/* last) and class_start [S + 2] (position in order where class s begins,     */
/* s = 0..S, with s = S the out-of-range nodes, and class_start[S + 1] = R).  */
/* w points at class 0's fragment-ordered weights (layout as above);         */
/* consecutive classes are w_class_stride floats apart.  Out-of-range nodes  */
/* get zero output.  No host synchronisation is needed to build the inputs.  */
int mnx_indexed_block_linear_f32(const float* a, int64_t a_stride, int32_t nseg, const int64_t* seg_col,
                                 const int32_t* seg_comp, const int32_t* seg_len, const float* w,
                                 int64_t w_class_stride, int32_t num_classes, const int32_t* order,
                                 const int32_t* class_start, int32_t N, int64_t R, int32_t d, float* out,
                                 int64_t out_stride, int64_t out_off, int32_t out_comp, mnx_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Bond vectors diff[e] = pos[ei[e][1]] - pos[ei[e][0]] - shifts[e] (shifts  */
/* may be NULL) for edge_index rows [sender, receiver], the reference's      */
/* bond_diff = pos[target] - pos[source] (src/molix/data/tasks/              */
/* neighbor_list.py:86-95), and its gradient grad_pos [n][3] (overwritten)   */
/* = per atom, sum of grad_diff over its incoming minus its outgoing edges.  */
/* Edges with an endpoint outside [0, n) give NaN and no gradient.           */
/* ------------------------------------------------------------------------ */
int mnx_bond_vectors_f32(const float* pos, int64_t num_atoms, const int64_t* edge_index,
                         const float* shifts, int64_t num_edges, float* diff, mnx_stream_t stream);
int mnx_bond_vectors_bwd_f32(const int64_t* edge_index, const float* grad_diff, int64_t num_edges,
                             int64_t num_atoms, float* grad_pos, mnx_stream_t stream);

/* Radial edge embedding of MACE: the Bessel basis times the cutoff envelope,
 *   out[e][k] = c(r[e]) (phi_k(r[e]) - mu[k]) / sigma[k],
 *   phi_k(r) = sqrt(2 / r_cut) sin((k+1) pi r / r_cut) / (r + eps),  k < num_radial,
 * c = 1 (cutoff 0), 0.5 (cos(pi r / r_cut) + 1) (cutoff 1) or the polynomial
 * envelope of the given exponent (cutoff 2), 0 for r >= r_cut; mu / sigma both
 * NULL for the unnormalised basis.  out [num_edges][num_radial]; the backward
 * gives grad_r [num_edges] from grad [num_edges][num_radial].  Replaces
 * BesselRBF(r) * cutoff(r) (src/molrep/embedding/radial.py:36-148,
 * cutoff.py:23-161, src/molzoo/mace.py:180-182).  num_radial <= 32. */
int mnx_bessel_cutoff_f32(const float* r, int64_t num_edges, int32_t num_radial, double r_cut, double eps,
                          const float* mu, const float* sigma, int32_t cutoff, int32_t exponent, float* out,
                          mnx_stream_t stream);
int mnx_bessel_cutoff_bwd_f32(const float* r, int64_t num_edges, int32_t num_radial, double r_cut, double eps,
                              const float* mu, const float* sigma, int32_t cutoff, int32_t exponent,
                              const float* grad, float* grad_r, mnx_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Hidden stack of the radial weight MLP (replaces mlp[:-1] of               */
/* RadialWeightMLP, src/molrep/interaction/radial_mlp.py:38-93:              */
/* [Linear(in, hidden) -> SiLU] x layers) for the forward and the gradient   */
/* with respect to the edge features.  raw parameters: per layer W_j         */
/* [hidden][in_j] (torch.nn.Linear layout) then b_j [hidden], contiguous;    */
/* mnx_radial_pack_f32 rearranges them once into frag                        */
/* [mnx_radial_frag_floats(...)] floats (16-byte aligned; hidden layers as   */
/* power-of-two row scales and two fp16 planes of the scaled weights, for    */
/* near-fp32 split-fp16 products), which the fwd and bwd kernels read.  feats [E][kin], h [E][hidden], grad_feats [E][kin]     */
/* (overwritten).  kin <= 64; hidden 32 or 64 with 1..4 layers, or 128 with  */
/* 1..2 layers (else MNX_ERR_UNSUPPORTED; the size queries return -1).       */
/* ------------------------------------------------------------------------ */
int64_t mnx_radial_raw_floats(int32_t kin, int32_t hidden, int32_t layers);
int64_t mnx_radial_frag_floats(int32_t kin, int32_t hidden, int32_t layers);
int mnx_radial_pack_f32(const float* raw, int32_t kin, int32_t hidden, int32_t layers, float* frag,
                        mnx_stream_t stream);
int mnx_radial_fwd_f32(const float* feats, int64_t num_edges, int32_t kin, int32_t hidden,
                       int32_t layers, const float* frag, float* h, mnx_stream_t stream);
int mnx_radial_bwd_f32(const float* feats, int64_t num_edges, int32_t kin, int32_t hidden,
                       int32_t layers, const float* frag, const float* grad_h, float* grad_feats,
                       mnx_stream_t stream);

/* Second derivative of the radial MLP's SiLU activations (nn.SiLU between   */
/* the hidden Linears, src/molrep/interaction/radial_mlp.py:76-82, twice     */
/* differentiated by a force-matching loss): for gx = g s'(x), s = SiLU,     */
/* grad_x = gg g s''(x) and grad_grad_out = gg s'(x), elementwise over n     */
/* values (16-byte aligned pointers; outputs overwritten).                   */
int mnx_silu_bwd2_f32(const float* x, const float* grad, const float* grad_grad, int64_t n,
                      float* grad_x, float* grad_grad_out, mnx_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Output layer of the radial weight MLP (the last Linear of                 */
/* RadialWeightMLP, src/molrep/interaction/radial_mlp.py:38-93): per-edge    */
/* tensor-product weights w[e][n] = sum_k h[e][k] W[n][k] + bias[n]          */
/* (mnx_edge_weights_f32; bias may be NULL) and the input gradient           */
/* grad_h[e][k] = sum_n grad_w[e][n] W[n][k] (mnx_edge_weights_bwd_f32,      */
/* overwritten).  W is the torch.nn.Linear weight [N][K].  Products are      */
/* near-fp32 (relative error per product below 3 * 2^-22): rows of h and    */
/* grad_w and output columns of W are scaled by powers of two, each scaled   */
/* value is split into two fp16 parts and three partial products are        */
/* accumulated in fp32 on the matrix cores; the scales are undone exactly.   */
/* mnx_edge_weights_pack_f32 scales, splits and arranges W once into frag    */
/* [mnx_edge_weights_frag_elems(K, N, backward)] 16-bit values (16-byte      */
/* aligned: the fp16 planes, then the column scales as fp32), backward = 0  */
/* for the forward layout, 1 for the backward one.                           */
/* K in {16, 32, 64, 128} (else MNX_ERR_UNSUPPORTED; the size query returns  */
/* -1); the backward needs N % 8 == 0; h and grad_w 16-byte aligned.         */
/* ------------------------------------------------------------------------ */
int64_t mnx_edge_weights_frag_elems(int32_t K, int32_t N, int32_t backward);
int mnx_edge_weights_pack_f32(const float* weight, int32_t K, int32_t N, int32_t backward, uint16_t* frag,
                              mnx_stream_t stream);
int mnx_edge_weights_f32(const float* h, int64_t num_edges, int32_t K, const uint16_t* frag,
                         const float* bias, int32_t N, float* w, mnx_stream_t stream);
int mnx_edge_weights_bwd_f32(const float* grad_w, int64_t num_edges, int32_t N, const uint16_t* frag,
                             int32_t K, float* grad_h, mnx_stream_t stream);
/* The forward on selected rows of h: w[i] = W h[rows[i]] + b for i < num_rows
 * (rows int32 [num_rows]; NULL: rows[i] = i), e.g. the lead edge of each
 * undirected pair (mnx_edge_reverse). */
int mnx_edge_weights_rows_f32(const float* h, const int32_t* rows, int64_t num_rows, int32_t K,
                              const uint16_t* frag, const float* bias, int32_t N, float* w, mnx_stream_t stream);
/* The input gradient of a layer whose rows are shared by two directed edges
 * (mnx_edge_reverse): grad_h[i][k] = sum_n (grad_w[pairs[i][0]][n] +
 * grad_w[pairs[i][1]][n]) W[n][k] for the num_pairs rows of h, pairs int32
 * [num_pairs][2], grad_w per directed edge.  With pairs = NULL it is
 * mnx_edge_weights_bwd_f32 (num_pairs = num_edges). */
int mnx_edge_weights_bwd_pairs_f32(const float* grad_w, const int32_t* pairs, int64_t num_pairs, int32_t N,
                                   const uint16_t* frag, int32_t K, float* grad_h, mnx_stream_t stream);
/* The same over a column slice of the gradient: grad_w points at the slice's first column, rows
 * ld floats apart (ld >= N, a multiple of 4), N the slice width and frag W's matching rows
 * [N][K] packed for the backward; pairs may be NULL.  accumulate != 0 adds the product to grad_h
 * instead of overwriting it, so slices taken in turn (e.g. as the tensor product's backward
 * finishes each path group's columns) sum to the whole product in launch order. */
int mnx_edge_weights_bwd_cols_f32(const float* grad_w, int64_t ld, const int32_t* pairs, int64_t num_rows,
                                  int32_t N, const uint16_t* frag, int32_t K, float* grad_h, int32_t accumulate,
                                  mnx_stream_t stream);
/* The same written into (or, accumulate != 0, added to) a column block of a wider result:
 * grad_h's rows ldh floats apart (ldh >= K, a multiple of 4; grad_h 16-byte aligned), e.g. the
 * scalar columns of an edge tensor's gradient taking the latent layer's input gradient in place
 * (src/molzoo/allegro.py:469-473).  mnx_edge_weights_bwd_cols_f32 is this with ldh = K. */
int mnx_edge_weights_bwd_into_f32(const float* grad_w, int64_t ld, const int32_t* pairs, int64_t num_rows,
                                  int32_t N, const uint16_t* frag, int32_t K, float* grad_h, int64_t ldh,
                                  int32_t accumulate, mnx_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Fused weight gradient of the tensor product and the output layer of the    */
/* radial weight MLP (the per-edge weights w[e] = W h[e] + b of               */
/* src/molrep/interaction/radial_mlp.py:76-82 consumed by ConvTP,             */
/* tensor_product.py:72-79,101-111):                                          */
/*   grad_h[e][k] = sum_n gw[e][n] W[n][k],  n = p * C + c,                    */
/*   gw[e][n] = d<grad_out, tp_scatter(x, Y, w)> / d w[e][n]                   */
/* without materialising gw (E x num_paths*C): it is produced per edge in     */
/* registers from x [N][NX*C], Y [E][NY], grad_out [N][NO*C] and the edge's   */
/* sender / receiver (edge_index int64 [E][2], column 0 = sender) and         */
/* multiplied on the matrix cores (near-fp32 split-fp16 products, as          */
/* mnx_edge_weights_bwd_f32).  frag: W [num_paths*C][K] packed by             */
/* mnx_edge_weights_pack_f32(..., backward = 1).  grad_h [E][K] overwritten.  */
/* C a multiple of 16, K in {16, 32, 64, 128}.  Together with                 */
/* mnx_tp_bwd_f32(..., grad_w = NULL) this replaces the TP backward's grad_w  */
/* and mnx_edge_weights_bwd_f32.                                              */
/* ------------------------------------------------------------------------ */
int mnx_tp_weight_grad_f32(int32_t config, int32_t channels, const float* x, const float* Y,
                           const float* grad_out, const int64_t* edge_index, int64_t num_nodes,
                           int64_t num_edges, const uint16_t* frag, int32_t K, float* grad_h,
                           mnx_stream_t stream);
/* The same grad_h for the edges of a receiver CSR (row_ptr, perm, senders as  */
/* from mnx_csr_build), in batches of up to 32 consecutive edges of one      */
/* receiver: batches [num_batches][2] = (receiver, first CSR slot), covering */
/* every slot once.  A wavefront per batch stages its receiver's output       */
/* gradient rows in LDS and forms gw from them and the senders' rows; the   */
/* contraction runs group (paths sharing l1) by group, 16-channel chunk by   */
/* chunk, path by path, so frag is W packed by mnx_edge_weights_pack_f32     */
/* (backward) after permuting W's rows into that order:                      */
/* mnx_tp_weight_grad_rows fills rows [num_paths * C] (host memory) with the */
/* original row of each permuted one.  grad_h [num_edges][K] by edge id.     */
int mnx_tp_weight_grad_rows(int32_t config, int32_t C, int32_t* rows);
int mnx_tp_weight_grad_batched_f32(int32_t config, int32_t C, const float* x, const float* Y,
                                   const float* grad_out, const int32_t* row_ptr, const int32_t* perm,
                                   const int32_t* senders, const int32_t* batches, int64_t num_batches,
                                   int64_t num_nodes, int64_t num_edges, const uint16_t* frag, int32_t K,
                                   float* grad_h, mnx_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Tensor-product backward fused with the output layer's input gradient      */
/* (replaces the TP backward's grad_w output plus mnx_edge_weights_bwd_f32;  */
/* the reference lets autograd write the per-edge weight gradient of        */
/* cuet.ChannelWiseTensorProduct, tensor_product.py:72-79,101-111, and read */
/* it back in the last Linear of RadialWeightMLP, radial_mlp.py:76-82):     */
/*   grad_x, grad_Y as mnx_tp_bwd_rows_f32 (grad_x accumulated: zero it),  */
/*   grad_h[e][k] = sum_n gw[e][n] W[n][k]   (grad_h [E][K] overwritten),   */
/* with gw formed by the receiver walk and multiplied on the matrix cores   */
/* from LDS, never written to memory.  W: the layer's weight                */
/* [num_paths*C][K] fp32 (nn.Linear layout).  ny: the config's harmonics    */
/* count (mnx_tp_config_info).  Supported when mnx_tp_bwd_gh_supported      */
/* (C a multiple of 64, K in {64, 128}, every path group's W slice fits     */
/* the LDS); the workspace holds the per-(group, channel block) partial     */
/* rows of grad_h (summed in a fixed order by a last kernel) and W's        */
/* pre-split fragments.  grad_Y may be NULL. */
int mnx_tp_bwd_gh_supported(int32_t config, int32_t channels, int32_t K);
size_t mnx_tp_bwd_gh_workspace_bytes(int32_t config, int32_t channels, int64_t num_edges, int32_t K,
                                     int32_t ny);
int mnx_tp_bwd_gh_rows_f32(int32_t config, int32_t channels, const float* x, const float* Y, const float* w,
                           const int32_t* wrow, const float* grad_out, const int32_t* row_ptr,
                           const int32_t* perm, const int32_t* senders_sorted, int64_t num_nodes,
                           int64_t num_edges, int32_t ny, const float* W, int32_t K, float* grad_x,
                           float* grad_Y, float* grad_h, void* workspace, size_t workspace_bytes,
                           mnx_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Channelwise tensor product + scatter for irreps outside the compiled      */
/* configurations, driven by a path table (replaces the same cuet call,      */
/* cuet.ChannelWiseTensorProduct(irreps_in1, irreps_sh, irreps_out,          */
/* layout=ir_mul, shared_weights=False, internal_weights=False) with         */
/* indices_1 / indices_out / size_out, src/molrep/interaction/               */
/* tensor_product.py:72-79,104-111, for any irreps with l <= 3: a            */
/* multiplicity per input block, any parities, several blocks of one l).     */
/*                                                                           */
/* table (host memory, int32): [P, NX, NY, NO, NW] followed by P records     */
/* [triple, xoff, yoff, ooff, woff, mul], with triple = mnx_tp_any_triple    */
/* (l1, l2, l3) and the offsets in floats within a row of x [N][NX],         */
/* Y [E][NY], out [N][NO] and w [E][NW]:                                     */
/*   out[r][ooff + m3*mul + c] += w[e][woff + c] * sum_{m1,m2}                */
/*       sqrt(2 l3 + 1) C[m1][m2][m3] x[s][xoff + m1*mul + c] Y[e][yoff + m2] */
/* summed over the edges e = (s -> r).  The output blocks must tile the      */
/* output row and the weight segments the weight row.  P <= 64, at most      */
/* 65535 chunks of 64 channels over all paths.                               */
/* ------------------------------------------------------------------------ */
#define MNX_TP_ANY_MAX_PATHS 64
/* Index of the coupling triple (l1, l2 -> l3), l <= 3, or -1. */
int mnx_tp_any_triple(int32_t l1, int32_t l2, int32_t l3);
/* out [N][NO] is overwritten. */
int mnx_tp_any_fwd_f32(const int32_t* table, int32_t table_len, const float* x, const float* Y,
                       const float* w, const int32_t* row_ptr, const int32_t* perm,
                       const int32_t* senders_sorted, int64_t num_nodes, int64_t num_edges,
                       float* out, mnx_stream_t stream);
/* Gradients of <grad_out, out>: grad_x [N][NX] and grad_Y [E][NY] accumulated
 * with atomics (zeroed by the caller), grad_w [E][NW] overwritten; any may be
 * NULL. */
int mnx_tp_any_bwd_f32(const int32_t* table, int32_t table_len, const float* x, const float* Y,
                       const float* w, const float* grad_out, const int32_t* row_ptr,
                       const int32_t* perm, const int32_t* senders_sorted, int64_t num_nodes,
                       int64_t num_edges, float* grad_x, float* grad_Y, float* grad_w,
                       mnx_stream_t stream);

/* ------------------------------------------------------------------------ */
/* C [M][N] = A^T B for tall operands A [K][M], B [K][N] (row strides lda,   */
/* ldb >= the widths; K rows >> M, N): the weight gradients of the per-edge  */
/* layers when training (dW = grad^T h over all edges of the radial MLP's    */
/* output layer, src/molrep/interaction/radial_mlp.py:76-82, which torch's   */
/* autograd computes as one GEMM over the edges), fp32-accurate on the bf16  */
/* matrix cores, deterministic.  Workspace from                              */
/* mnx_tall_tn_workspace_bytes (per-slab partial tiles); C is overwritten,   */
/* and colsum_a [M] (may be NULL) receives the column sums of A (the bias    */
/* gradient of the same layer) from the same pass.                           */
/* ------------------------------------------------------------------------ */
size_t mnx_tall_tn_workspace_bytes(int64_t K, int32_t M, int32_t N);
int mnx_tall_tn_f32(const float* A, int64_t lda, const float* B, int64_t ldb, int64_t K, int32_t M,
                    int32_t N, float* C, float* colsum_a, void* workspace, size_t workspace_bytes,
                    mnx_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Per-edge channelwise tensor product with shared weights, no scatter: the  */
/* layer product of Allegro (src/molzoo/allegro.py:352-359, applied at       */
/* :457-458 to the scaled edge features and the aggregated harmonics of each */
/* edge's source; there cuet.ChannelWiseTensorProduct with                   */
/* shared_weights=True, followed by cuet.Linear(tp.irreps_out, irreps_in)).  */
/*   out[e][o3 + m3][c] = w[p][c] sum cf_p[m1][m2][m3] x[e][o1+m1][c] Y[e][o2+m2] */
/* config from mnx_tp_config with input, harmonics and output l all          */
/* 0..l_max (only the paths whose output irrep is an input irrep are         */
/* computed, the ones the projection reads); channels 8, 16, 32, 64 or 128.  */
/* Layouts (ir_mul): x [E][NX * C], Y [E][NY], w [num_paths][C],             */
/* out [E][NO * C] (mnx_tp_config_info gives NX, NY, NO, num_paths).         */
/* x_scale [E][C] (or NULL) multiplies x channel by channel first (Allegro's */
/* env weights, allegro.py:447-450).  The backward overwrites grad_x         */
/* [E][NX * C], grad_Y [E][NY], grad_w [num_paths][C] and grad_x_scale       */
/* [E][C] (each may be NULL); grad_w is summed over edges in a fixed order   */
/* (bitwise reproducible) through a workspace of                             */
/* mnx_edge_tp_bwd_workspace_bytes bytes.                                    */
/* ------------------------------------------------------------------------ */
int mnx_edge_tp_fwd_f32(int32_t config, int32_t channels, const float* x, const float* Y,
                        const float* w, const float* x_scale, int64_t num_edges, float* out,
                        mnx_stream_t stream);
size_t mnx_edge_tp_bwd_workspace_bytes(int32_t config, int32_t channels, int64_t num_edges);
int mnx_edge_tp_bwd_f32(int32_t config, int32_t channels, const float* x, const float* Y,
                        const float* w, const float* x_scale, const float* grad_out,
                        int64_t num_edges, float* grad_x, float* grad_Y, float* grad_w,
                        float* grad_x_scale, void* workspace, size_t workspace_bytes,
                        mnx_stream_t stream);

/* ------------------------------------------------------------------------ */
/* The same product fused with the projection after it (allegro.py:363-367,  */
/* cuet.Linear(tp.irreps_out, irreps_in), applied at :465-466), 16 channels: */
/*   out[e][I_l + m][c'] = sum_{b, c} proj[(J_l + b) * 16 + c][c']           */
/*                          * TP_b(x_scale x, Y; w)[e][m][c]                 */
/* for every projected irrep l = 0..l_max (I_l its first component, ir_mul), */
/* b over the paths with output irrep l (J_l the first of them in the        */
/* projection's row blocks).  mnx_edge_tp_proj_info writes, per projected    */
/* irrep in row order, (l, paths, J_l, I_l) into blocks (4 ints each, at     */
/* most 4 irreps) and returns their count (0: no fused kernel for config,   */
/* -1: config out of range); out is [E][NI * 16] with NI =                   */
/* sum (2l + 1).  proj is [num_paths * 16][16] (row J*16 + c: input channel  */
/* c of path block J; the reference's weights of that irrep times its        */
/* 1/sqrt(fan_in)).  No projection gradient; the backward's other outputs   */
/* and fixed order of summation are those of mnx_edge_tp_bwd_f32 with        */
/* channels = 16, through a workspace of                                     */
/* mnx_edge_tp_proj_bwd_workspace_bytes bytes (0: no fused kernel).          */
/* x_shared != 0: x is [E][NX], one value per component shared by all 16    */
/* channels (x[e][i][c] = x[e][i], e.g. harmonics whose channel weights come */
/* in through x_scale), and grad_x [E][NX] is the sum over the channels.     */
/* x_scale2 [E][16] (or NULL) multiplies x_scale (the scale is their         */
/* product); grad_x_scale2 is its gradient (either gradient may be NULL).    */
/* ------------------------------------------------------------------------ */
int32_t mnx_edge_tp_proj_info(int32_t config, int32_t* blocks);
size_t mnx_edge_tp_proj_bwd_workspace_bytes(int32_t config, int64_t num_edges);
int mnx_edge_tp_proj_fwd_f32(int32_t config, const float* x, int32_t x_shared, const float* Y,
                             const float* w, const float* x_scale, const float* x_scale2,
                             const float* proj, int64_t num_edges, float* out, mnx_stream_t stream);
int mnx_edge_tp_proj_bwd_f32(int32_t config, const float* x, int32_t x_shared, const float* Y,
                             const float* w, const float* x_scale, const float* x_scale2,
                             const float* proj, const float* grad_out, int64_t num_edges,
                             float* grad_x, float* grad_Y, float* grad_w, float* grad_x_scale,
                             float* grad_x_scale2, void* workspace, size_t workspace_bytes,
                             mnx_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Per-channel scaling of an ir_mul edge tensor (Allegro's output env        */
/* scaling, src/molzoo/allegro.py:95-128 _scale_by_channel):                 */
/*   out[e][d][c] = t[e][d][c] * s[e][c]  (t, out [E][D][F], s [E][F]),       */
/* and its backward in one pass: grad_t = grad * s (broadcast over d),       */
/* grad_s[e][c] = sum_d grad[e][d][c] t[e][d][c] (d ascending).  D in        */
/* {1, 4, 9, 16}, F a multiple of 4, every pointer 16-byte aligned; NULL     */
/* grad_t / grad_s are skipped.                                               */
/* ------------------------------------------------------------------------ */
int mnx_channel_scale_f32(const float* t, const float* s, int64_t E, int32_t D, int32_t F, float* out,
                          mnx_stream_t stream);
int mnx_channel_scale_bwd_f32(const float* grad, const float* t, const float* s, int64_t E, int32_t D, int32_t F,
                              float* grad_t, float* grad_s, mnx_stream_t stream);
/* Per-edge outer product of components and channels (the env-weighted      */
/* harmonics of Allegro's pair embedding, src/molzoo/allegro.py:55-92):      */
/*   out[e][d][c] = y[e][d] * s[e][c]  (y [E][D], s [E][F], out [E][D][F]);  */
/* backward grad_y[e][d] = sum_c grad[e][d][c] s[e][c], grad_s[e][c] =        */
/* sum_d grad[e][d][c] y[e][d], one pass.  D in {1, 4, 9, 16}; F a multiple  */
/* of 4 with F / 4 a power of two <= 64 for the backward; s, out, grad and   */
/* grad_s 16-byte aligned.                                                    */
int mnx_channel_outer_f32(const float* y, const float* s, int64_t E, int32_t D, int32_t F, float* out,
                          mnx_stream_t stream);
int mnx_channel_outer_bwd_f32(const float* grad, const float* y, const float* s, int64_t E, int32_t D, int32_t F,
                              float* grad_y, float* grad_s, mnx_stream_t stream);
/* The same product with one component over a stack of L inputs (the cutoff */
/* envelope on Allegro's per-layer scalar features and their stack,         */
/* src/molzoo/allegro.py:628-641): s is a host array of L device pointers   */
/* to [E][F] inputs; out[e][l][c] = y[e] * s_l[e][c] (out [E][L][F]);        */
/* backward grad_s_l[e][c] = grad[e][l][c] y[e] (grad_s a host array of L   */
/* device pointers, or NULL), grad_y[e] = sum_l sum_c grad[e][l][c]          */
/* s_l[e][c] (NULL: not formed), one pass.  1 <= L <= 8; F a multiple of 4   */
/* with F / 4 a power of two <= 64; every [E][F] and [E][L][F] array 16-byte */
/* aligned.                                                                   */
int mnx_channel_outer_stack_f32(const float* y, const float* const* s, int32_t L, int64_t E, int32_t F, float* out,
                                mnx_stream_t stream);
int mnx_channel_outer_stack_bwd_f32(const float* grad, const float* y, const float* const* s, int32_t L, int64_t E,
                                    int32_t F, float* grad_y, float* const* grad_s, mnx_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MOLNEX_H */
