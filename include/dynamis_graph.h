/*
 * dynamis_graph.h -- C ABI of the gfx950 (MI355X) neighbour-graph library
 * (libdynamis_graph.so, built from dynamis_amd/csrc/).
 *
 * Plain pointers and sizes only.  Device pointers are HIP device addresses; every call
 * is asynchronous on the given stream unless stated otherwise.  Calls never allocate
 * device memory: the caller passes a workspace of dg_graph_workspace_size() bytes.
 * Status codes are returned instead of exceptions; dg_last_error() holds the message of
 * the last failure on the calling thread.
 *
 * Contract of the edge set (shared by every entry point):
 *   (src, dst, S) is an edge iff S is integer, S_d = floor(f_dst,d) - floor(f_src,d) on
 *   non-periodic axes, and 1e-8f < d2 <= radius^2 with the fp64 canonical
 *       v  = (p_src - p_dst) + S . cell,   d2 = |v|^2
 *   (fixed operation order, see dynamis_amd/csrc/dg_common.hpp).  f = p . cell^-1.
 *   This is the set the reference's cell list enumerates
 *   (dynamis_state/src/csrc/graph/radius_graph_kernels.cu:18-442), with the predicate
 *   evaluated in fp64 instead of fp32.
 *
 * References are file:line in Dynamis-MD/Dynamis.
 */
#ifndef DYNAMIS_GRAPH_H
#define DYNAMIS_GRAPH_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    DG_OK = 0,
    DG_ERR_INVALID = 1,   /* bad argument (shape, radius, singular cell, ...) */
    DG_ERR_WORKSPACE = 2, /* workspace too small */
    DG_ERR_HIP = 3,       /* HIP runtime error (launch, copy) */
    DG_ERR_RANGE = 4,     /* data-dependent: atom > 255 cells outside the cell, NaN
                             position or target index out of range (reported by
                             dg_graph_read_totals) */
    DG_ERR_CAPACITY = 5   /* edge capacity smaller than the edge count */
} dg_status;

typedef enum { DG_F32 = 0, DG_F64 = 1, DG_I64 = 2, DG_I32 = 3 } dg_dtype;

/* Status flag bits of dg_graph_read_totals(). */
#define DG_FLAG_RANGE 1
#define DG_FLAG_NONFINITE 2
#define DG_FLAG_CAPACITY 4
#define DG_FLAG_TARGET 8

/* Description of one radius-graph build.
 * Mirrors the arguments of radius_graph_pbc_ex (dynamis_state/src/csrc/graph/
 * radius_graph.cpp:51-92): pos [n_atoms,3], cell [3,3] with lattice vectors as rows,
 * pbc [3], radius, target_indices [n_targets] (NULL -> all atoms are targets). */
typedef struct dg_graph_desc {
    int64_t n_atoms;
    int64_t n_targets; /* ignored when has_targets == 0 */
    int32_t has_targets;
    int32_t pos_dtype; /* dg_dtype */
    double cell[9];
    uint8_t pbc[3];
    uint8_t pad_[5];
    double radius;
} dg_graph_desc;

/* Bytes of device workspace needed by dg_graph_count / dg_graph_write for this
 * description; 0 on invalid input (see dg_last_error).  Host only. */
size_t dg_graph_workspace_size(const dg_graph_desc* desc);

/* Stage 1 of a build: SFC reorder of the atoms into the cell list (Morton tile order),
 * per-target degree count and the edge-offset scan.
 * Replaces radius_graph_pbc_counts_ex (radius_graph.cpp:94-127) and the count half of
 * radius_graph_pbc_cuda_impl_ex (radius_graph_kernels.cu:480-846).
 *   pos          device, [n_atoms,3] of pos_dtype, row-major
 *   target_idx   device int64 [n_targets] or NULL
 *   counts_out   device int32 [n_targets] (caller order) or NULL
 * The total edge count and status flags stay in the workspace; read them with
 * dg_graph_read_totals (one device->host copy and stream sync). */
dg_status dg_graph_count(const dg_graph_desc* desc, const void* pos, const int64_t* target_idx,
                         void* workspace, size_t workspace_bytes, int32_t* counts_out,
                         hipStream_t stream);

/* Counts only: dg_graph_count without recording the neighbour lists the write stage would
 * expand (the sweep skips them).  Replaces radius_graph_pbc_counts_ex (radius_graph.cpp:94-127,
 * the counts-only path of radius_graph_kernels.cu:798-808).  Same outputs; a dg_graph_write
 * that follows on the same workspace is still correct, but writes every tile from its
 * slower fix-up pass. */
dg_status dg_graph_counts(const dg_graph_desc* desc, const void* pos, const int64_t* target_idx,
                          void* workspace, size_t workspace_bytes, int32_t* counts_out,
                          hipStream_t stream);

/* Synchronous: copies {total_edges, flags} out of the workspace (waits for the stream).
 * Returns DG_ERR_RANGE if a data-dependent error flag is set. */
dg_status dg_graph_read_totals(const dg_graph_desc* desc, const void* workspace,
                               int64_t* total_edges, int64_t* flags, hipStream_t stream);

/* Stage 2 of a build (after dg_graph_count on the same workspace, inputs unchanged):
 * writes every edge.  Replaces the B4 write of radius_graph_kernels.cu:848-933.
 *   edge_src, edge_dst   device int64 [capacity]  (edge_index[0], edge_index[1])
 *   cell_shift           device float32 [capacity,3]  (integer-valued; "cell_offsets")
 *   edge_vec             device [capacity,3] of vec_dtype or NULL (canonical v)
 *   edge_dist            device [capacity] of vec_dtype or NULL (sqrt(d2))
 * Edges are grouped by target in the SFC processing order; within a target the order
 * is fixed (deterministic) but unspecified.  Tiles that would overrun `capacity` are
 * skipped and DG_FLAG_CAPACITY is raised.  Outputs aligned to 16 bytes are written in
 * 16-byte groups (the fast path; torch allocations are); other alignments give the same
 * bytes, more slowly.  With edge_vec or edge_dist, the stage reuses the count stage's
 * sort scratch in the workspace (a later dg_graph_write on the same workspace is still
 * valid; the count's results it needs are kept). */
dg_status dg_graph_write(const dg_graph_desc* desc, const void* pos, const int64_t* target_idx,
                         void* workspace, size_t workspace_bytes, int64_t capacity,
                         int64_t* edge_src, int64_t* edge_dst, float* cell_shift, void* edge_vec,
                         void* edge_dist, int32_t vec_dtype, hipStream_t stream);

/* dg_graph_write with the ids written for the atoms mapped: edge_src / edge_dst receive
 * out_ids[i] for atom i (device int64 [n_atoms], values in [0, 2^31); NULL: i itself), while
 * positions are still read as pos[i].  No counterpart in the reference: it fuses the remap
 * that DistGraphBuilder's steady step applies to a local build's edges
 * (dist_graph_builder.py:469-474, the index_select of the local edges) into the write stage. */
dg_status dg_graph_write_ids(const dg_graph_desc* desc, const void* pos, const int64_t* target_idx,
                             void* workspace, size_t workspace_bytes, int64_t capacity,
                             const int64_t* out_ids, int64_t* edge_src, int64_t* edge_dst,
                             float* cell_shift, void* edge_vec, void* edge_dist, int32_t vec_dtype,
                             hipStream_t stream);

/* One-call build into caller-preallocated outputs of `capacity` edges:
 * dg_graph_count then dg_graph_write, back to back on the stream with no host round trip
 * (the write pass reads the count pass's per-tile offsets on the device).  Same outputs,
 * in the same order.  Read the edge count afterwards with dg_graph_read_totals: if it
 * exceeds `capacity` (DG_ERR_CAPACITY), the tiles that did not fit were skipped -- rebuild
 * into larger buffers.  This is the caller-owned-buffer form of
 * radius_graph_pbc_cuda_impl_ex (radius_graph_kernels.cu:480-934), for callers that keep
 * edge buffers across rebuilds (the molecular-dynamics loop). */
dg_status dg_graph_build(const dg_graph_desc* desc, const void* pos, const int64_t* target_idx,
                         void* workspace, size_t workspace_bytes, int64_t capacity,
                         int32_t* counts_out, int64_t* edge_src, int64_t* edge_dst,
                         float* cell_shift, void* edge_vec, void* edge_dist, int32_t vec_dtype,
                         hipStream_t stream);

/* Allocation-free one-call build.  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The same build as dg_graph_build (same kernels, same
 * outputs in the same order), with the workspace taken from a static device array inside
 * the library (64 MiB per GPU, held until the process ends) instead of a caller buffer;
 * it calls no hipMalloc / hipFree.  Builds whose dg_graph_workspace_size() exceeds
 * 64 MiB (about 140k atoms at 0.1 atoms/A^3 and r = 6 A) are refused with
 * DG_ERR_WORKSPACE.  The edge count and status flags are copied on the stream to
 *   totals_out   device int64 [2]: {total_edges, flags (DG_FLAG_*)}
 * which the caller reads when it needs them (an edge count above `capacity`, or
 * DG_FLAG_CAPACITY, means the tiles that did not fit were skipped).  Every call on one
 * GPU shares that GPU's array: calls that overlap on one GPU race.  Calls on one stream
 * are ordered by it; a call on another stream while the previous call's work is still
 * pending on the GPU, or while another host thread is enqueueing a call on the same GPU,
 * is refused with DG_ERR_INVALID (a host-side check of an event the library records
 * behind every call; calls on a stream under graph capture are not checked, and ordering
 * such calls is the caller's part).  The stream must belong to the
 * current device (DG_ERR_INVALID otherwise). */
dg_status dg_graph_build_noalloc(const dg_graph_desc* desc, const void* pos,
                                 const int64_t* target_idx, int64_t capacity, int32_t* counts_out,
                                 int64_t* edge_src, int64_t* edge_dst, float* cell_shift,
                                 void* edge_vec, void* edge_dist, int32_t vec_dtype,
                                 int64_t* totals_out, hipStream_t stream);

/* Order-preserving filter of an edge list to radius (keep iff d2 <= radius^2, canonical
 * fp64 d2).  Replaces filter_edges_to_radius (dist_graph_ops.cpp:5-35,
 * dist_graph_ops_kernels.cu:16-43,62-102).
 *   edge_src/edge_dst int64 [n_edges], cell_shift [n_edges,3] of shift_dtype (DG_F32,
 *     DG_F64, DG_I64 or DG_I32)
 *   keep_idx out int64 [n_edges]: indices of kept edges, ascending
 *   n_kept   out int64 (device, one value); -1 if an edge names an atom outside
 *            [0, n_atoms) (such edges are never read through: no position is gathered)
 *   workspace of dg_filter_workspace_size(n_edges) bytes */
size_t dg_filter_workspace_size(int64_t n_edges);
dg_status dg_filter_edges_to_radius(const void* pos, int32_t pos_dtype, int64_t n_atoms,
                                    const double* cell, double radius, const int64_t* edge_src,
                                    const int64_t* edge_dst, const void* cell_shift,
                                    int32_t shift_dtype, int64_t n_edges, int64_t* keep_idx,
                                    int64_t* n_kept, void* workspace, size_t workspace_bytes,
                                    hipStream_t stream);

/* The same filter as a count / write pair that writes the kept edges themselves (in order,
 * shifts in shift_dtype), for exact-size outputs without an index gather: the form the
 * Python filter_edges_to_radius uses.  Replaces the same reference function as above.
 *   dg_filter_count: n_kept out int64 (device, one value; -1 if an edge names an atom
 *     outside [0, n_atoms)); workspace of
 *     dg_filter2_workspace_size(n_edges) bytes, kept for dg_filter_write
 *   dg_filter_write: out_src/out_dst int64 [n_kept], out_shift [n_kept,3] of shift_dtype;
 *     same inputs and workspace as the dg_filter_count call before it */
size_t dg_filter2_workspace_size(int64_t n_edges);
dg_status dg_filter_count(const void* pos, int32_t pos_dtype, int64_t n_atoms, const double* cell,
                          double radius, const int64_t* edge_src, const int64_t* edge_dst,
                          const void* cell_shift, int32_t shift_dtype, int64_t n_edges,
                          int64_t* n_kept, void* workspace, size_t workspace_bytes,
                          hipStream_t stream);
dg_status dg_filter_write(const void* pos, int32_t pos_dtype, int64_t n_atoms, const double* cell,
                          double radius, const int64_t* edge_src, const int64_t* edge_dst,
                          const void* cell_shift, int32_t shift_dtype, int64_t n_edges,
                          const void* workspace, size_t workspace_bytes, int64_t* out_src,
                          int64_t* out_dst, void* out_shift, hipStream_t stream);

/* The same filter in one pass over the edge list (a decoupled look-back gives each block
 * of 4096 edges the kept count before it): kept edges go, in order, to the first n_kept
 * rows of outputs of capacity n_edges.  Replaces the same reference function; the form
 * the Python filter_edges_to_radius uses.
 *   out_src/out_dst int64 [n_edges], out_shift [n_edges,3] of shift_dtype (capacity)
 *   n_kept  out int64 (device, one value): -1 if an edge names an atom outside
 *           [0, n_atoms), -2 if a block's wait for its predecessors gave up (a bounded wait;
 *           not expected), else the number of kept edges
 *   workspace of dg_filter_compact_workspace_size(n_edges) bytes */
size_t dg_filter_compact_workspace_size(int64_t n_edges);
dg_status dg_filter_compact(const void* pos, int32_t pos_dtype, int64_t n_atoms, const double* cell,
                            double radius, const int64_t* edge_src, const int64_t* edge_dst,
                            const void* cell_shift, int32_t shift_dtype, int64_t n_edges,
                            int64_t* out_src, int64_t* out_dst, void* out_shift, int64_t* n_kept,
                            void* workspace, size_t workspace_bytes, hipStream_t stream);

/* SFC keys exactly as partition/sfc_kernels.cu:19-109 (curve 0 = Morton 21-bit,
 * 1 = "Hilbert" order 7), normalised by the global min / range of pos
 * (sfc_kernels.cu:196-198, range 0 -> 1).  pos fp32 [n,3]; keys int64 [n];
 * workspace of dg_sfc_workspace_size(n) bytes.  Replaces the key stage of
 * sfc_partition_cuda_impl (sfc_kernels.cu:178-213). */
size_t dg_sfc_workspace_size(int64_t n);
dg_status dg_sfc_keys(const float* pos, int64_t n, int32_t curve, int64_t* keys, void* workspace,
                      size_t workspace_bytes, hipStream_t stream);

/* Stable ascending sort permutation of int64 keys (ties keep index order).
 * Replaces at::sort(sfc_keys) in sfc_kernels.cu:224.  perm int64 [n].  No host
 * synchronisation: a fixed sequence of launches on the stream (a HIP graph can capture
 * it); key bytes in which all keys agree are skipped on the device. */
dg_status dg_sfc_order(const int64_t* keys, int64_t n, int64_t* perm, void* workspace,
                       size_t workspace_bytes, hipStream_t stream);


/* Partition labels from a permutation: unweighted closed form (sfc_kernels.cu:114-136)
 * or exact int64 weighted cut (sfc_kernels.cu:153-173, weights int64 [n] or NULL).
 * labels int64 [n]. */
dg_status dg_sfc_labels(const int64_t* perm, int64_t n, int64_t n_parts, const int64_t* weights,
                        int64_t* labels, void* workspace, size_t workspace_bytes,
                        hipStream_t stream);

/* Halo send/recv plan of one rank from its edges (every edge's dst in this rank's atom
 * set).  Replaces extract_halo_info (dist_graph_ops.cpp:38-60,
 * dist_graph_ops_kernels.cu:104-188; binding dynamis_state_bindings.cpp:256).
 *   recv: atoms a = src of an edge with pid[a] != my_rank, once each, grouped by peer
 *         pid[a] ascending, by global id within a peer;
 *   send: pairs (p, d) with d = dst of an edge whose src is owned by p != my_rank, grouped
 *         by p, by global id d within a peer; reported as the position of d in my_outer
 *         (-1 if d is not in my_outer);
 *   interior_mask[j] = my_outer[j] is the dst of no such edge.
 * Two stages on one workspace of dg_halo_workspace_size(n_atoms, world_size) bytes:
 * dg_halo_count (offsets + interior mask), dg_halo_read_totals (synchronous), then
 * dg_halo_write (the index lists, into buffers of the read sizes). */
/* ------------------------------------------------------------------ batches of structures
 * radius_graph_pbc_cuda with a batch (radius_graph_pbc_cuda.py:64-110) builds structure by
 * structure.  These entry points build the graphs of a whole batch of small structures
 * (all sharing the PBC flags and radius, each with its own cell) in one launch sequence:
 * all-pairs over each structure's atoms and periodic images, the canonical fp64 predicate
 * and shift convention of dg_graph_*.  Edges come grouped by target: structures in batch
 * order, targets in index order (within a target the order is fixed but unspecified).
 * The atom indices are those of the batch (structure b's atoms follow structures 0..b-1). */
typedef struct dg_batch_desc {
    int64_t n_images;   /* structures in the batch (>= 1) */
    int64_t n_atoms;    /* atoms of the whole batch */
    int32_t pos_dtype;  /* DG_F32 / DG_F64 */
    uint8_t pbc[3];     /* shared by every structure */
    double radius;      /* cutoff (rounded to fp32 by the caller, as dg_graph_desc) */
} dg_batch_desc;

size_t dg_batch_workspace_size(const dg_batch_desc* desc);

/* Stage 1: per-atom degrees and the batch's edge count.
 *   pos      device [n_atoms,3] of pos_dtype, the structures one after another
 *   natoms   device int64 [n_images], atoms per structure (summing to n_atoms)
 *   cells    device float64 [n_images,3,3], row-major lattice vectors (rounded to
 *            pos_dtype by the caller, as dg_graph_desc.cell)
 *   counts_out  device int32 [n_atoms] or NULL
 * Asynchronous; then dg_batch_read_totals. */
dg_status dg_batch_count(const dg_batch_desc* desc, const void* pos, const int64_t* natoms,
                         const double* cells, int32_t* counts_out, void* workspace,
                         size_t workspace_bytes, hipStream_t stream);

/* Synchronous: the batch's edge count and status flags.  DG_ERR_INVALID for a singular
 * cell or atom counts that do not add up, DG_ERR_RANGE for non-finite positions. */
dg_status dg_batch_read_totals(const dg_batch_desc* desc, const void* workspace,
                               int64_t* total_edges, int64_t* flags, hipStream_t stream);

/* Stage 2: every edge, into outputs of `capacity` rows, and the edge count of every
 * structure (edges_per_image: device int64 [n_images] or NULL; "num_neighbors_image"). */
dg_status dg_batch_write(const dg_batch_desc* desc, const void* pos, void* workspace,
                         size_t workspace_bytes, int64_t capacity, int64_t* edge_src,
                         int64_t* edge_dst, float* cell_shift, int64_t* edges_per_image,
                         hipStream_t stream);

typedef struct dg_halo_desc {
    int64_t n_atoms;    /* N: length of pid, range of atom ids */
    int64_t n_edges;    /* E */
    int64_t num_local;  /* length of my_outer */
    int64_t my_rank;
    int64_t world_size; /* 1 .. 4096 */
    int32_t pid_dtype;  /* DG_I32 or DG_I64 */
    int32_t pad_;
} dg_halo_desc;

size_t dg_halo_workspace_size(int64_t n_atoms, int64_t world_size);
/*   edge_src/edge_dst int64 [n_edges]; pid [n_atoms]; my_outer int64 [num_local]
 *   send_offsets, recv_offsets  out int64 [world_size+1]
 *   interior_mask               out uint8 (0/1) [num_local] */
dg_status dg_halo_count(const dg_halo_desc* desc, const int64_t* edge_src, const int64_t* edge_dst,
                        const void* pid, const int64_t* my_outer, int64_t* send_offsets,
                        int64_t* recv_offsets, uint8_t* interior_mask, void* workspace,
                        size_t workspace_bytes, hipStream_t stream);
/* Synchronous.  DG_ERR_RANGE if an edge endpoint, pid value or my_outer entry was out of
 * range. */
dg_status dg_halo_read_totals(const void* workspace, int64_t* total_send, int64_t* total_recv,
                              hipStream_t stream);
/*   send_local_indices out int64 [total_send]
 *   recv_ghost_indices out int64 [total_recv]  (num_local + k)
 *   recv_atom_global   out int64 [total_recv] */
dg_status dg_halo_write(const dg_halo_desc* desc, const void* pid, int64_t* send_local_indices,
                        int64_t* recv_ghost_indices, int64_t* recv_atom_global, void* workspace,
                        size_t workspace_bytes, hipStream_t stream);

/* Message of the last failure on this thread ("" if none). */
const char* dg_last_error(void);

/* Library version string. */
const char* dg_version(void);

#ifdef __cplusplus
}
#endif
#endif /* DYNAMIS_GRAPH_H */
