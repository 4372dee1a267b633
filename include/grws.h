/*
 * grws.h -- C ABI of the MI355X-native Graph_RWS hot path (libgrws.so).
 *
 * This is the drop-in boundary that replaces the reference's pybind11 module
 * `core_lib` (core/wrapper/bind.cpp:78-161, re-exported by core/__init__.py).
 * Plain C types only: device pointers, sizes, dtype codes and a hipStream_t
 * passed as `void*`.  No torch types cross this boundary.
 *
 * Conventions (every entry point):
 *   - returns GRWS_OK (0) or a negative GRWS_E_* code; the message of the
 *     last failure on the calling thread is returned by grws_last_error();
 *   - never allocates device memory: outputs and workspaces are provided by
 *     the caller, sized by the matching *_bytes / *_capacity query;
 *   - all device work is ordered on `stream`; entry points that must return
 *     a data-dependent size to the host say so and synchronise that stream.
 *     The BCSR build runs its windows of over 16,384 edges on a second
 *     stream of the device (one per device, made on first use), forked from
 *     `stream` and joined back into it by events before the call returns;
 *   - calls on different streams and threads are independent (re-entrant):
 *     the only global state is that per-device stream and the no-alloc
 *     entry point's device array.
 *
 * Tile geometry: tile_rows is 16 (one row window); tile_cols is 8 (the
 * reference default, config.h:16-18) or 16 (MFMA-native).
 */
#ifndef GRWS_H
#define GRWS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GRWS_ABI_VERSION 1

/* element types */
enum {
    GRWS_F32 = 0,
    GRWS_F16 = 1,
    GRWS_BF16 = 2
};

/* status codes */
enum {
    GRWS_OK = 0,
    GRWS_E_INVALID = -1,  /* bad argument: null pointer, negative size, bad tile shape */
    GRWS_E_DTYPE = -2,    /* unsupported element type or combination */
    GRWS_E_CAPACITY = -3, /* caller buffer or workspace too small */
    GRWS_E_HIP = -4,      /* HIP runtime / launch failure */
    GRWS_E_RANGE = -5     /* index data out of range */
};

/* Message of the last failure on the calling thread ("" if none). */
const char* grws_last_error(void);

/* GRWS_ABI_VERSION of the loaded library. */
int grws_abi_version(void);

/*
 * A BCSR graph as stored by BCSRGraph (data/bcsr.py:23-62):
 *   window_offset [num_windows+1] int64 prefix sum of tiles per window,
 *   col_indices   [num_tiles*tile_cols] int32 global column per tile slot,
 *                 ascending and unique per window, -1 padding,
 *   values        [num_tiles*tile_rows*tile_cols], row-major per tile.
 */
typedef struct grws_bcsr {
    const int64_t* window_offset;
    const int32_t* col_indices;
    const void* values;
    int64_t num_windows;
    int64_t num_tiles;
    int32_t tile_rows;    /* must be 16 */
    int32_t tile_cols;    /* 8 or 16 */
    int32_t values_dtype; /* GRWS_F32 / GRWS_F16 / GRWS_BF16 */
    int32_t max_window_slabs; /* 0 = unknown; else an upper bound of every window's
                                 slabs (16 column slots), used by a plan-less grws_spmm to
                                 size its 32-bit offsets.  A wrong bound gives wrong sums. */
} grws_bcsr;

/*
 * SpMM work schedule (built once per graph by grws_spmm_plan_build).
 * A "slab" is 16 consecutive column slots of a window (one tile at
 * tile_cols=16, two at tile_cols=8).  Windows with more than slabs_per_item
 * slabs are split over several items whose partial sums are combined in a
 * fixed order (deterministic, no atomics).
 */
typedef struct grws_spmm_plan {
    const int32_t* items; /* [num_items][4] = window, slab_begin, slab_end, partial slot or -1 */
    const int32_t* split; /* [num_split][3] = window, first slot, number of slots */
    int64_t num_items;
    int64_t num_split;
    int64_t num_slots;
    int32_t slabs_per_item;
    int32_t reserved;
} grws_spmm_plan;

/* ------------------------------------------------------------------------ */
/* SpMM forward  Y[16W x N] = A * X                                          */
/* Replaces core_lib.spmm_tc (bind.cpp:124-130 -> spmm_wrapper.cu:33-95,     */
/* kernel spmm_tc.cuh:40-195).  Unlike the reference it computes every one   */
/* of the N output columns and writes every row (no memset needed).          */
/* ------------------------------------------------------------------------ */

/* Upper bounds of the plan arrays for a graph (host arithmetic only). */
int grws_spmm_plan_capacity(int64_t num_windows, int64_t num_tiles, int32_t tile_cols,
                            int32_t slabs_per_item, int64_t* max_items, int64_t* max_split);

/* Default slabs_per_item for a graph and output width (host heuristic). */
int32_t grws_spmm_default_slabs(int64_t num_windows, int64_t num_tiles, int32_t tile_cols,
                                int64_t n_cols);

/* Workspace bytes needed by grws_spmm_plan_build. */
size_t grws_spmm_plan_workspace_bytes(int64_t num_windows);

/* Builds the plan on the device.  items: int32 [max_items*4], split: int32
 * [max_split*3] (device).  Synchronises `stream` and writes the host array
 * counts_out[3] = {num_items, num_split, num_slots}. */
int grws_spmm_plan_build(const int64_t* window_offset, int64_t num_windows, int64_t num_tiles,
                         int32_t tile_cols, int32_t slabs_per_item, int32_t* items,
                         int64_t max_items, int32_t* split, int64_t max_split, void* workspace,
                         size_t workspace_bytes, int64_t* counts_out, void* stream);

/* Reorders a built plan's items (int32 [num_items][4], device) for a
 * shorter launch: the kernels walk the item list in eighths, one per XCD,
 * and within each eighth the items go longest first (stable), so that long
 * items (a power-law graph's hub windows) do not start last.  No
 * counterpart in the reference (its kernel launches one block per window,
 * spmm_wrapper.cu:33-95).  Results are identical in either order; the
 * window order lets neighbouring windows share X rows in the L2, so this
 * pays on graphs without such locality (bindings apply it when the plan
 * splits windows).  Workspace from grws_spmm_plan_order_workspace_bytes;
 * stream-ordered, no sync. */
size_t grws_spmm_plan_order_workspace_bytes(int64_t num_items);
int grws_spmm_plan_order(int32_t* items, int64_t num_items, void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes grws_spmm needs (0 when the plan has no split windows or
 * plan is NULL). */
size_t grws_spmm_workspace_bytes(const grws_spmm_plan* plan, int64_t n_cols);

/*
 * Y = A X.  x: [x_rows, ldx] row-major, first n_cols columns used; y:
 * [16*num_windows, ldy].  x_dtype == y_dtype; A's values may be F32 or
 * x_dtype.  F16/BF16 use MFMA with fp32 accumulation; F32 uses fp32 MFMA.
 * Column slots of -1, or outside [0, x_rows), contribute nothing.
 * plan may be NULL (one work item per window, no splitting).  workspace
 * (grws_spmm_workspace_bytes) must be 16-byte aligned.
 */
int grws_spmm(const grws_bcsr* A, const grws_spmm_plan* plan, const void* x, int32_t x_dtype,
              int64_t x_rows, int64_t ldx, int64_t n_cols, void* y, int32_t y_dtype, int64_t ldy,
              void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Packed tiles: a compact copy of A's values for graphs that are multiplied */
/* many times (full-graph training).  No counterpart in the reference, which */
/* streams the dense 16x16 tiles (spmm_tc.cuh:113-193) on every call; the    */
/* dense arrays stay the graph of record and grws_spmm_packed gives          */
/* bit-identical results to grws_spmm.                                       */
/*                                                                           */
/* Layout (16x16 tiles of F16/BF16 values only): header[num_tiles][4][3]     */
/* uint32 -- for row group q (rows 4q..4q+3) {mask_lo, mask_hi, start}, mask */
/* bit (r%4)*16 + c set iff slot (r, c) holds a value whose bit pattern is   */
/* not zero, start = index of the group's first such value in values[];     */
/* values[num_values] = those values in tile, then slot, order.  At most     */
/* 2^30 - 16 values.                                                         */
/* ------------------------------------------------------------------------ */
typedef struct grws_packed_tiles {
    const uint32_t* header;
    const void* values;
    int64_t num_values;
} grws_packed_tiles;

/* Workspace bytes for both packing calls. */
size_t grws_pack_tiles_workspace_bytes(int64_t num_tiles);

/* Pass 1: counts the nonzero values per tile into the workspace and writes
 * the host *num_values (synchronises `stream`).  GRWS_E_CAPACITY past the
 * 2^30 - 16 limit. */
int grws_pack_tiles_count(const grws_bcsr* A, void* workspace, size_t workspace_bytes,
                          int64_t* num_values, void* stream);

/* Pass 2: writes header [num_tiles*12] uint32 and values (A's dtype),
 * reading the counts pass 1 left in the same, unchanged, workspace.  The
 * values buffer holds num_values + 8 elements: grws_spmm_packed may read
 * the 8 after the last value (their contents do not matter). */
int grws_pack_tiles_fill(const grws_bcsr* A, uint32_t* header, void* values, int64_t num_values,
                         void* workspace, size_t workspace_bytes, void* stream);

/* grws_spmm with A's values read from packed tiles P (P NULL: grws_spmm).
 * Needs 16x16 tiles whose values have the x dtype (F16/BF16).  The same
 * result, bit for bit, as grws_spmm on the dense arrays (which are still
 * read when the call runs on the element-masked kernel, e.g. X rows not
 * 16-byte aligned). */
int grws_spmm_packed(const grws_bcsr* A, const grws_packed_tiles* P, const grws_spmm_plan* plan,
                     const void* x, int32_t x_dtype, int64_t x_rows, int64_t ldx, int64_t n_cols,
                     void* y, int32_t y_dtype, int64_t ldy, void* workspace, size_t workspace_bytes,
                     void* stream);

/* ------------------------------------------------------------------------ */
/* Grouped tiles: A's tiles re-cut so that group_size consecutive windows    */
/* share one sorted list of the union of their columns (16 per slab), each   */
/* window keeping one 16x16 sub-tile per slab, packed as above.  The SpMM    */
/* (spmm_tc.cuh:113-193 computes Y = A X window by window, gathering each    */
/* window's columns) then gathers every union column's X row once per group  */
/* instead of once per window: on graphs with community structure the       */
/* windows of a group share most columns (c3, 4 windows: 74.5M column slots  */
/* become 40.0M).  No counterpart in the reference; the dense arrays stay    */
/* the graph of record.  Sums run over each row's columns in ascending order */
/* as in grws_spmm, 16 union columns per MFMA step instead of 16 of the      */
/* window's own, so fp32 rounding of the sums may differ in the last bits.   */
/*                                                                          */
/* Layout: group_offset int64 [num_groups+1] (slabs of group q are          */
/* [group_offset[q], group_offset[q+1])), col_indices int32 [num_slabs*16]   */
/* (the group's columns ascending, -1 after its last), header uint32         */
/* [num_slabs][group_size][12] (the packed header of window q*G + i's       */
/* sub-tile of each slab), values [num_values + 8] (A's dtype).  Built for   */
/* columns < num_cols (others dropped); x_rows must not exceed it.           */
/* ------------------------------------------------------------------------ */
typedef struct grws_grouped_tiles {
    const int64_t* group_offset;
    const int32_t* col_indices;
    const uint32_t* header;
    const void* values;
    int64_t num_groups;
    int64_t num_slabs;
    int64_t num_values;
    int64_t max_group_slabs;
    int64_t num_cols;
    int32_t group_size; /* 2, 4 or 8 */
} grws_grouped_tiles;

/* Workspace for both build calls (tile slots: sort keys, ranks, positions). */
size_t grws_group_tiles_workspace_bytes(const grws_bcsr* A, int64_t num_cols, int32_t group_size);

/* Pass 1 (synchronises `stream`): the union columns per group; writes the
 * host *num_slabs, *num_values and the longest group *max_group_slabs. */
int grws_group_tiles_count(const grws_bcsr* A, int64_t num_cols, int32_t group_size, void* workspace,
                           size_t workspace_bytes, int64_t* num_slabs, int64_t* num_values,
                           int64_t* max_group_slabs, void* stream);

/* Pass 2: writes the four arrays, reading what pass 1 left in the same,
 * unchanged, workspace. */
int grws_group_tiles_fill(const grws_bcsr* A, int64_t num_cols, int32_t group_size, int64_t num_slabs,
                          int64_t* group_offset, int32_t* col_indices, uint32_t* header, void* values,
                          int64_t num_values, void* workspace, size_t workspace_bytes, void* stream);

/* Y[16W x n_cols] = A X (+ R on rows < r_rows when r is not NULL, as in
 * grws_spmm_residual) over grouped tiles (16-bit X, values, R and Y of one
 * dtype; n_cols and ldx multiples of 8, X 16-byte aligned). */
int grws_spmm_grouped(const grws_bcsr* A, const grws_grouped_tiles* Gt, const void* x, int32_t x_dtype,
                      int64_t x_rows, int64_t ldx, int64_t n_cols, const void* r, int64_t ldr, int64_t r_rows,
                      void* y, int32_t y_dtype, int64_t ldy, void* stream);

/* Y = A X + R: as grws_spmm_packed (P may be NULL for the dense tiles),
 * with R [r_rows x ldr] in the y dtype added to rows < r_rows of the
 * product in fp32 before Y is rounded; rows >= r_rows get A X alone.  R may
 * be Y itself (each element is read before it is written).  No counterpart
 * in the reference, which adds the self path's product with a separate
 * tensor add after the SpMM (layers/layer.py:150-191); the graph
 * convolution fuses that add here. */
int grws_spmm_residual(const grws_bcsr* A, const grws_packed_tiles* P, const grws_spmm_plan* plan,
                       const void* x, int32_t x_dtype, int64_t x_rows, int64_t ldx, int64_t n_cols,
                       const void* r, int64_t ldr, int64_t r_rows, void* y, int32_t y_dtype, int64_t ldy,
                       void* workspace, size_t workspace_bytes, void* stream);

/* Tuning overrides of the SpMM dispatch, for benchmarks and tests only.
 * No counterpart in the reference.  Names: GRWS_SPMM_NBLK, GRWS_SPMM_WAVES,
 * GRWS_SPMM_KERNEL, GRWS_SPMM_ORDER, GRWS_SPMM_NARROW, GRWS_SPMM_C320,
 * GRWS_GRP_WPW, GRWS_GRP_NBLK, GRWS_GRP_C320, GRWS_GRP_K32, GRWS_GRP_DMA.  Each starts from the
 * environment variable of that name, read once when the library is loaded;
 * value -1 clears the override (the measured default then applies).  The
 * overrides are process-wide: set them only where no other thread is in
 * an SpMM call.  get returns -1 when unset or for an unknown name. */
int grws_spmm_set_tuning(const char* name, int32_t value);
int32_t grws_spmm_get_tuning(const char* name);

/*
 * grws_spmm_residual without a workspace argument; it allocates nothing.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The partial sums of split windows go to
 * a device array the library owns, GRWS_SPMM_NOALLOC_SCRATCH_BYTES on every
 * GPU it runs on, held until the process ends; a call whose plan needs more
 * (grws_spmm_workspace_bytes(plan, n_cols)) returns GRWS_E_CAPACITY.  All
 * calls on one GPU share that array: calls that overlap in time on one GPU
 * (different streams or threads) race and give wrong results.  The stream
 * must belong to the current device (a stream of another device returns
 * GRWS_E_INVALID).  r may be NULL (Y = A X).
 */
#define GRWS_SPMM_NOALLOC_SCRATCH_BYTES (16u << 20)
int grws_spmm_noalloc(const grws_bcsr* A, const grws_packed_tiles* P, const grws_spmm_plan* plan,
                      const void* x, int32_t x_dtype, int64_t x_rows, int64_t ldx, int64_t n_cols,
                      const void* r, int64_t ldr, int64_t r_rows, void* y, int32_t y_dtype, int64_t ldy,
                      void* stream);

/* ------------------------------------------------------------------------ */
/* CSR -> BCSR on host cores.  Replaces core_lib.csr_to_bcsr_cpu             */
/* (bind.cpp:143-150 -> convert_wrapper.cpp:27-180): same layout, same       */
/* "last duplicate in CSR order wins" rule.  Host pointers.                  */
/* ------------------------------------------------------------------------ */

/* Pass 1: tiles per window, written as the prefix sum window_offset
 * [num_windows+1]; *num_tiles_out = total tiles. */
int grws_csr_to_bcsr_host_count(int64_t num_rows, const int64_t* row_ptr, const int32_t* col_idx,
                                int32_t tile_rows, int32_t tile_cols, int64_t* window_offset,
                                int64_t* num_tiles_out, int32_t num_threads);

/* Pass 2: fills col_indices [num_tiles*tile_cols] and values
 * [num_tiles*tile_rows*tile_cols] (float32). */
int grws_csr_to_bcsr_host_fill(int64_t num_rows, const int64_t* row_ptr, const int32_t* col_idx,
                               const float* values, int32_t tile_rows, int32_t tile_cols,
                               const int64_t* window_offset, int32_t* col_indices,
                               float* out_values, int32_t num_threads);

/* ------------------------------------------------------------------------ */
/* On-device BCSR build.  Replaces core_lib.csr_to_bcsr_cpu on device        */
/* graphs (bind.cpp:143-150 -> convert_wrapper.cpp:27-180, called from       */
/* data/bcsr.py:190-234): identical window_offset / col_indices / values,    */
/* identical "last duplicate in input order wins" rule.  With transpose != 0 */
/* it builds the BCSR of A^T instead (windows over A's columns), the cached  */
/* transpose the backward pass runs on in place of the reference's atomic    */
/* scatter (spmm_tc.cuh:211-270).  Device pointers.                          */
/* ------------------------------------------------------------------------ */

/* Workspace bytes of one build (count + fill share it). */
size_t grws_bcsr_build_workspace_bytes(int64_t nnz, int64_t num_rows, int64_t num_cols,
                                       int32_t transpose);

/*
 * Phase 1.  Edges of A [num_rows x num_cols] given either as CSR (row_ptr
 * [num_rows+1], rows NULL) or as COO (rows [nnz], row_ptr NULL); cols [nnz];
 * values [nnz] float32 or NULL (all ones).  Writes window_offset
 * [ceil(R/16)+1] (R = num_rows, or num_cols when transposed), synchronises
 * `stream` and returns the tile count in *num_tiles_out.  GRWS_E_RANGE when a
 * row or column is out of range or row_ptr is not a CSR row pointer.
 */
int grws_bcsr_build_count(const int64_t* row_ptr, const int32_t* rows, const int32_t* cols,
                          const float* values, int64_t nnz, int64_t num_rows, int64_t num_cols,
                          int32_t tile_cols, int32_t transpose, int64_t* window_offset,
                          void* workspace, size_t workspace_bytes, int64_t* num_tiles_out,
                          void* stream);

/* Phase 2.  Same sizes and the workspace phase 1 left (unmodified); fills
 * col_indices [num_tiles*tile_cols] (-1 padding) and values
 * [num_tiles*16*tile_cols] of values_dtype (round to nearest even). */
int grws_bcsr_build_fill(int64_t nnz, int64_t num_rows, int64_t num_cols, int32_t tile_cols,
                         int32_t transpose, const int64_t* window_offset, int64_t num_tiles,
                         int32_t* col_indices, void* values, int32_t values_dtype,
                         void* workspace, size_t workspace_bytes, void* stream);

/* BCSR -> COO: every slot with a column in [0, num_cols) and a non-zero
 * value becomes one edge (row = 16*window + row in tile), tile by tile and
 * each tile's slots in (row, column) order.  Feeds the
 * transposed build of a graph that exists only as BCSR (sampled subgraphs,
 * from_components).  count synchronises `stream`. */
size_t grws_bcsr_to_coo_workspace_bytes(int64_t num_tiles);
int grws_bcsr_to_coo_count(const grws_bcsr* A, int64_t num_cols, void* workspace,
                           size_t workspace_bytes, int64_t* nnz_out, void* stream);
int grws_bcsr_to_coo_fill(const grws_bcsr* A, int64_t num_cols, int32_t* rows, int32_t* cols,
                          float* values, void* workspace, size_t workspace_bytes, void* stream);

/* COO -> CSR, replacing BCSRGraph._coo_to_csr (data/bcsr.py:162-187):
 * stable sort by (src, dst) (the reference sorts on src*num_rows+dst with a
 * non-stable argsort, :170-171), row_ptr int64 [num_rows+1], col_idx = dst,
 * values = weights in sorted order or ones.  Synchronises `stream`. */
size_t grws_coo_to_csr_workspace_bytes(int64_t nnz, int64_t num_rows, int64_t num_cols);
int grws_coo_to_csr(const int32_t* src, const int32_t* dst, const float* weights, int64_t nnz,
                    int64_t num_rows, int64_t num_cols, int64_t* row_ptr, int32_t* col_idx,
                    float* values, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Reindex + prune.  Replaces core_lib.reindex_bcsr (bind.cpp:153-159 ->     */
/* reindex_wrapper.cu:27-68, kernel reindex.cuh:33-102): out_cols[i] =       */
/* pos * tile_rows + g % tile_rows where pos is the index of window          */
/* g / tile_rows (C division) in the sorted active_windows; a slot whose     */
/* window is absent gets column 0 and its tile_rows values are zeroed IN     */
/* PLACE in `values` ([num_indices / tile_cols][tile_rows][tile_cols]).      */
/* ------------------------------------------------------------------------ */
int grws_reindex_prune(const int32_t* in_cols, int64_t num_indices, void* values,
                       int32_t values_dtype, const int32_t* active_windows, int64_t num_active,
                       int32_t tile_rows, int32_t tile_cols, int32_t* out_cols, void* stream);

/* ------------------------------------------------------------------------ */
/* Node-wise fanout sampling, one hop.  Takes the place of the per-hop       */
/* column-sampling phase of core_lib.sample_all_layers (bind.cpp:99-121 ->   */
/* sampling_wrapper.cu:365-438, phase 1 = sampling.cuh:65-448) for the       */
/* mini-batch path that draws a fixed fanout per node (BCSRSampler's         */
/* sample_layers, sampler/sampler.py:186-279, calls it once per hop, hop 0   */
/* from the seeds with the last fanout, sampler.py:204).                     */
/*                                                                          */
/* For every frontier node v (CSR indptr int64 [num_nodes+1], indices int32  */
/* [nnz]): deg <= fanout takes every neighbour, otherwise Floyd's algorithm  */
/* picks fanout distinct CSR positions with draws                            */
/*   u = word 0 of Philox4x32-10(counter (v_lo, v_hi, d, 0), key (seed_lo,   */
/*       seed_hi)),  t = (u64(u) * (j+1)) >> 32,  j = deg-fanout+d.          */
/* Edges are written in frontier order, then ascending CSR position:        */
/* edge_dst = frontier position (int32), edge_src = neighbour id (int64),   */
/* edge_val (optional, may be NULL) = 1/sqrt((deg(v)+1)(deg(src)+1)) from    */
/* out-degrees.  fanout in [1, 64]; edge_capacity >= num_frontier * fanout.  */
/* Synchronises `stream`; *num_edges_out = edges written.  GRWS_E_RANGE for  */
/* an id outside [0, num_nodes) or an invalid indptr.                        */
/* ------------------------------------------------------------------------ */
size_t grws_sample_hop_workspace_bytes(int64_t num_frontier);
int grws_sample_hop(const int64_t* indptr, const int32_t* indices, int64_t num_nodes, int64_t nnz,
                    const int64_t* frontier, int64_t num_frontier, int32_t fanout, uint64_t seed,
                    int32_t* edge_dst, int64_t* edge_src, float* edge_val, int64_t edge_capacity,
                    void* workspace, size_t workspace_bytes, int64_t* num_edges_out, void* stream);

/* ------------------------------------------------------------------------ */
/* Unique + relabel of one hop's sources.  Takes the place of the reference's */
/* next-seed extraction and active-window bookkeeping                       */
/* (sampling_wrapper.cu:283-347 prepare_windows_and_masks, :421-433) and of  */
/* the global -> local mapping its layers apply afterwards (reindex.cuh:33-  */
/* 102): frontier nodes keep local ids [0, F) in frontier order (the         */
/* "destination nodes first" block layout of data/bcsr.py:266-306 and       */
/* layers/layer.py:159-161); sources outside the frontier are appended in    */
/* ascending global id.  Writes src_local [num_edges] int32 and              */
/* next_frontier [num_src] int64 (the frontier followed by the new ids;      */
/* next_capacity >= num_frontier + num_edges).  Frontier ids must be         */
/* distinct (GRWS_E_INVALID otherwise).  Synchronises `stream`.              */
/* ------------------------------------------------------------------------ */
/* ------------------------------------------------------------------------ */
/* One hop in one call: grws_sample_hop + relabel + the hop's BCSR block     */
/* (what BCSRGraph.from_dgl_block builds from a sampled block,               */
/* data/bcsr.py:266-306), with a single synchronisation.  Same results as    */
/* the three separate calls.                                                 */
/*                                                                          */
/* The relabel uses caller-owned state instead of sorting: node_map int32    */
/* [num_nodes], all -1, and bitmap uint32 [ceil(num_nodes/32)], all 0; every */
/* call leaves them so (grws_sample_state_init sets them up).  Calls sharing */
/* one state must not overlap.                                               */
/*                                                                          */
/* Outputs: next_frontier int64 [max_src] (frontier, then new sources in     */
/* ascending id), window_offset int64 [ceil(F/16)+1], col_indices int32 and  */
/* values (values_dtype) for up to max_tiles tiles; the bounds come from     */
/* grws_sample_block_capacity.  counts_out[3] = {edges, sources, tiles}.     */
/* Synchronises `stream`.                                                    */
/* ------------------------------------------------------------------------ */
/* ------------------------------------------------------------------------ */
/* A whole mini-batch in one call: every hop of grws_sample_block, hop h      */
/* from the previous hop's sources, with a single synchronisation at the     */
/* end.  Takes the place of the reference's per-hop loop with a host sync    */
/* per hop (sampling_wrapper.cu:365-438, the sync at :340-344) for the       */
/* node-wise path; BCSRSampler.sample_layers (sampler/sampler.py:186-279)    */
/* passes the fanouts in hop order (reversed, sampler.py:204).  Results are   */
/* those of num_hops grws_sample_block calls, bit for bit.                   */
/*                                                                          */
/* State: node_map int32 [num_nodes] (all -1) and state uint32               */
/* [grws_sample_blocks_state_words(num_nodes)] (all 0), both set up by       */
/* grws_sample_blocks_state_init and left so by every call; the first        */
/* ceil(num_nodes/32) words of state are the bitmap grws_sample_block and    */
/* grws_repack_* take.  Calls sharing one state must not overlap.            */
/*                                                                          */
/* Outputs per hop h (device pointers in host arrays of num_hops entries):   */
/* next_frontier[h] int64 [max_src[h]], window_offset[h] int64              */
/* [ceil(F_h/16)+1 <= ceil(cap/16)+1, see below], col_indices[h] int32       */
/* [max_tiles[h]*tile_cols], values[h] [max_tiles[h]*16*tile_cols], with     */
/* max_src/max_tiles from grws_sample_blocks_capacity; window_offset[h]      */
/* needs ceil(F_cap_h/16)+1 entries where F_cap_0 = num_seeds and            */
/* F_cap_h = max_src[h-1].  counts_out[3*h .. 3*h+2] = {edges, sources,      */
/* tiles} of hop h.  num_hops in [1, 8], fanouts in [1, 64].                 */
/* ------------------------------------------------------------------------ */
size_t grws_sample_blocks_state_words(int64_t num_nodes);
int grws_sample_blocks_state_init(int32_t* node_map, uint32_t* state, int64_t num_nodes, void* stream);
int grws_sample_blocks_capacity(int64_t num_seeds, const int32_t* fanouts, int32_t num_hops, int32_t tile_cols,
                                int64_t num_nodes, int64_t* max_src, int64_t* max_tiles);
size_t grws_sample_blocks_workspace_bytes(int64_t num_seeds, const int32_t* fanouts, int32_t num_hops,
                                          int32_t tile_cols, int64_t num_nodes);
int grws_sample_blocks(const int64_t* indptr, const int32_t* indices, int64_t num_nodes, int64_t nnz,
                       const int64_t* seeds, int64_t num_seeds, const int32_t* fanouts, int32_t num_hops,
                       uint64_t seed, int32_t* node_map, uint32_t* state, int32_t tile_cols, int32_t values_dtype,
                       int64_t* const* next_frontier, int64_t* const* window_offset, int32_t* const* col_indices,
                       void* const* values, void* workspace, size_t workspace_bytes, int64_t* counts_out,
                       void* stream);

/* grws_sample_blocks plus, for each hop h with transpose_hops[h] != 0, the  */
/* BCSR of that hop's block transposed (windows of 16 sources, columns = the */
/* hop's frontier rows 0 .. 16 ceil(F_h/16) - 1), built in the same call     */
/* with no further sync.  It is the matrix the backward SpMM over the block  */
/* multiplies by (the reference's spmm_transpose, spmm_wrapper.cu:109-152,   */
/* reached from layers/layer.py:66-79), bit for bit the BCSR a device build */
/* of the block's transpose makes: every cell with a nonzero value, a       */
/* window's distinct rows ascending.  Outputs per such hop:                  */
/* t_window_offset[h] int64 [max_t_windows[h]+1] (windows past               */
/* ceil(sources/16) hold no tiles), t_col_indices[h] int32                   */
/* [max_t_tiles[h]*tile_cols], t_values[h] [max_t_tiles[h]*16*tile_cols],    */
/* capacities from grws_sample_blocks_transposed_capacity; entries of hops   */
/* not transposed are ignored.  counts_out[5*h .. 5*h+4] = {edges, sources,  */
/* tiles, transposed tiles, most tiles in one transposed window}.            */
int grws_sample_blocks_transposed_capacity(int64_t num_seeds, const int32_t* fanouts, int32_t num_hops,
                                           int32_t tile_cols, int64_t num_nodes, int64_t* max_t_windows,
                                           int64_t* max_t_tiles);
size_t grws_sample_blocks_transposed_workspace_bytes(int64_t num_seeds, const int32_t* fanouts, int32_t num_hops,
                                                     int32_t tile_cols, int64_t num_nodes,
                                                     const int32_t* transpose_hops);
int grws_sample_blocks_transposed(const int64_t* indptr, const int32_t* indices, int64_t num_nodes, int64_t nnz,
                                  const int64_t* seeds, int64_t num_seeds, const int32_t* fanouts, int32_t num_hops,
                                  uint64_t seed, int32_t* node_map, uint32_t* state, int32_t tile_cols,
                                  int32_t values_dtype, int64_t* const* next_frontier,
                                  int64_t* const* window_offset, int32_t* const* col_indices, void* const* values,
                                  const int32_t* transpose_hops, int64_t* const* t_window_offset,
                                  int32_t* const* t_col_indices, void* const* t_values, void* workspace,
                                  size_t workspace_bytes, int64_t* counts_out, void* stream);

/* grws_sample_blocks(_transposed) for replay from a captured HIP graph: the */
/* same work, enqueued on `stream` with no host sync.  Capacities, grids and */
/* the workspace are those of max_seeds seeds (>= 1); the batch's seed      */
/* count is read on the device from *num_seeds_dev (0 .. max_seeds; outside */
/* that range the batch is empty and the error flag is set), and the seeds  */
/* from seeds[0 .. count).  transpose_hops may be NULL (no transposes).      */
/* Instead of counts_out, the counters are left in device memory:          */
/* counts_dev[0 .. 5 num_hops + 1] = {F[0..H], E[H], T[H], TT[H], TM[H],    */
/* err}: F[h] frontier sizes (F[h+1] = sources of hop h), E edges, T tiles, */
/* TT / TM tiles of the transposed block and most tiles in one of its       */
/* windows, err a flag word for grws_sample_blocks_error.  The reference    */
/* syncs once per hop (sampling_wrapper.cu:340-344); this call syncs never, */
/* so a caller can capture it once and replay it per batch.                 */
int grws_sample_blocks_enqueue(const int64_t* indptr, const int32_t* indices, int64_t num_nodes, int64_t nnz,
                               const int64_t* seeds, int64_t max_seeds, const int64_t* num_seeds_dev,
                               const int32_t* fanouts, int32_t num_hops, uint64_t seed, int32_t* node_map,
                               uint32_t* state, int32_t tile_cols, int32_t values_dtype,
                               int64_t* const* next_frontier, int64_t* const* window_offset,
                               int32_t* const* col_indices, void* const* values, const int32_t* transpose_hops,
                               int64_t* const* t_window_offset, int32_t* const* t_col_indices,
                               void* const* t_values, void* workspace, size_t workspace_bytes, int64_t* counts_dev,
                               void* stream);
/* The status (and grws_last_error message) of an enqueued batch's error    */
/* flag, counts_dev[5 num_hops + 1] read back by the caller: GRWS_OK for 0. */
int grws_sample_blocks_error(int64_t err);

/* n device-to-device copies in one launch (32 ranges per launch): bytes[i] */
/* bytes from src[i] to dst[i], both 16-byte aligned.  Used to hand out a   */
/* replayed batch's outputs as compact tensors.  Asynchronous on `stream`.  */
int grws_copy_ranges(const void* const* src, void* const* dst, const int64_t* bytes, int32_t n, void* stream);

/* n int64 fills in one launch (32 ranges per launch): count[i] elements   */
/* from dst[i] (8-byte aligned) set to value[i].  No counterpart in the     */
/* reference: the captured mini-batch step uses it with grws_copy_ranges to */
/* load a batch into its bucket's static buffers (the window offsets past   */
/* the batch's windows, the padding labels) in two launches instead of one */
/* per array.  Asynchronous on `stream`.                                    */
int grws_fill_ranges_i64(int64_t* const* dst, const int64_t* count, const int64_t* value, int32_t n, void* stream);

/* Input features of a sampled batch: dst row i = src row idx[i] for        */
/* i < n, row_bytes bytes per row, rows ld_src / ld_dst bytes apart; idx is  */
/* int64 (idx_is_i64 != 0) or int32.  An index outside [0, src_rows) gives a */
/* zero row and, when err is not NULL, sets *err to 1 (nothing else writes   */
/* *err: the caller clears it).  Replaces the producer's feature gather      */
/* (helper/engine.py:132-141 gathers features[input_nodes] per batch) with   */
/* one launch that moves 16-byte units whenever the row length, pitches and  */
/* base addresses allow.  Asynchronous on `stream`.                          */
int grws_gather_rows(const void* src, int64_t src_rows, int64_t ld_src, const void* idx, int32_t idx_is_i64,
                     int64_t n, int64_t row_bytes, void* dst, int64_t ld_dst, int32_t* err, void* stream);

int grws_sample_state_init(int32_t* node_map, uint32_t* bitmap, int64_t num_nodes, void* stream);
size_t grws_sample_block_workspace_bytes(int64_t num_frontier, int32_t fanout, int64_t num_nodes);
int grws_sample_block_capacity(int64_t num_frontier, int32_t fanout, int32_t tile_cols,
                               int64_t* max_src, int64_t* max_tiles);
int grws_sample_block(const int64_t* indptr, const int32_t* indices, int64_t num_nodes, int64_t nnz,
                      const int64_t* frontier, int64_t num_frontier, int32_t fanout, uint64_t seed,
                      int32_t* node_map, uint32_t* bitmap, int32_t tile_cols, int32_t values_dtype,
                      int64_t* next_frontier, int64_t max_src, int64_t* window_offset,
                      int32_t* col_indices, void* values, int64_t max_tiles, void* workspace,
                      size_t workspace_bytes, int64_t* counts_out, void* stream);

/* ------------------------------------------------------------------------ */
/* Window top-K sampling: the reference-compatible core_lib.sample_all_layers */
/* (bind.cpp:99-121 -> sampling_wrapper.cu:365-438), one call per phase.     */
/* ------------------------------------------------------------------------ */

/* HACS scoring parameters (sampler/sampler.py:101-151, sampling.cuh:251-    */
/* 270).  Pass NULL or use_hacs = 0 for the default score                   */
/* trunc((1 + 10|v|) * 1000).  Device arrays; the counts bound every lookup. */
typedef struct grws_hacs {
    const float* static_scores;     /* [num_static_scores], indexed by column */
    const int32_t* window_part_ids; /* [num_window_part_ids] part of each window or -1 */
    const int32_t* part_starts;     /* [num_parts] first column of each part */
    const int32_t* part_ends;       /* [num_parts] one past its last column */
    int64_t num_static_scores;
    int64_t num_window_part_ids;
    int64_t num_parts;
    float alpha, beta, delta, gamma_bonus, score_scale;
    int32_t use_hacs;
    int32_t locality_enabled;
} grws_hacs;

/* S = roundup32(fanout), the reference's per-window output stride         */
/* (sampling_wrapper.cu:88).                                                 */
int32_t grws_window_sample_num(int32_t fanout);

/* Seeds -> sorted unique active windows and OR-ed row masks, replacing     */
/* prepare_windows_and_masks (sampling_wrapper.cu:283-347): id -> (id / tile_rows, */
/* 1 << id % tile_rows); -1 is skipped.  Other ids outside [0, num_nodes)    */
/* are skipped when drop_out_of_range != 0 (the inter-hop filter of         */
/* sampling_wrapper.cu:424-429) and are GRWS_E_RANGE otherwise.  Outputs    */
/* hold num_ids entries; *num_active_out = windows written.  Synchronises.  */
size_t grws_window_seeds_workspace_bytes(int64_t num_ids);
int grws_window_seeds(const int32_t* ids, int64_t num_ids, int64_t num_nodes, int32_t tile_rows,
                      int32_t drop_out_of_range, int32_t* active_windows, int32_t* masks,
                      void* workspace, size_t workspace_bytes, int64_t* num_active_out,
                      void* stream);

/* Phase 1 + 2, replacing warp_centric_find_top_k_kernel (sampling.cuh:65-  */
/* 448) and the tile-count scan (sampling_wrapper.cu:160-177): per active    */
/* window, the columns ranked by the reference's score, top-CAP by (total    */
/* desc, column asc) with CAP = 32/128/256 for S <= 32/128/256, re-sorted    */
/* ascending, first min(kept, S) kept.  Writes sampled_cols [num_active * S] */
/* (-1 padded), sampled_slots [num_active * S] (the column's slot index in   */
/* its input window), out_window_offset [num_active+1] int64; synchronises   */
/* and returns the output tile count.  fanout in [1, 256].  A workspace     */
/* larger than grws_window_topk_workspace_bytes(num_active) lends the rest   */
/* to windows of more than 1,024 slots as a chunk table and key scratch     */
/* (8 bytes per slot; grws_window_topk_key_scratch_bytes(A) covers every    */
/* window of A): their keys are then computed once, spread over many        */
/* work-groups, instead of within the window's own work-group or once per   */
/* selection pass.  The results do not depend on it.                         */
size_t grws_window_topk_workspace_bytes(int64_t num_active);
size_t grws_window_topk_key_scratch_bytes(const grws_bcsr* A);
int grws_window_topk(const grws_bcsr* A, const int32_t* active_windows, int64_t num_active,
                     int32_t fanout, const grws_hacs* hacs, int32_t* sampled_cols,
                     int32_t* sampled_slots, int64_t* out_window_offset, void* workspace,
                     size_t workspace_bytes, int64_t* num_tiles_out, void* stream);

/* Phase 3, replacing build_col_to_val_map_kernel + recompress_sampled_bcsr */
/* _kernel (sampling.cuh:471-579, 707-773): out_cols [num_tiles*tile_cols]   */
/* and out_values [num_tiles*16*tile_cols] in A's values dtype, sized        */
/* exactly (the reference over-allocates and pre-fills -1 / -1.0,           */
/* sampling_wrapper.cu:215-218).                                             */
int grws_window_recompress(const grws_bcsr* A, const int32_t* active_windows, int64_t num_active,
                           int32_t fanout, const int32_t* sampled_cols,
                           const int32_t* sampled_slots, const int64_t* out_window_offset,
                           int64_t num_tiles, int32_t* out_cols, void* out_values, void* stream);

/* Every layer of sample_all_layers (sampling_wrapper.cu:365-438) in one     */
/* call with one synchronisation: layer l's seeds are the batch's (l = 0,   */
/* ids outside [0, num_nodes) other than -1 are GRWS_E_RANGE) or layer      */
/* l-1's sampled columns (-1 and ids past num_nodes dropped), its windows   */
/* those of grws_window_seeds (tile_rows 16), its sample those of           */
/* grws_window_topk and grws_window_recompress with fanouts[l]: the same    */
/* results.  The outputs are caller buffers sized by the bounds query       */
/* (layer l: window_offset [max_active+1], active_windows and masks         */
/* [max_active], col_indices [max_tiles*tile_cols], values                  */
/* [max_tiles*16*tile_cols] in A's values dtype); counts [2*num_layers]     */
/* (host) receives each layer's active windows A and tiles T: the layer's  */
/* arrays are the first A+1, A, A, T*tile_cols and T*16*tile_cols entries.  */
/* phase_ms [2*num_layers] (host, or NULL) receives each layer's            */
/* top-K and recompression times.  Workspace beyond                         */
/* grws_window_sample_layers_workspace_bytes is key scratch as for          */
/* grws_window_topk.  Replaces the per-layer calls' host syncs (two per     */
/* layer) with one.                                                         */
int grws_window_sample_layers_bounds(const grws_bcsr* A, int64_t num_nodes, int64_t num_seeds,
                                     const int32_t* fanouts, int32_t num_layers, int64_t* max_active,
                                     int64_t* max_tiles);
size_t grws_window_sample_layers_workspace_bytes(const grws_bcsr* A, int64_t num_nodes, int64_t num_seeds,
                                                 const int32_t* fanouts, int32_t num_layers);
int grws_window_sample_layers(const grws_bcsr* A, int64_t num_nodes, const int32_t* seeds, int64_t num_seeds,
                              const int32_t* fanouts, int32_t num_layers, const grws_hacs* hacs,
                              int64_t* const* window_offset, int32_t* const* col_indices, void* const* values,
                              int32_t* const* active_windows, int32_t* const* masks, int64_t* counts,
                              float* phase_ms, void* workspace, size_t workspace_bytes, void* stream);
/* grws_window_sample_layers without its read-back (sampling_wrapper.cu:    */
/* 365-438 with no host sync at all), so that a caller can capture it once  */
/* in a HIP graph and replay it per batch: the seed count is read on the   */
/* device from num_seeds_dev[0]; every buffer, the workspace and the grids  */
/* are sized by max_seeds (bounds and workspace queries with max_seeds); a  */
/* larger device count is flagged (GRWS_E_CAPACITY) and clamped.  When the  */
/* stream reaches the end of the call, out_dev [2*num_layers + 1] (device)  */
/* holds each layer's active windows and tiles (as counts above) and then   */
/* the batch's error flags, for grws_window_sample_layers_status.  No      */
/* phase timings.  Same results as grws_window_sample_layers.  side_stream  */
/* (or NULL): a second stream the caller owns on the same device (one of   */
/* another device: GRWS_E_INVALID); the windows of over 1,024 slots run on  */
/* it, forked from and joined back to `stream` with events, also while      */
/* `stream` is being captured (a capture then records the two branches side */
/* by side).  With NULL they run on the library's extra stream, or on       */
/* `stream` itself under capture.                                           */
int grws_window_sample_layers_enqueue(const grws_bcsr* A, int64_t num_nodes, const int32_t* seeds,
                                      int64_t max_seeds, const int64_t* num_seeds_dev, const int32_t* fanouts,
                                      int32_t num_layers, const grws_hacs* hacs, int64_t* const* window_offset,
                                      int32_t* const* col_indices, void* const* values,
                                      int32_t* const* active_windows, int32_t* const* masks, void* workspace,
                                      size_t workspace_bytes, int64_t* out_dev, void* stream, void* side_stream);
/* The status (and grws_last_error message) of an enqueued call's error     */
/* flags, out_dev[2*num_layers] read back by the caller: GRWS_OK for 0.     */
int grws_window_sample_layers_status(int64_t err);

size_t grws_relabel_workspace_bytes(int64_t num_frontier, int64_t num_edges);
int grws_relabel(const int64_t* frontier, int64_t num_frontier, const int64_t* edge_src,
                 int64_t num_edges, int64_t num_nodes, int32_t* src_local, int64_t* next_frontier,
                 int64_t next_capacity, void* workspace, size_t workspace_bytes,
                 int64_t* num_src_out, void* stream);

/* ------------------------------------------------------------------------ */
/* Weight gradient C[M x N] = A^T B, A [K x M] and B [K x N] row-major       */
/* F16/BF16, fp32 accumulation, C in F32 or the input dtype.  The backward   */
/* of the graph convolution (layers/layer.py:61-92: grad_weight =            */
/* features^T @ grad_input_aggr, and the self path's weight through          */
/* autograd, layer.py:171-175) has K = node count and M, N = layer widths;  */
/* K is split over work-groups and the fp32 partials added in a fixed order  */
/* (deterministic).  M, N, lda, ldb multiples of 8; A and B 16-byte aligned. */
/* ------------------------------------------------------------------------ */
size_t grws_gemm_tn_workspace_bytes(int64_t K, int64_t M, int64_t N);
int grws_gemm_tn(const void* a, int64_t lda, const void* b, int64_t ldb, int32_t in_dtype, int64_t K,
                 int64_t M, int64_t N, void* c, int64_t ldc, int32_t out_dtype, void* workspace,
                 size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Halo-aware subgraph repack: the device part of BCSRSampler.repack_subgraph */
/* (sampler/sampler.py:420-690).  window_ids: int64, strictly ascending, in  */
/* [0, num_windows).  State: the sampler's bitmap (uint32 [ceil(n/32)], all  */
/* 0) and node map (int32 [n], all -1), n = num_nodes; every successful call */
/* sequence prepare -> [externals] -> finish leaves both as found (prepare   */
/* leaves the candidate marks in the bitmap for the next two calls; a failed */
/* prepare clears them).                                                     */
/*   prepare: new_offsets int64 [num_selected+1] (device); synchronises and  */
/*     writes counts_out[3] = {tiles, internal nodes, external candidates}.  */
/*   externals: the candidates ascending into int64 [candidates] (device).   */
/*   finish: kept_external (ascending, device) or NULL to keep every         */
/*     candidate (num_kept must then equal the candidate count); outputs:    */
/*     input_nodes int64 [internal + kept] (internal nodes window by window, */
/*     then the kept externals), halo/inner cols int32 [tiles*tc] and values */
/*     [tiles*16*tc] in the graph's values dtype (masked columns -1 with     */
/*     zero values; inner also masks columns >= internal).  Synchronises and */
/*     writes flags_out[0] = 1 when a halo value is NaN.                     */
/* ------------------------------------------------------------------------ */
size_t grws_repack_workspace_bytes(int64_t num_selected, int64_t num_nodes);
int grws_repack_prepare(const grws_bcsr* g, int64_t num_nodes, const int64_t* window_ids,
                        int64_t num_selected, uint32_t* bitmap, int64_t* new_offsets,
                        int64_t* counts_out, void* workspace, size_t workspace_bytes, void* stream);
int grws_repack_externals(const uint32_t* bitmap, int64_t num_nodes, int64_t* external_out,
                          void* workspace, size_t workspace_bytes, void* stream);
int grws_repack_finish(const grws_bcsr* g, int64_t num_nodes, const int64_t* window_ids,
                       int64_t num_selected, const int64_t* new_offsets, int64_t num_internal,
                       const int64_t* kept_external, int64_t num_kept, int32_t* node_map,
                       uint32_t* bitmap, int64_t* input_nodes, int32_t* halo_cols, void* halo_values,
                       int32_t* inner_cols, void* inner_values, int32_t* flags_out, void* workspace,
                       size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Fused hidden-layer tail: out = dropout(LayerNorm(act(z))) per row, the   */
/* sequence of models/model.py:259-264 (act, self.norms[l], dropout).  act  */
/* 0 = identity, 1 = ReLU; LayerNorm over dim (biased variance, eps) with   */
/* fp32 gamma/beta; dropout with probability p, scale 1/(1-p), element     */
/* (r, c) kept iff word c%4 of Philox4x32-10 at counter (r_lo, r_hi, c/4,  */
/* 0), key seed, is >= p * 2^32; the backward recomputes it.  seed_dev,     */
/* when not NULL, points to a device uint64 read in place of seed (a seed   */
/* drawn on the device, so a captured graph draws a new mask per replay).   */
/* z/out/dout/dz                                                            */
/* in F32/F16/BF16; dim a multiple of 4, <= 1024; rows and leading          */
/* dimensions multiples of 4 elements, 8-byte aligned.  mean/rstd: fp32     */
/* [rows] saved for the backward (both NULL to skip).  The backward writes  */
/* dz (z's dtype) and fp32 dgamma/dbeta [dim], summed in a fixed order for  */
/* a given device (the number of partial sums is the device's resident      */
/* work-group count).                                                       */
/* ------------------------------------------------------------------------ */
int grws_act_norm_dropout_fwd(const void* z, int32_t z_dtype, int64_t ldz, int64_t rows, int64_t dim,
                              int32_t act, const float* gamma, const float* beta, float eps, float p,
                              uint64_t seed, const uint64_t* seed_dev, void* out, int32_t out_dtype,
                              int64_t ldo, float* mean, float* rstd, void* stream);
size_t grws_act_norm_dropout_bwd_workspace_bytes(int64_t rows, int64_t dim);
int grws_act_norm_dropout_bwd(const void* dout, int32_t dout_dtype, int64_t ldg, const void* z,
                              int32_t z_dtype, int64_t ldz, int64_t rows, int64_t dim, int32_t act,
                              const float* mean, const float* rstd, const float* gamma, float p,
                              uint64_t seed, const uint64_t* seed_dev, void* dz, int64_t lddz,
                              float* dgamma, float* dbeta, void* workspace, size_t workspace_bytes,
                              void* stream);

/* ------------------------------------------------------------------------ */
/* Cross-entropy over a subset of the rows of logits [total_rows x ld]      */
/* (helper/engine.py:22-41: F.cross_entropy(logits[idx], labels[idx]) and   */
/* the argmax hit count).  rows: int64 [n] row ids (NULL = rows 0..n-1),    */
/* labels: int64 [n]; label -100 is ignored (torch's ignore_index).         */
/* Forward, no sync: lse_out fp32 [n], loss_out fp32 device scalar (mean    */
/* over counted rows; NaN when none counts or a label is out of range,      */
/* where torch asserts), counts_out int64 [3] device = {argmax hits,        */
/* counted rows, bad input flag}.  Backward: grad rows of `rows` get        */
/* (softmax - onehot) * dloss / counted (0 for ignored rows); other rows of */
/* grad are left as they are (zero them first).  rows must be distinct.     */
/* ------------------------------------------------------------------------ */
size_t grws_cross_entropy_workspace_bytes(int64_t n);
int grws_cross_entropy_fwd(const void* logits, int32_t dtype, int64_t ld, int64_t total_rows,
                           int64_t classes, const int64_t* rows, const int64_t* labels, int64_t n,
                           float* lse_out, float* loss_out, int64_t* counts_out, void* workspace,
                           size_t workspace_bytes, void* stream);
int grws_cross_entropy_bwd(const void* logits, int32_t dtype, int64_t ld, int64_t total_rows,
                           int64_t classes, const int64_t* rows, const int64_t* labels, int64_t n,
                           const float* lse, const float* dloss, const int64_t* counts, void* grad,
                           int32_t grad_dtype, int64_t ldg, void* stream);

/* ------------------------------------------------------------------------ */
/* Measurement only: no counterpart in the reference.  The random row-      */
/* gather ceiling that bounds the SpMM's X reads, for benchmark reports.    */
/* n_idx row indices (int32, a multiple of 8; values outside [0, rows)      */
/* read zeros) into a table of `rows` rows pitch_bytes apart (16-byte       */
/* aligned, at most 2^31 bytes);                                            */
/* every index loads the row's first segments * 128 bytes (1, 5 or 10, at   */
/* most the pitch), 16 bytes per lane.  `blocks` work-groups of 256 lanes   */
/* (1..65536) share the list; out[4 * blocks] receives one word per wave    */
/* (a fold of what it read).  Asynchronous on `stream`; time it with events */
/* on that stream.                                                          */
/* ------------------------------------------------------------------------ */
int grws_probe_row_gather(const void* table, int64_t rows, int64_t pitch_bytes, int32_t segments,
                          const int32_t* idx, int64_t n_idx, uint32_t* out, int32_t blocks, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GRWS_H */
