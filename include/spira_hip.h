/*
 * spira_hip.h -- C ABI of libspira_hip.so, the gfx950 (MI355X) kernel library
 * behind the spira sparse-convolution extension.
 *
 * Plain pointers and sizes only.  Every pointer argument is device memory on
 * the current HIP device unless stated otherwise; `stream` is a hipStream_t.
 * Every function returns 0 on success or a non-zero status; the message of
 * the last failure on the calling thread is spira_hip_last_error().
 *
 * Keys are packed voxel coordinates: key_bits = 64 packs x24|y24|z16,
 * key_bits = 32 packs x12|y12|z8 (reference compress_layout.h:11-44).
 * Key arrays are uint64_t / uint32_t bit patterns (torch int64 / int32).
 *
 * Each declaration names the reference interface it replaces; reference
 * paths are under source/csrc/spira/ of SPIN-Research-Group/Spira.
 */
#ifndef SPIRA_HIP_H_
#define SPIRA_HIP_H_

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Message of the last failed call on this thread (reference: SpiraException,
 * common/exception.h:9-28). */
const char *spira_hip_last_error(void);

/* ---------------------------------------------------------------- coords */

/* coords [n,3] int32 -> keys [n] (reference: kernels Compress,
 * cuda/kernels/compress.cuh:9-23). */
int spira_hip_pack(const int32_t *coords, int64_t n, int key_bits, void *keys, hipStream_t stream);

/* keys [n] -> coords [n,3] int32 (reference: cuda_unflatten,
 * torch/cuda_arg_sort_coordinates.cu:41-65; kernel UnCompress compress.cuh:28-46). */
int spira_hip_unpack(const void *keys, int64_t n, int key_bits, int32_t *coords, hipStream_t stream);

/* Workspace bytes for spira_hip_flatten_sort. */
int spira_hip_flatten_sort_workspace(int64_t n, int key_bits, size_t *bytes);

/* Pack, then stable ascending sort on the unsigned key; perm_out[i] is the
 * input row of sorted key i (reference: cuda_flatten_sort,
 * torch/cuda_arg_sort_coordinates.cu:11-39; FlattenSort arg_sort_coodrinates.cu:36-88). */
int spira_hip_flatten_sort(const int32_t *coords, int64_t n, int key_bits, void *keys_out, int32_t *perm_out,
                           void *workspace, size_t workspace_bytes, hipStream_t stream);

/* spira_hip_flatten_sort without any allocation: the workspace is a fixed
 * 32 MiB device array inside the library (one per GPU, held until the
 * process ends), so n is limited to 1048576 points; larger n is rejected.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Calls that overlap on one GPU share the
 * array and race; serialise them (one stream, or events). */
int spira_hip_flatten_sort_noalloc(const int32_t *coords, int64_t n, int key_bits, void *keys_out, int32_t *perm_out,
                                   hipStream_t stream);

/* Workspace bytes for spira_hip_radix_sort_pairs. */
int spira_hip_radix_sort_workspace(int64_t n, int key_bits, size_t *bytes);

/* Stable ascending sort of n (key, int32 value) pairs, keys unsigned 32- or
 * 64-bit: (keys_in, vals_in) -> (keys_out, vals_out); the inputs are left
 * unchanged, n < 2^30; vals_in may be null (the values are then the input
 * indices).  A hand-written LSD radix sort (digits of up to 9 bits over the
 * bits in which the keys differ, decoupled look-back, staged coalesced
 * scatter); flatten_sort keeps rocPRIM's sort, which is faster at the
 * benchmark sizes (reference:
 * the cub::DeviceRadixSort::SortPairs call of FlattenSort,
 * cuda/functions/arg_sort_coodrinates.cu:36-88). */
int spira_hip_radix_sort_pairs(const void *keys_in, const int32_t *vals_in, void *keys_out, int32_t *vals_out,
                               int64_t n, int key_bits, void *workspace, size_t workspace_bytes, hipStream_t stream);

/* Status of the last spira_hip_radix_sort_pairs that used `workspace` (same
 * n and key_bits): waits for `stream` and returns an error if a tile's
 * look-back wait ran out of its spin bound, in which case that sort's output
 * is incomplete.  Tiles take tickets in dispatch order and wait only on
 * earlier tickets, so this is not expected to happen.  (No reference
 * counterpart: CUB's sort has no bounded waits.) */
int spira_hip_radix_sort_status(const void *workspace, int64_t n, int key_bits, hipStream_t stream);

/* Workspace bytes for spira_hip_downsample, _plan and _execute. */
int spira_hip_downsample_workspace(int64_t n, int key_bits, size_t *bytes);

/* out = sorted unique (keys & stride mask); *d_count (device) = number of
 * unique keys.  Strides must be powers of two.  Blocks once on `stream` to
 * read the plan (below); the count stays on the device (reference:
 * cuda_downsample, torch/cuda_arg_sort_coordinates.cu:68-105; SortUnique
 * arg_sort_coodrinates.cu:139-192). */
int spira_hip_downsample(const void *keys, int64_t n, int key_bits, int sx, int sy, int sz, void *out_keys,
                         uint32_t *d_count, void *workspace, size_t workspace_bytes, hipStream_t stream);

/* The two halves of spira_hip_downsample, so that a caller downsampling one
 * key set to several strides reads every plan with one host synchronisation
 * (reference: cuda_streamed_output_generate, torch/cuda_arg_sort_coordinates.cu:107-200).
 * _plan (n > 0) writes the record below to device memory and fills the
 * workspace's segment tables; _execute takes a host copy of that record and
 * the same workspace, untouched in between.  Sorted keys whose runs of equal
 * masked x hold at most 32768 keys take the segmented path; any other input
 * takes the general sort + unique path.  Same result either way. */
typedef struct spira_hip_downsample_plan {
  uint32_t unsorted;     /* some key is smaller than its predecessor          */
  uint32_t num_segments; /* runs of equal masked x                            */
  uint32_t max_segment;  /* keys in the longest run                           */
  uint32_t reserved;
  uint64_t varying;      /* OR over all keys of (masked key ^ first masked key) */
} spira_hip_downsample_plan_t;

int spira_hip_downsample_plan(const void *keys, int64_t n, int key_bits, int sx, int sy, int sz,
                              spira_hip_downsample_plan_t *plan, void *workspace, size_t workspace_bytes,
                              hipStream_t stream);
int spira_hip_downsample_execute(const void *keys, int64_t n, int key_bits, int sx, int sy, int sz,
                                 const spira_hip_downsample_plan_t *plan, void *out_keys, uint32_t *d_count,
                                 void *workspace, size_t workspace_bytes, hipStream_t stream);

/* Workspace bytes for spira_hip_downsample_chain. */
int spira_hip_downsample_chain_workspace(int64_t n, int key_bits, size_t *bytes);

/* Downsample one key set to a chain of strides without reading anything back:
 * level l (strides[3l .. 3l+2]) is sorted unique (keys & stride mask), written
 * to out_keys[l] (capacity n each), its count to d_counts[l] (device).  Each
 * stride must be a power of two and a multiple of the previous level's (the
 * first of 1), with (x ratio) * (y ratio) at most 16.  The keys must be sorted ascending (as
 * flatten_sort leaves them); *d_unsorted (device, zeroed by the caller) is
 * set to 1 when they are not, in which case the outputs are undefined and
 * the caller takes spira_hip_downsample per stride instead.  Same results as
 * spira_hip_downsample per stride.  (reference: cuda_streamed_output_generate,
 * torch/cuda_arg_sort_coordinates.cu:107-200, which masks, sorts and uniques
 * the full key set once per stride.) */
int spira_hip_downsample_chain(const void *keys, int64_t n, int key_bits, int levels, const int32_t *strides,
                               void *const *out_keys, uint32_t *d_counts, uint32_t *d_unsorted, void *workspace,
                               size_t workspace_bytes, hipStream_t stream);

/* ----------------------------------------------------------- kernel maps */

#define SPIRA_KMAP_OS 0     /* [Tp, K] int32, column iz*O + o (z-major)            */
#define SPIRA_KMAP_WS 1     /* [K, Tp] int32, row o*kz + iz (canonical)             */
#define SPIRA_KMAP_HYBRID 2 /* [K, Tp] int32, row row_perm[o*kz + iz]               */
#define SPIRA_KMAP_NOZ 3    /* [Tp, K] int32, canonical columns, no z-scan          */

/* Kernel-map search of sorted unique `sources` for every target and kernel
 * offset; Tp = round_up(num_targets, 128), O = kx*ky, K = O*kz.  row_perm is a
 * HOST array of K entries (hybrid layout only, else NULL).  tile_counts
 * (nullable, [K, Tp/64], WS / HYBRID layouts) receives the number of valid
 * entries of every (row, 64-target tile) for spira_hip_kmap_scan.
 * (reference: kernels BinarySearch_kz_{ostationary,wstationary,hybrid} and
 * BinarySearch_no_z_ostationary, cuda/kernels/query_sorted.cuh:8-297, launched
 * by cuda/functions/query_sorted_index.cu:12-143, 912-937; offsets from
 * torch/cuda_sparse_convolution_mapping.cu:10-50, 114-157). */
int spira_hip_kmap_search(const void *sources, int64_t num_sources, const void *targets, int64_t num_targets,
                          int key_bits, int kx, int ky, int kz, int sx, int sy, int sz, int layout,
                          const int32_t *row_perm, int32_t *kernel_map, int32_t *tile_counts, hipStream_t stream);

/* One output-stationary search (layout SPIRA_KMAP_OS, no row permutation, no
 * tile counts) of a batch. */
typedef struct {
  const void *sources;
  int64_t num_sources;
  const void *targets;
  int64_t num_targets;
  int kx, ky, kz, sx, sy, sz;
  int32_t *kernel_map; /* [round_up(num_targets, 128), kx*ky*kz] */
} spira_hip_kmap_job_t;

/* The n searches of `jobs` (keys of key_bits bits), each exactly as
 * spira_hip_kmap_search with layout SPIRA_KMAP_OS: maps of one kernel shape
 * (2x2x2, 3x3x3 or 5x5x5) share a launch, so that the searches of a network's maps
 * overlap; other shapes run one launch each.  (Replaces the per-layer
 * BinarySearch_kz_ostationary launches of BinarySearchStreamed<CT>,
 * torch/cuda_sparse_convolution_mapping.cu:894-1645.) */
int spira_hip_kmap_search_batch(int n, const spira_hip_kmap_job_t *jobs, int key_bits, hipStream_t stream);

/* Workspace bytes for spira_hip_kmap_scan over num_counts tile counts. */
int spira_hip_kmap_scan_workspace(int64_t num_counts, size_t *bytes);

/* Exclusive scan of `rows` x `ntiles` tile counts (row-major) into
 * tile_offsets, plus per-row totals nbsizes [rows], their exclusive scan
 * naddrs [rows+1] and the scan of the totals rounded up to `quantum`,
 * qnaddrs [rows+1]; sizes [2] = {total, quantised total}.  naddrs, qnaddrs and
 * sizes may be NULL.  (reference: cub ReduceByKey / DeviceSelect sizing and
 * exclusive_scan_for_kernel(_quantified), cuda/functions/query_sorted_index.cu:146-209,
 * cuda/kernels/quantifier_wstat.cuh:8-66). */
int spira_hip_kmap_scan(const int32_t *tile_counts, int rows, int64_t ntiles, int quantum, int32_t *tile_offsets,
                        int32_t *nbsizes, int32_t *naddrs, int32_t *qnaddrs, int32_t *sizes, void *workspace,
                        size_t workspace_bytes, hipStream_t stream);

/* Stable compaction of rows [row0, row0+rows) of a [*, Tp] map into
 * in_idx[p] = source, out_idx[p] = target in (row, target) order, using the
 * tile offsets of spira_hip_kmap_scan (reference: cub::DeviceSelect::If with
 * GetEntryPair, cuda/functions/query_sorted_index.cu:170-188, plus the
 * narrow/transpose to nbmaps [2, P], torch/cuda_sparse_convolution_mapping.cu:361-364). */
int spira_hip_kmap_emit_pairs(const int32_t *kernel_map, int64_t aligned_targets, int row0, int rows,
                              const int32_t *tile_offsets, int32_t *in_idx, int32_t *out_idx, hipStream_t stream);

/* Gather / scatter masks [mask_rows, S] and [mask_rows, T]: -1, or the rank
 * of the entry within its row; `half` also fills the mirrored rows
 * mask_rows-1-r with sources and targets swapped (reference:
 * GenerateMasksFromKernelMap(_Half), cuda/kernels/generate_masks_from_kernel_map.cuh:10-62,
 * launched by cuda/functions/query_sorted_index.cu:424-495, 703-776). */
int spira_hip_kmap_emit_masks(const int32_t *kernel_map, int64_t num_sources, int64_t num_targets,
                              int64_t aligned_targets, int row0, int rows, int mask_rows, int half,
                              const int32_t *tile_offsets, int32_t *source_masks, int32_t *target_masks,
                              hipStream_t stream);

/* Inverse of an output-stationary map for transposed layers:
 * out [aligned_sources, K] = -1 except out[s, k] = t where map[t, k] = s
 * (reference: cuda_convert_transposed_os, torch/cuda_sparse_convolution_mapping.cu:1809-1830;
 * kernel Convert_out_in_map_kernel, cuda/kernels/convert_transposed_os.cuh:7-16). */
int spira_hip_convert_transposed_os(const int32_t *out_in_map, int64_t aligned_targets, int num_offsets,
                                    int64_t aligned_sources, int32_t *out, hipStream_t stream);

/* spira_hip_convert_transposed_os for a map whose entries partition the
 * sources [0, num_sources): every source in exactly one entry, as in a
 * down-sampling map whose kernel equals its stride (the networks' k = 2,
 * stride-2 maps).  One pass writes whole rows: no fill, then scatter.  Any
 * other map gives wrong rows here; take spira_hip_convert_transposed_os.
 * (No counterpart in the reference: a special case of
 * cuda_convert_transposed_os, torch/cuda_sparse_convolution_mapping.cu:1809-1830.) */
int spira_hip_convert_transposed_os_partition(const int32_t *out_in_map, int64_t aligned_targets, int num_offsets,
                                              int64_t num_sources, int64_t aligned_sources, int32_t *out,
                                              hipStream_t stream);

/* Workspace bytes for spira_hip_convert_transposed_os_partition_order. */
int spira_hip_convert_transposed_os_partition_order_workspace(int64_t num_coarse, int num_offsets, size_t *bytes);

/* spira_hip_convert_transposed_os_partition (out [aligned_sources, K]), and
 * with it, without a sort, the inverse's row order as spira_hip_kmap_row_order
 * gives it: order [num_sources], ordered_map [num_sources, K] and
 * group_masks [ceil(num_sources / 128) * 2].  The inverse has one valid entry
 * per row, so that order is the rows grouped by column in source order.
 * out_in_map holds num_coarse rows; K <= 8 and K * ceil(num_coarse / 256) <=
 * 16384.  If the valid entries are fewer than num_sources (some source lies
 * in no entry), out is still the exact inverse (such rows all -1), order is
 * the identity, ordered_map equals out and every group mask holds all K
 * columns.  (No counterpart in the reference: the row order is this
 * library's own.) */
int spira_hip_convert_transposed_os_partition_order(const int32_t *out_in_map, int64_t num_coarse, int num_offsets,
                                                    int64_t num_sources, int64_t aligned_sources, int32_t *out,
                                                    int32_t *order, int32_t *ordered_map, uint64_t *group_masks,
                                                    void *workspace, size_t workspace_bytes, hipStream_t stream);

/* Workspace bytes for spira_hip_kmap_row_order. */
int spira_hip_kmap_row_order_workspace(int64_t num_targets, size_t *bytes);

/* order = the targets of an output-stationary map [>= num_targets, K] sorted
 * (stably) by neighbour count, most neighbours first, then by the bitmask of
 * their valid columns, so that rows with the same neighbour pattern are
 * processed together and the longest blocks start first; group_masks
 * (nullable, needs K <= 128, [ceil(num_targets / 128), 2]) receives for each
 * group of 128 consecutive ordered rows the 128-bit union of their valid
 * columns (word 0: columns 0..63, word 1: 64..127), and ordered_map
 * (nullable, [num_targets, K]) the map rows in that order.  (No reference
 * counterpart: the reference's output-stationary kernels walk targets in
 * index order, cuda/kernels/output_stat.cuh:20-1031.) */
int spira_hip_kmap_row_order(const int32_t *out_in_map, int64_t num_targets, int num_offsets, int32_t *order,
                             uint64_t *group_masks, int32_t *ordered_map, void *workspace, size_t workspace_bytes,
                             hipStream_t stream);

/* One row-order job of spira_hip_kmap_row_order_batch: the arguments of
 * spira_hip_kmap_row_order for one map (group_masks required). */
typedef struct {
  const int32_t *out_in_map;
  int64_t num_targets;
  int num_offsets;
  int32_t *order;
  uint64_t *group_masks;
  int32_t *ordered_map;
} spira_hip_row_order_job_t;

/* Workspace bytes for spira_hip_kmap_row_order_batch. */
int spira_hip_kmap_row_order_batch_workspace(int n, const spira_hip_row_order_job_t *jobs, size_t *bytes);

/* spira_hip_kmap_row_order for 1 to 16 maps of at most 27 offsets in one
 * chain of launches: the maps' rows are concatenated and sorted together
 * (each key prefixed with its map's index), then the group unions, the group
 * orders and the ordered rows of all maps run as one launch each.  Every
 * map's outputs equal spira_hip_kmap_row_order's.  (No reference
 * counterpart: the row order is this library's own.) */
int spira_hip_kmap_row_order_batch(int n, const spira_hip_row_order_job_t *jobs, void *workspace,
                                   size_t workspace_bytes, hipStream_t stream);

/* Workspace bytes for spira_hip_voxelize. */
int spira_hip_voxelize_workspace(int64_t num_points, size_t *bytes);

/* Voxelization front-end: coords = floor(points / voxel) in float64 (points
 * [num_points, 3] float32, or float64 with points_f64), then the first point
 * of every value of x*73856093 ^ y*19349663 ^ z*83492791 (the coordinates
 * cast to uint64; distinct voxels with colliding hashes collapse to the
 * first), sorted lexicographically by (x, y, z).  The *count (device) first
 * rows of coords [num_points, 3] int32 are the result; the count is written
 * on the stream (no host synchronisation).  Voxels at x = y = z = INT32_MAX
 * are not supported (the sentinel).  (reference: sparse_quantize and
 * ravel_hash, datasets/helpers.py:8-30.) */
int spira_hip_voxelize(const void *points, int64_t num_points, int points_f64, double vx, double vy, double vz,
                       int32_t *coords, uint32_t *count, void *workspace, size_t workspace_bytes,
                       hipStream_t stream);

/* ptr[0..n) = value (reference: the cudaMemsetAsync(-1) mask initialisation,
 * cuda/functions/query_sorted_index.cu:475-477). */
int spira_hip_fill_i32(int32_t *ptr, int64_t n, int32_t value, hipStream_t stream);

/* -------------------------------------------------------------- features */

#define SPIRA_F16 0 /* feature / weight storage dtype: IEEE half */
#define SPIRA_F32 1 /* feature / weight storage dtype: float    */

#define SPIRA_OUT_STORE 0     /* write the output in the storage dtype */
#define SPIRA_OUT_STORE_F32 1 /* write an fp32 buffer                  */
#define SPIRA_OUT_ADD_F32 2   /* add into an fp32 buffer               */

/* Bytes of the prepared (MFMA-ready) copy of weights [K, c_in, c_out]; 0 when
 * the dtype runs without one (fp32). */
int spira_hip_prepared_weights_bytes(int num_offsets, int c_in, int c_out, int dtype, size_t *bytes);

/* Prepare weights [K, c_in, c_out] for the fp16 MFMA kernels: transposed to
 * [K, c_out, c_in] and zero-padded to 32 output / 16 input channels.  A
 * prepared copy stays valid until the weights change.  (No reference
 * counterpart: the reference reads row-major weights in every kernel.) */
int spira_hip_prepare_weights(const void *weights, int num_offsets, int c_in, int c_out, int dtype, void *prepared,
                              hipStream_t stream);

/* Launch choices of the fp16 output-stationary kernel (spira_hip_conv_os);
 * a field left 0 is the library's own choice, so a zeroed struct (or a null
 * pointer) is the default schedule.  They change the schedule, never the
 * result:
 *   col_tile       output channels per column tile: 32, 64, 96 or 128;
 *   step_channels  input channels per pipeline step: 32, 64 or 128;
 *   offset_splits  blocks a row tile's kernel offsets are split over (fp32
 *                  partial sums in the workspace + a finalize pass);
 *   offset_pack    kernel offsets per step for 16-, 32- and 64-channel
 *                  inputs of kernels above 27 offsets: 1 (none), 2 or 4;
 *   block_order    1: the blocks that the hardware sends to one XCD (one
 *                  of 8 L2 slices) take one contiguous range of row tiles,
 *                  so that each L2 serves a slab of the map; 2, 3, 4: runs
 *                  of 4, 8, 16 consecutive blocks per XCD, dealt to the
 *                  XCDs in turn (neighbouring row tiles share an L2, every
 *                  XCD gets its share of the long blocks that a row-ordered
 *                  map puts first); 0 (default): row tiles in dispatch
 *                  order.
 * (No reference counterpart: these are the selector's CDNA4 parameters; the
 * reference selector sweeps gather / scatter tile sizes instead,
 * source/spira/nn/conv.py:217-307.) */
typedef struct {
  int col_tile;
  int step_channels;
  int offset_splits;
  int offset_pack;
  int block_order;
  int row_walk; /* 1: each target walks its own valid offsets on the vector ALU (fp16,
                   c_in <= 16, no row order or concatenation, storage-dtype output;
                   otherwise ignored): for few channels and large, sparse kernels */
  int balance_offsets; /* > 0: with a row order (group masks), a row tile with more
                          valid offsets than this is split over ceil(valid / this)
                          blocks (at most 8), whose fp32 partial tiles a second pass
                          sums in a fixed order (storage-dtype output, no offset
                          splits or packing): the longest tiles of a row-ordered map
                          no longer set the launch's length; -1: off; 0: the
                          library's choice */
  int blocks_per_cu; /* 1 .. 8: at most this many resident blocks per CU (dynamic
                        LDS reserves the rest), so that a small grid spreads over
                        all CUs; -1: no cap; 0: the library's choice (with a row
                        order: the grid's blocks per CU, rounded down, at least 1) */
} spira_hip_os_tuning_t;

/* Workspace bytes of spira_hip_conv_os: an fp32 [num_targets, c_out]
 * partial-sum buffer when a small layer (fewer row blocks than CUs) splits
 * its offsets over blocks, or, under work balance (balance_offsets), a work
 * list and fp32 partial tiles.  The workspace must be zero-filled before its
 * first use; every call leaves it zero-filled, so a caller keeps one buffer
 * per stream (calls that overlap on one buffer race). */
int spira_hip_conv_os_workspace(int64_t num_targets, int num_offsets, int c_in, int c_out, int dtype, int out_mode,
                                const spira_hip_os_tuning_t *tuning, size_t *bytes);

/* The launch spira_hip_conv_os would make for a layer (c_in2 > 0: the
 * concatenated form; has_map 0: the identity map) under `tuning`: plan[0..5]
 * = column tile (output channels), step channels, offset splits, kernel
 * offsets per step, grid x, grid y.  Runs on the host only.  (No reference
 * counterpart: it lets a caller or a test see what a tuning changes.)  plan[6]
 * = block order. */
int spira_hip_conv_os_plan(int64_t num_targets, int num_offsets, int c_in, int c_in2, int c_out, int has_map,
                           int out_mode, const spira_hip_os_tuning_t *tuning, int32_t *plan);

/* Output-stationary implicit GEMM: targets[t] = sum_j sources[map[t, j]] @
 * weights[j] for map entries >= 0; map is [>= num_targets, num_offsets]
 * (null: the identity map, with one offset and num_sources == num_targets,
 * i.e. a dense GEMM such as a 1x1x1 layer),
 * weights [num_offsets, c_in, c_out]; fp32 accumulation.  fp16 needs
 * `prepared` (spira_hip_prepare_weights); fp32 reads `weights`.  With
 * out_mode SPIRA_OUT_STORE an optional epilogue is applied per element:
 * v = v * scale[c] + shift[c] + residual[t, c], then max(v, 0) if relu
 * (scale / shift fp32 [c_out], residual [num_targets, c_out] in the storage
 * dtype; each nullable).  row_order (nullable, [num_targets]) is a
 * permutation of the targets (spira_hip_kmap_row_order) that the fp16 path
 * walks instead of 0..T-1, in which case out_in_map must hold the rows in
 * that order (row i = target row_order[i]); group_masks (nullable, needs
 * num_offsets <= 128) are the 128-row valid-column unions of
 * spira_hip_kmap_row_order for the rows in that order, which let a block skip
 * offsets none of its rows uses.  Both change the schedule, not the result,
 * as does `tuning` (nullable; the workspace size depends on it).
 * (reference: cuda_sparse_convolution_forward_os,
 * torch/cuda_sparse_convolution_forward.cu:448-496; SparseConvolutionForward_OS
 * cuda/functions/sparse_convolution.cu:1354-1393; kernels
 * conv_forward_cuda_setting{1,2,3}_mode0_*, cuda/kernels/output_stat.cuh:20-1031;
 * the epilogue replaces the separate bias / batch-norm / ReLU / residual ops of
 * source/spira/nn/conv.py:415-416 and scripts/models/spira/modules/blocks.py:12-84). */
int spira_hip_conv_os(int64_t num_targets, int num_offsets, const int32_t *out_in_map, const int32_t *row_order,
                      const uint64_t *group_masks, const void *sources,
                      int64_t num_sources, int c_in, const void *weights, const void *prepared, int c_out, int dtype,
                      void *targets, int out_mode, const float *scale, const float *shift, const void *residual,
                      int relu, const spira_hip_os_tuning_t *tuning, void *workspace, size_t workspace_bytes,
                      hipStream_t stream);

/* spira_hip_conv_os over the channel concatenation [sources | sources2] of two
 * fp16 feature arrays ([num_sources, c_in] and [num_sources, c_in2]; c_in a
 * multiple of 32, c_in2 of 8) without materialising it: the gather picks
 * each 32-channel block from the part that holds it.  `prepared` holds the
 * weights of the whole [K, c_in + c_in2, c_out] layer; every other argument
 * is as in spira_hip_conv_os.  (Replaces the skip-connection torch.cat in
 * front of a decoder layer, source/spira/operators.py:11-13; no counterpart
 * in the reference's C++.) */
int spira_hip_conv_os_concat(int64_t num_targets, int num_offsets, const int32_t *out_in_map,
                             const int32_t *row_order, const uint64_t *group_masks, const void *sources,
                             const void *sources2, int64_t num_sources, int c_in, int c_in2, const void *prepared,
                             int c_out, void *targets, int out_mode, const float *scale, const float *shift,
                             const void *residual, int relu, const spira_hip_os_tuning_t *tuning, void *workspace,
                             size_t workspace_bytes, hipStream_t stream);

/* Fused weight-stationary pass over a compacted pair list: for compacted row r
 * (pairs naddrs[r]..naddrs[r+1] of in_idx/out_idx) target_acc[out] +=
 * sources[in] @ weights[weight_offset + r]; with mirror_rows = Kw > 0 also
 * target_acc[in] += sources[out] @ weights[weight_offset + Kw-1-r] for every
 * r with 2r+1 != Kw.  qnaddrs / quantized_pairs are the 128-rounded scans.
 * target_acc is fp32 [num_targets, c_out], accumulated atomically.
 * (reference: cuda_sparse_convolution_forward_ws_merged,
 * torch/cuda_sparse_convolution_forward.cu:186-250; SparseConvolutionForward_WS_Merged
 * cuda/functions/sparse_convolution.cu:1267-1295; kernels fetch_on_demand_gemm_*,
 * cuda/kernels/weight_stat.cuh:33-1221). */
int spira_hip_conv_ws_fused(int64_t num_sources, int64_t num_targets, const int32_t *in_idx, const int32_t *out_idx,
                            int rows, const int32_t *naddrs, const int32_t *qnaddrs, int64_t num_pairs,
                            int64_t quantized_pairs, int weight_offset, int mirror_rows, const void *sources,
                            int c_in, const void *weights, const void *prepared, int num_weights, int c_out,
                            int dtype, float *target_acc, hipStream_t stream);

/* Gather: buffer[padded_offsets[k] + source_masks[k, s]] = sources[s] for
 * mask entries >= 0.  padded_offsets is a HOST array of num_offsets entries.
 * (reference: Gather / PaddedGatherWarpOptimized,
 * cuda/functions/sparse_convolution.cu:655-697, cuda/kernels/padded_gather_warp_optimized.cuh:11-63). */
int spira_hip_ws_gather(int64_t num_sources, int c_in, int num_offsets, int dtype, const void *sources,
                        const int32_t *source_masks, const int64_t *padded_offsets, void *buffer, hipStream_t stream);

/* Grouped GEMM: buffer_out[rows of offset k] (fp32) = buffer_in[rows of
 * offset k] @ weights[k]; rows / padded_offsets are HOST arrays; fp16 uses
 * `prepared` weights of these num_offsets offsets.
 * (reference: bucketed cublas{H,S}gemmStridedBatched, BatchedMatMul
 * cuda/helpers.cu:104-161, driven by cuda/functions/sparse_convolution.cu:1048-1117). */
int spira_hip_ws_gemm(int num_offsets, const int32_t *rows, const int64_t *padded_offsets, int c_in, int c_out,
                      int dtype, const void *buffer_in, const void *weights, const void *prepared, float *buffer_out,
                      hipStream_t stream);

/* Scatter: targets[t] = epilogue(base[t] + sum_k buffer[padded_offsets[k] + target_masks[k, t]])
 * (base: nullable fp32 [num_targets, c_out]; the epilogue of spira_hip_conv_os)
 * (reference: Scatter / PaddedScatterWarpOptimized,
 * cuda/functions/sparse_convolution.cu:699-742, cuda/kernels/padded_scatter_warp_optimized.cuh:11-63). */
int spira_hip_ws_scatter(int64_t num_targets, int c_out, int num_offsets, int dtype, const int32_t *target_masks,
                         const int64_t *padded_offsets, const float *buffer, const float *base, const float *scale,
                         const float *shift, const void *residual, int relu, void *targets, hipStream_t stream);

/* targets (storage dtype) = epilogue(acc) for an fp32 accumulation buffer
 * [num_targets, c_out], with the epilogue of spira_hip_conv_os (reference:
 * the half outputs of the weight-stationary kernels, cuda/kernels/weight_stat.cuh:914,
 * and the hybrid final add, torch/cuda_sparse_convolution_forward.cu:336). */
int spira_hip_finalize(const float *acc, int64_t num_targets, int c_out, int dtype, const float *scale,
                       const float *shift, const void *residual, int relu, void *targets, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SPIRA_HIP_H_ */
