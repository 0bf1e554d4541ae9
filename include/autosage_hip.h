/*
 * autosage_hip.h — C ABI of the MI355X (gfx950) sparse hot path.
 *
 * Every entry point takes raw device pointers, int64 sizes and a HIP stream
 * (passed as `void*`, a hipStream_t; NULL means the default stream).  The
 * library never allocates device memory: outputs and workspaces are owned by
 * the caller (the Python host layer allocates them with torch), and the
 * library keeps no per-call state.  The one exception is
 * as_spmm_csr_split_f32_static, whose workspace is a static device array.
 * All launches are asynchronous on the given stream; no entry point
 * synchronises the host.
 *
 * Return value: AS_OK (0) or a positive as_status; as_last_error() then
 * returns a thread-local message describing the failure.
 *
 * Data layout (all row-major, contiguous):
 *   crow  int64[n + 1]   CSR row pointer, crow[0] == 0, crow[n] == nnz
 *   col   int64[nnz]     column of each nonzero, 0 <= col < n (square graph)
 *   val   float[nnz]     optional per-nonzero weight (NULL = unweighted)
 *   x     float[n, f]    dense features; y float[n, f] output
 *
 * Each declaration names the reference interface it replaces
 * (paths relative to the AutoSAGE reference tree).
 */
#ifndef AUTOSAGE_HIP_H
#define AUTOSAGE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AS_ABI_VERSION 9

typedef enum as_status {
  AS_OK = 0,
  AS_ERR_INVALID_ARGUMENT = 1,
  AS_ERR_LAUNCH = 2,
  AS_ERR_UNSUPPORTED = 3,
  AS_ERR_WORKSPACE = 4
} as_status;

/* Element types of the entry points that take a dtype (AS_DTYPE_F32 only
 * where stated). */
enum {
  AS_DTYPE_F32 = 0,
  AS_DTYPE_BF16 = 1,
  AS_DTYPE_F16 = 2
};

/* Hub-row strategy for as_spmm_csr_split_f32 (no reference counterpart; the
 * reference always reassociates, csrc/spmm_hub.cu:40-47,81-90). */
enum {
  AS_HUB_EXACT = 0,   /* wave per hub row, edge order preserved: bit-exact   */
  AS_HUB_SPLIT64 = 1  /* waves split the row's edges, fp64 partials reduced
                         in LDS in wave order: deterministic, reassociated   */
};

/* Thread-local text of the last error (empty string when none). */
const char* as_last_error(void);

/* AS_ABI_VERSION of the loaded library. */
int as_abi_version(void);

/* Y = A·X over all rows.  Replaces autosage::spmm_csr_cuda
 * (csrc/spmm_csr_vec4.cu:97-176) behind the op
 * `spmm_csr(Tensor crow, Tensor col, Tensor? val, Tensor x) -> Tensor`
 * (csrc/spmm_binding.cpp:66).  `vec4` != 0 allows float4 lanes (the
 * reference's AUTOSAGE_VEC4 switch, csrc/spmm_csr_vec4.cu:135-148).
 * Per output element the sum runs in CSR edge order with fmaf, so the result
 * is bit-identical to the sequential CPU CSR product. */
int as_spmm_csr_f32(const int64_t* crow, const int64_t* col, const float* val,
                    const float* x, float* y, int64_t n, int64_t nnz,
                    int64_t f, int vec4, void* stream);

/* Bytes of workspace as_bin_rows_by_degree needs for n rows. */
size_t as_bin_workspace_bytes(int64_t n);

/* Degree binning of csrc/launcher_spmm.cu:49-59: rows with
 * crow[r+1]-crow[r] >= threshold are heavy.  Writes order[0..H) = heavy rows
 * ascending and order[H..n) = light rows ascending (the two at::nonzero lists
 * concatenated), counts[0] = H, counts[1] = n - H.  threshold must be > 0. */
int as_bin_rows_by_degree(const int64_t* crow, int64_t n, int64_t threshold,
                          int32_t* order, int32_t* counts, void* workspace,
                          size_t workspace_bytes, void* stream);

/* Bytes of workspace as_spmm_csr_split_f32 needs for n rows. */
size_t as_spmm_split_workspace_bytes(int64_t n);

/* Degree-split SpMM.  Replaces autosage::spmm_csr_split_cuda
 * (csrc/launcher_spmm.cu:22-72) behind the op
 * `spmm_csr_split(Tensor crow, Tensor col, Tensor? val, Tensor x,
 *  int feature_tile, int warps_per_block, int hub_threshold) -> Tensor`
 * (csrc/spmm_binding.cpp:67-69, argument checks :49-52).
 * feature_tile in {64,128}: features per pass of the light-row kernel;
 * waves_per_block in {2,4,8}: waves per workgroup of the hub kernel;
 * hub_threshold > 0: rows with degree >= it are hub rows;
 * hub_mode: AS_HUB_EXACT or AS_HUB_SPLIT64. */
int as_spmm_csr_split_f32(const int64_t* crow, const int64_t* col,
                          const float* val, const float* x, float* y,
                          int64_t n, int64_t nnz, int64_t f, int feature_tile,
                          int waves_per_block, int64_t hub_threshold, int vec4,
                          int hub_mode, void* workspace, size_t workspace_bytes,
                          void* stream);

/* Feature-sliced exact SpMM.  Replaces the same ops as as_spmm_csr_f32 and
 * as_spmm_csr_split_f32 (autosage::spmm_csr_cuda, csrc/spmm_csr_vec4.cu:97-176;
 * autosage::spmm_csr_split_cuda, csrc/launcher_spmm.cu:22-72) with the same
 * bits: per output element one fp32 accumulator updated in CSR edge order
 * (fmaf with a weight, acc + x without), the chain of the sequential CPU CSR
 * product (autosage/ops.py:124-143, csrc/spmm_csr_vec4.cu:42-50).  The
 * features are cut into 32-wide slices, one XCD per slice (or XCDs sharing
 * one), so each XCD's L2 caches one slice of X.  An n × n_cols CSR
 * (n_cols = N for a square graph; x has n_cols rows, y has n rows).
 *
 * Plan: built once per graph (crow, col unmodified since), any X, F and
 * weights.  Holds the rows sorted by degree (longest first, stable), the
 * columns as int32, and for each of `phases` (1 to 8) column phases one
 * 16-byte task per row: the row's edges whose column lies in the phase's
 * equal share of [0, n_cols) (found by a lower bound over the row's
 * columns).  The product runs one launch per phase, each continuing the
 * rows' fp32 chains in Y, so every phase count gives the same bits; with
 * columns ascending in every row each launch gathers from a 1/phases window
 * of X (for other column orders the cut is arbitrary, the bits the same).  int32 flags at byte 0 of the plan: bit 0 = a column
 * outside [0, n_cols) (its edges read row 0 of X instead), bit 1 = a row of
 * 2^31 or more edges; a plan with flags set gives wrong results and should
 * be refused by the caller.  The build needs a scratch workspace of
 * as_spmm_fslice_plan_workspace_bytes(n) bytes (free once the build has run
 * on the stream); *plan_tag receives the value the SpMM call checks.  No
 * reference counterpart: the reference bins rows on every call
 * (csrc/launcher_spmm.cu:49-59). */
size_t as_spmm_fslice_plan_bytes(int64_t n, int64_t nnz, int64_t phases);
size_t as_spmm_fslice_plan_workspace_bytes(int64_t n);
int as_spmm_fslice_plan(const int64_t* crow, const int64_t* col, int64_t n,
                        int64_t n_cols, int64_t nnz, int64_t phases,
                        void* plan, size_t plan_bytes, void* workspace,
                        size_t workspace_bytes, int64_t* plan_tag,
                        void* stream);

/* Workspace of as_spmm_csr_fslice_f32: the slice-major copy of X
 * (ceil(F / 32) · n_cols · 128 bytes). */
size_t as_spmm_fslice_workspace_bytes(int64_t n_cols, int64_t f);

/* Y = A·X with the plan of as_spmm_fslice_plan; val may be NULL.  Any F and
 * alignment (float4 lanes when F % 4 == 0 and x, y are 16-byte aligned).
 * A wrong plan_tag (it carries the phase count) or a plan smaller than
 * as_spmm_fslice_plan_bytes(n, nnz, phases) returns AS_ERR_INVALID_ARGUMENT; a plan of
 * another graph is not detected
 * (the caller keys plans by graph). */
int as_spmm_csr_fslice_f32(const int64_t* crow, const float* val,
                           const float* x, float* y, int64_t n, int64_t n_cols,
                           int64_t nnz, int64_t f, const void* plan,
                           size_t plan_bytes, int64_t plan_tag,
                           void* workspace, size_t workspace_bytes,
                           void* stream);

/* The two steps of as_spmm_csr_fslice_f32 apart: the slice-major copy of X
 * into `xs` (as_spmm_fslice_workspace_bytes(n_cols, f) bytes), then the
 * product from it (one launch per column phase of the plan).  A caller that multiplies one X by several graphs, or
 * times the kernels one by one, copies X once.  Same checks and bits. */
int as_spmm_fslice_relayout_f32(const float* x, int64_t n_cols, int64_t f,
                                void* xs, size_t xs_bytes, void* stream);
int as_spmm_csr_fslice_sliced_f32(const int64_t* crow, const float* val,
                                  const void* xs, size_t xs_bytes, float* y,
                                  int64_t n, int64_t n_cols, int64_t nnz,
                                  int64_t f, const void* plan,
                                  size_t plan_bytes, int64_t plan_tag,
                                  void* stream);

/* Largest row count of as_spmm_csr_split_f32_static. */
#define AS_STATIC_MAX_ROWS (1 << 22)

/* The degree-split SpMM of as_spmm_csr_split_f32 (same arguments, kernels
 * and bits) without a workspace argument and without allocating: the row
 * order and binning tables live in a static device array of about 18 MiB
 * that every GPU the library runs on keeps until the process ends.  No
 * counterpart in the reference; for callers that cannot allocate device
 * memory (HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  n <= AS_STATIC_MAX_ROWS, else AS_ERR_WORKSPACE.  The stream
 * must belong to the current device.  All calls on one GPU share that GPU's
 * array: calls that overlap on one GPU (other streams, other host threads)
 * race and must be ordered by the caller. */
int as_spmm_csr_split_f32_static(const int64_t* crow, const int64_t* col,
                                 const float* val, const float* x, float* y,
                                 int64_t n, int64_t nnz, int64_t f,
                                 int feature_tile, int waves_per_block,
                                 int64_t hub_threshold, int vec4,
                                 int hub_mode, void* stream);

/* Preferred bytes of workspace for as_spmm_csr_colslice_f32: slice points,
 * row order and two partial buffers of a quarter of the rows each. */
size_t as_spmm_colslice_workspace_bytes(int64_t n, int64_t f);

/* Column-sliced SpMM, an alternative schedule for the same product as
 * as_spmm_csr_f32 (no reference counterpart; it serves the op
 * `spmm_csr(...)`'s callers through the scheduler, autosage/_auto.py:266-441).
 * Precondition: columns ascend (non-strictly) within every row.  The column
 * space is cut into 8 ranges, one per XCD, so that each XCD's L2 caches only
 * its eighth of X; per-slice partials are accumulated in fp64 and added in
 * slice order, then rounded once (rows shorter than 128 are summed whole in
 * fp64): deterministic, within about one fp32 rounding of the exact sum, not
 * bit-identical to the sequential product.
 * The rows run in chunks, the partial reduction of one chunk beside the
 * slice work of the next.  The workspace (256-byte aligned) holds n·28 B of
 * slice points, the row order and two partial buffers of c·f·64 B for
 * chunks of c rows; any size down to c = 1 works, in more chunks.
 * sliced_rows: the number of rows of degree >= as_spmm_colslice_min_degree(1),
 * if the caller knows it (it is fixed per graph), else -1.  It only sizes the
 * launches (too small: waves loop over several rows; too large: idle
 * waves); the result is the same for any value. */
int as_spmm_csr_colslice_f32(const int64_t* crow, const int64_t* col,
                             const float* val, const float* x, float* y,
                             int64_t n, int64_t nnz, int64_t f,
                             void* workspace, size_t workspace_bytes,
                             int64_t sliced_rows, void* stream);

/* Degree from which rows are sliced, for F features of type dtype
 * (AS_DTYPE_*): with column slices (column_slices != 0) 256 for fp32 with
 * F <= 64, 128 for wider fp32 rows and 512 for bf16 / fp16; with edge slices
 * 1024. */
int64_t as_spmm_colslice_min_degree(int column_slices, int64_t f, int dtype);

/* Bytes of a column-sliced plan for n rows (n·28 B of slice points and row
 * order, plus the binning tables). */
size_t as_spmm_colslice_plan_bytes(int64_t n);

/* Builds the per-graph part of the column-sliced SpMM (as_spmm_csr_colslice_f32,
 * as_spmm_csr_rounded_16) into `plan` (256-byte aligned): the slice points
 * of every row of slicing degree and the degree-binned row order.  No
 * reference counterpart: the reference bins the rows on every call
 * (csrc/launcher_spmm.cu:49-59, at::nonzero); a plan is built once per graph
 * and serves every later call with the same F, dtype and slicing, whatever
 * X and the weights.  *plan_tag receives the settings the plan was built
 * for (slicing degree, light buckets), checked by the planned call.
 * dtype AS_DTYPE_F32 (column_slices != 0 only), AS_DTYPE_BF16 or
 * AS_DTYPE_F16; the columns of the graph ascend within rows for column
 * slices.  Asynchronous on `stream`. */
int as_spmm_colslice_plan(const int64_t* crow, const int64_t* col, int64_t n,
                          int64_t nnz, int64_t f, int dtype, int column_slices,
                          void* plan, size_t plan_bytes, int64_t* plan_tag,
                          void* stream);

/* Preferred workspace bytes of as_spmm_csr_colslice_planned: the two partial
 * buffers only, of min(sliced_rows, rows of a chunk) partial rows each for
 * 16-bit elements, and for fp32 with F % 4 == 0 on graphs of more than 2^24
 * edges; of a chunk's rows otherwise (fp32 chunks are cut to buffers that
 * cannot hold their sliced rows there, see below).  sliced_rows = the most
 * rows of slicing degree that one row block of the plan holds
 * (as_spmm_colslice_row_blocks), or -1 for a chunk's rows.  The bits do not
 * depend on the workspace: a sliced row that finds no partial row is summed
 * by one wavefront with the same operations in the same order (16-bit
 * elements: whole, by their order-free rule; fp32 cooperative hub rows and
 * narrow lanes: the chunk is cut instead). */
size_t as_spmm_colslice_planned_workspace_bytes(int64_t n, int64_t nnz,
                                                int64_t f, int dtype,
                                                int64_t sliced_rows);

/* Row blocks of a column-sliced plan for n rows of type dtype: returns their
 * count B and writes their first rows begins[0..B] (begins[B] = n) when
 * capacity > B.  Host only. */
int64_t as_spmm_colslice_row_blocks(int64_t n, int dtype, int64_t* begins,
                                    int64_t capacity);

/* as_spmm_csr_colslice_f32 (dtype AS_DTYPE_F32, column_slices != 0) or
 * as_spmm_csr_rounded_16 (AS_DTYPE_BF16 / AS_DTYPE_F16) with the slice
 * points and row order read from a plan that as_spmm_colslice_plan built
 * for this graph (same crow, col, n and nnz, unmodified since) with the
 * same F, dtype and column_slices: the same bits, without the per-call
 * slice point and binning launches.  A plan_tag of other settings returns
 * AS_ERR_INVALID_ARGUMENT; a plan of another graph is not detected (the
 * caller keys plans by graph).  The workspace holds the partial buffers
 * only (any size down to two partial rows, as for the unplanned calls).
 * sliced_rows / grouped_rows: launch-sizing hints for every dtype, the
 * rows of degree >= as_spmm_colslice_min_degree(column_slices, f, dtype) and
 * of degree < as_spmm_colslice_group_degree(f, dtype), or -1; the result is
 * the same for any value. */
int as_spmm_csr_colslice_planned(const int64_t* crow, const int64_t* col,
                                 const void* val, const void* x, void* y,
                                 int64_t n, int64_t nnz, int64_t f, int dtype,
                                 int column_slices, const void* plan,
                                 size_t plan_bytes, int64_t plan_tag,
                                 void* workspace, size_t workspace_bytes,
                                 int64_t sliced_rows, int64_t grouped_rows,
                                 void* stream);

/* Row shards.  No reference counterpart: the reference runs one graph on one
 * GPU.  A graph split by rows over several GPUs gives each GPU the CSR of
 * its rows [r0, r1) (crow rebased to start at 0, the columns unchanged) and
 * the whole of X, n_cols = N rows; Y holds the shard's n = r1 - r0 rows.
 * These two entries are as_spmm_colslice_plan and
 * as_spmm_csr_colslice_planned for such an n × n_cols CSR: the column
 * slices cut [0, n_cols), so a shard's slice points, and with them its
 * rows' sums, are those of the same rows in the whole graph (a shard of at
 * most 2^24 edges adds its hub rows' wave sums through LDS, which can move
 * the fp64 sum of a row by less than 2^-52 of its largest partial).  The
 * square entries are these with n_cols = n. */
int as_spmm_colslice_plan_rect(const int64_t* crow, const int64_t* col,
                               int64_t n, int64_t n_cols, int64_t nnz,
                               int64_t f, int dtype, int column_slices,
                               void* plan, size_t plan_bytes,
                               int64_t* plan_tag, void* stream);
int as_spmm_csr_colslice_planned_rect(const int64_t* crow, const int64_t* col,
                                      const void* val, const void* x, void* y,
                                      int64_t n, int64_t n_cols, int64_t nnz,
                                      int64_t f, int dtype, int column_slices,
                                      const void* plan, size_t plan_bytes,
                                      int64_t plan_tag, void* workspace,
                                      size_t workspace_bytes,
                                      int64_t sliced_rows,
                                      int64_t grouped_rows, void* stream);

/* SpMM with bf16 or fp16 features, weights and output (dtype
 * AS_DTYPE_BF16 / AS_DTYPE_F16; val may be NULL).  The reference has no
 * kernel for these types: its op raises for them (autosage/ops.py:156-157)
 * and its scheduler falls back to torch.sparse.mm with the weights cast to
 * the feature type (autosage/_auto.py:281-287); the CPU torch path has no
 * bf16/fp16 CSR product.  Result: every output is the fp64 sum of the exact
 * products, rounded to fp32 and then to the element type (round to nearest
 * even both times).  The fp64 sum does not depend on the order of the
 * additions when it is exact (the products' bits span at most 53 places);
 * otherwise its error is below 2^-52 of the largest partial sum, and two
 * schedules can round differently only for a sum that close to a tie.
 * Same kernels and workspace layout as as_spmm_csr_colslice_f32 (size from
 * as_spmm_rounded_16_workspace_bytes: it needs partial rows for the sliced
 * rows only).  column_slices != 0: 8 column slices
 * (columns must ascend within rows); 0: rows of degree >= 1024 are cut into
 * 8 equal runs of edges instead (any column order).  x, y and val 2-byte
 * aligned; F a multiple of 8 with 16-byte aligned x takes 16-byte lanes.
 * Short rows of degree below as_spmm_rounded_16_group_degree(f) are
 * summed several to a wavefront (a lane group each), the other rows one
 * wavefront each or sliced.
 * sliced_rows: as for as_spmm_csr_colslice_f32, with the degree
 * as_spmm_colslice_min_degree(column_slices, f, dtype); grouped_rows: the number of
 * rows of degree below as_spmm_rounded_16_group_degree(f), else -1.  Both
 * only size the launches; the result is the same for any values. */
int as_spmm_csr_rounded_16(const int64_t* crow, const int64_t* col,
                           const void* val, const void* x, void* y,
                           int64_t n, int64_t nnz, int64_t f, int dtype,
                           int column_slices, void* workspace,
                           size_t workspace_bytes, int64_t sliced_rows,
                           int64_t grouped_rows, void* stream);

/* Workspace bytes for as_spmm_csr_rounded_16: as
 * as_spmm_colslice_workspace_bytes, with partial buffers for sliced_rows rows
 * (all of a chunk's when sliced_rows < 0).  A workspace with fewer partial
 * rows than a chunk's sliced rows also works: the sliced rows past them are
 * summed whole, one wavefront each, with the same bits. */
size_t as_spmm_rounded_16_workspace_bytes(int64_t n, int64_t f, int64_t sliced_rows);

/* The product of as_spmm_csr_rounded_16 (same bits) without slicing: one
 * launch, no workspace, every row summed whole by one wavefront.  For small
 * graphs, where the sliced schedule's set-up costs more than the product;
 * any column order. */
int as_spmm_csr_rows_16(const int64_t* crow, const int64_t* col, const void* val,
                        const void* x, void* y, int64_t n, int64_t nnz, int64_t f,
                        int dtype, void* stream);

/* Degree below which as_spmm_csr_rounded_16 sums rows several to a
 * wavefront for F features (32, 64 or 128 for F <= 64, <= 128, more; 0 when
 * F is not a multiple of 8). */
int64_t as_spmm_rounded_16_group_degree(int64_t f);

/* Degree below which the column-sliced SpMM (as_spmm_csr_colslice_planned,
 * as_spmm_csr_colslice_f32, as_spmm_csr_rounded_16) sums short rows several to
 * a wavefront, for F features of type dtype (AS_DTYPE_*): 4·G for the G lanes
 * per edge, 0 when they run one per wavefront.  The count of such rows is
 * the planned call's `grouped_rows` launch-sizing hint. */
int64_t as_spmm_colslice_group_degree(int64_t f, int dtype);

/* SDDMM with bf16 or fp16 query, key and output (dtype AS_DTYPE_BF16 /
 * AS_DTYPE_F16): out[e] is the fp64 sum of the exact products
 * query[row(e), f]·key[col[e], f], rounded to fp32 and then to the element
 * type (round to nearest even both times).  The reference has no kernel for
 * these types: its op takes float32 only (csrc/sddmm_csr_op.cu:94-95) and its
 * scheduler runs the gather-dot baseline (autosage/_auto.py:575-581).  The
 * schedule is that of as_sddmm_csr_split_f32 (rows of degree >=
 * hub_threshold cut into 2048-edge chunks, waves_per_block 2, 4 or 8, the
 * workspace from as_sddmm_split_workspace_bytes); an exact fp64 sum does not
 * depend on the order of the additions, so any schedule gives the same bits.
 * query, key and out 2-byte aligned; F a multiple of 8 up to 512 with
 * 16-byte aligned query and key takes 16-byte lanes. */
int as_sddmm_csr_rounded_16(const int64_t* crow, const int64_t* col,
                            const void* query, const void* key, void* out,
                            int64_t n, int64_t nnz, int64_t f, int dtype,
                            int waves_per_block, int64_t hub_threshold,
                            void* workspace, size_t workspace_bytes,
                            void* stream);

/* Bytes of workspace as_sddmm_csr_edges_16 needs for nnz edges. */
size_t as_sddmm_edges_16_workspace_bytes(int64_t nnz);

/* The SDDMM of as_sddmm_csr_rounded_16 (the same bits) on another schedule:
 * the edges in CSR order in blocks of 64, a few blocks per wavefront,
 * whatever the row lengths, each edge's row found from crow inside the
 * wavefront; no degree split.  Same arguments as as_sddmm_csr_rounded_16
 * without the split settings.  Replaces sddmm_csr (csrc/sddmm_csr_op.cu:108-134)
 * for the 16-bit types the reference leaves to its gather-dot baseline
 * (autosage/_auto.py:575-581). */
int as_sddmm_csr_edges_16(const int64_t* crow, const int64_t* col,
                          const void* query, const void* key, void* out,
                          int64_t n, int64_t nnz, int64_t f, int dtype,
                          void* workspace, size_t workspace_bytes,
                          void* stream);

/* as_sddmm_csr_edges_16 for a row shard (no reference counterpart; see the
 * row-shard entries of the column-sliced SpMM): n rows of the shard's CSR
 * and of `query` (its rows of the whole query), `key` the whole key of
 * n_keys rows.  The square entry is this with n_keys = n. */
int as_sddmm_csr_edges_16_rect(const int64_t* crow, const int64_t* col,
                               const void* query, const void* key, void* out,
                               int64_t n, int64_t n_keys, int64_t nnz,
                               int64_t f, int dtype, void* workspace,
                               size_t workspace_bytes, void* stream);

/* Row softmax of bf16 or fp16 scores (dtype AS_DTYPE_BF16 / AS_DTYPE_F16):
 * the scores convert exactly to fp32, the softmax is computed in fp32 (rows
 * of at most 64 edges by 16-lane groups, longer rows by a wavefront with a
 * running max and sum), and each probability is rounded once to the element
 * type.  The reference computes it with torch ops in the scores' own
 * type (autosage/_auto.py:744-759). */
int as_csr_row_softmax_16(const int64_t* crow, const void* scores, void* probs,
                          int64_t n, int64_t nnz, int dtype, void* stream);

/* Backward of the row softmax (no reference counterpart: the reference
 * registers no autograd, and its torch composition, autosage/_auto.py:744-759,
 * is differentiated by torch there): given probs = softmax(scores) row by row
 * and grad = dL/dprobs, grad_scores[e] = probs[e]·(grad[e] − t) with
 * t = Σ grad·probs over the row, in fp32: lane l of a wavefront adds edges
 * l, l+64, ... of the row with fmaf, in order, then a 32/16/8/4/2/1
 * butterfly.  dtype AS_DTYPE_F32, AS_DTYPE_BF16 or AS_DTYPE_F16 (16-bit
 * values convert exactly; each result is rounded once). */
int as_csr_row_softmax_backward(const int64_t* crow, const void* probs, const void* grad,
                                void* grad_scores, int64_t n, int64_t nnz, int dtype,
                                void* stream);

/* out[e] = <query[row(e)], key[col[e]]> for every nonzero, CSR order.
 * Replaces sddmm_csr (csrc/sddmm_csr_op.cu:108-134), op schema :192.
 * The dot product uses the reference kernel's summation order
 * (32 lane-strided fma chains, then a 16/8/4/2/1 tree,
 * csrc/sddmm_csr_op.cu:12-17,39-49). */
int as_sddmm_csr_f32(const int64_t* crow, const int64_t* col,
                     const float* query, const float* key, float* out,
                     int64_t n, int64_t nnz, int64_t f, void* stream);

/* Bytes of workspace as_sddmm_csr_split_f32 needs for n rows. */
size_t as_sddmm_split_workspace_bytes(int64_t n);

/* Degree-split SDDMM.  Replaces sddmm_csr_split
 * (csrc/sddmm_csr_op.cu:136-187), op schema :193-195: rows with degree
 * < hub_threshold go to the row kernel, the rest are cut into edge chunks
 * spread over workgroups of waves_per_block waves.  Bit-identical to
 * as_sddmm_csr_f32. */
int as_sddmm_csr_split_f32(const int64_t* crow, const int64_t* col,
                           const float* query, const float* key, float* out,
                           int64_t n, int64_t nnz, int64_t f,
                           int waves_per_block, int64_t hub_threshold,
                           void* workspace, size_t workspace_bytes,
                           void* stream);

/* Row softmax over CSR values: p_e = exp(s_e - max_row) / sum_row.
 * Replaces the torch composition _csr_row_softmax (autosage/_auto.py:744-759). */
int as_csr_row_softmax_f32(const int64_t* crow, const float* scores,
                           float* probs, int64_t n, int64_t nnz, void* stream);

/* Bytes of workspace as_csr_attention_f32 needs. */
size_t as_csr_attention_workspace_bytes(int64_t n, int64_t nnz);

/* Fused out = SpMM(softmax_row(scale * SDDMM(query, key)), value).
 * Replaces csr_attention_forward (autosage/_auto.py:762-780), which runs the
 * three stages separately and has no scale (scale = 1 reproduces it).
 * Bit-identical to as_sddmm_csr_f32 -> as_csr_row_softmax_f32 ->
 * as_spmm_csr_f32 when scale is 1 or a power of two. */
int as_csr_attention_f32(const int64_t* crow, const int64_t* col,
                         const float* query, const float* key,
                         const float* value, float* out, int64_t n,
                         int64_t nnz, int64_t f_qk, int64_t f_v, float scale,
                         void* workspace, size_t workspace_bytes,
                         void* stream);

/* Preferred bytes of workspace for as_csr_attention_colslice_f32 (called
 * without a plan; with one, as_csr_attention_plan_bytes(n) less). */
size_t as_csr_attention_colslice_workspace_bytes(int64_t n, int64_t nnz,
                                                 int64_t f_v);

/* Bytes of an attention plan for n rows. */
size_t as_csr_attention_plan_bytes(int64_t n);

/* Builds the per-graph part of the column-sliced attention into `plan`
 * (256-byte aligned): the slice points of every row of degree >= 128
 * (fp32) or >= 512 (bf16 / fp16) and the degree-binned row order.  No reference counterpart (the reference
 * composes its attention from torch ops, autosage/_auto.py:762-780); a plan
 * is built once per graph and serves every later attention call on it with
 * the same element type (dtype AS_DTYPE_F32 / BF16 / F16), whatever Q, K
 * and V.  It also serves the backward's pass over the graph (same element
 * type), and the backward's pass over the transposed graph takes a plan of
 * that graph.  *plan_tag receives the settings it was built for, checked by
 * the calls.  Columns ascending within rows; asynchronous on `stream`. */
int as_csr_attention_plan(const int64_t* crow, const int64_t* col, int64_t n,
                          int64_t nnz, int dtype, void* plan,
                          size_t plan_bytes, int64_t* plan_tag, void* stream);

/* as_csr_attention_plan for a row shard (no reference counterpart): the
 * slice points cut the whole column space [0, n_cols) of the graph the
 * shard's n rows come from.  With this plan the column-sliced attention
 * entries run the shard: query and out hold its n rows, key and value the
 * whole n_cols rows.  The square entry is this with n_cols = n. */
int as_csr_attention_plan_rect(const int64_t* crow, const int64_t* col,
                               int64_t n, int64_t n_cols, int64_t nnz,
                               int dtype, void* plan, size_t plan_bytes,
                               int64_t* plan_tag, void* stream);

/* Column-sliced attention, an alternative schedule for as_csr_attention_f32
 * (no reference counterpart; chosen by csr_attention_forward,
 * autosage/_auto.py:762-780, after a full-graph timing).  Precondition:
 * columns ascend within every row; f_qk and f_v multiples of 4 in [4, 256];
 * Q, K, V, out 16-byte aligned.  Rows of degree >= 128 are cut into the 8
 * column slices (one per XCD) with an online softmax per (row, slice) and
 * fp32 partial states merged per row; shorter rows run the online softmax in
 * one wave.  Deterministic; not bit-identical to as_csr_attention_f32.
 * plan: NULL (the slice points and row order are built in the workspace in
 * every call) or a plan of as_csr_attention_plan for this graph, unmodified
 * since, with plan_tag (a tag of other settings returns
 * AS_ERR_INVALID_ARGUMENT); the same bits either way.
 * A workspace smaller than the preferred size (256-byte aligned, at least
 * the slice points and row order when plan is NULL and one row of partial
 * states) runs the sliced rows in more chunks. */
int as_csr_attention_colslice_f32(const int64_t* crow, const int64_t* col,
                                  const float* query, const float* key,
                                  const float* value, float* out, int64_t n,
                                  int64_t nnz, int64_t f_qk, int64_t f_v,
                                  float scale, const void* plan,
                                  int64_t plan_tag, void* workspace,
                                  size_t workspace_bytes, void* stream);

/* The column-sliced attention on bf16 or fp16 query, key, value and output
 * (dtype AS_DTYPE_BF16 / AS_DTYPE_F16): the kernels of
 * as_csr_attention_colslice_f32 with 16-byte lanes of 8 elements, every
 * input converted exactly to fp32, the online softmax and the partial states
 * in fp32, and each output rounded once to the element type (round to
 * nearest even).  Scores and probabilities stay in registers.  The reference
 * composes its attention for any feature type from torch ops
 * (csr_attention_forward, autosage/_auto.py:762-780), rounding the scores and
 * probabilities to the feature type; there is no 16-bit kernel to replace.
 * f_qk and f_v multiples of 8 in [8, 512]; 16-byte aligned Q, K, V and out;
 * columns ascending within every row; the workspace of
 * as_csr_attention_colslice_workspace_bytes; plan and plan_tag as for
 * as_csr_attention_colslice_f32 (a plan built for this dtype).  Rows are
 * sliced from degree 512; shorter rows run several to a wavefront. */
int as_csr_attention_colslice_16(const int64_t* crow, const int64_t* col,
                                 const void* query, const void* key,
                                 const void* value, void* out, int64_t n,
                                 int64_t nnz, int64_t f_qk, int64_t f_v,
                                 float scale, int dtype, const void* plan,
                                 int64_t plan_tag, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* Bytes of workspace for as_csr_attention_backward_f32 (dtype AS_DTYPE_F32)
 * or as_csr_attention_backward_16 (AS_DTYPE_BF16 / AS_DTYPE_F16). */
size_t as_csr_attention_backward_workspace_bytes(int64_t n, int64_t nnz,
                                                 int64_t f_qk, int64_t f_v,
                                                 int dtype);

/* Gradients of out = softmax_row(scale · SDDMM(query, key)) · value (the
 * attention of as_csr_attention_colslice_f32) in two gather passes, fp32:
 * pass 1 over the rows of A (crow, col) recomputes the scores with an online
 * maximum and sum and writes grad_q and the row log-sum-exp; pass 2 over the
 * rows of the transposed graph (crow_t, col_t: the columns of A, sources
 * ascending) writes grad_k and grad_v.  out is the forward result, grad_out
 * dL/dout.  No reference counterpart: the reference registers no autograd
 * and differentiates its torch composition (autosage/_auto.py:762-780).
 * f_qk and f_v multiples of 4 in [4, 256]; all dense tensors 16-byte aligned;
 * columns ascending within the rows of both graphs; a workspace smaller
 * than the preferred size runs the sliced rows in more chunks.
 * plan / plan_t: NULL, or fp32 plans of as_csr_attention_plan for the graph
 * and for the transposed graph with their tags (the 16-bit entry takes plans
 * of its dtype); a pass without a plan
 * builds one in the workspace (as_csr_attention_plan_bytes(n) of the
 * preferred size are that region, needed unless both plans are given). */
int as_csr_attention_backward_f32(const int64_t* crow, const int64_t* col,
                                  const int64_t* crow_t, const int64_t* col_t,
                                  const float* query, const float* key,
                                  const float* value, const float* out,
                                  const float* grad_out, float* grad_q,
                                  float* grad_k, float* grad_v, int64_t n,
                                  int64_t nnz, int64_t f_qk, int64_t f_v,
                                  float scale, const void* plan,
                                  int64_t plan_tag, const void* plan_t,
                                  int64_t plan_t_tag, void* workspace,
                                  size_t workspace_bytes, void* stream);

/* as_csr_attention_backward_f32 for bf16 / fp16 query, key, value, grad_out
 * and gradients (dtype AS_DTYPE_BF16 / AS_DTYPE_F16; the attention of
 * as_csr_attention_colslice_16).  Inputs converted exactly to fp32, every
 * sum in fp32, each gradient rounded once to the element type.  The output
 * is not an argument: pass 1 sums t_r = Σ p·dP itself (the rounded 16-bit
 * output would carry 2^-9 of relative error into it) and keeps
 * Σ w·dP·K and Σ w·K apart (dQ = scale·(Σ w·dP·K − t·Σ w·K)/l).  No
 * reference counterpart (its torch composition works in the feature type).
 * f_qk and f_v multiples of 8 in [8, 512]; plans (of this dtype, for the
 * graph and for its transpose) and workspace as for the fp32 entry, sized
 * with this dtype.  Short rows of both passes run several to a wave. */
int as_csr_attention_backward_16(const int64_t* crow, const int64_t* col,
                                 const int64_t* crow_t, const int64_t* col_t,
                                 const void* query, const void* key,
                                 const void* value, const void* grad_out,
                                 void* grad_q, void* grad_k, void* grad_v,
                                 int64_t n, int64_t nnz, int64_t f_qk,
                                 int64_t f_v, float scale, int dtype,
                                 const void* plan, int64_t plan_tag,
                                 const void* plan_t, int64_t plan_t_tag,
                                 void* workspace, size_t workspace_bytes,
                                 void* stream);

/* Bytes of workspace for the induced-sample entry points (n int32). */
size_t as_induced_sample_workspace_bytes(int64_t n);

/* Induced sub-graph of a row sample, on the device.  Replaces the torch
 * composition _induced_sample_csr (autosage/_auto.py:95-154) given its
 * sorted sample `selected` (s distinct rows).  Two calls with the same
 * workspace: _count writes new_crow[0..s] (kept edges: those whose column is
 * sampled); the caller reads new_crow[s] to size new_col/new_val; _fill
 * writes the kept edges in CSR order with columns renamed to their sample
 * index, and their values when val is given.  Bit-identical to the
 * reference's outputs. */
int as_induced_sample_count(const int64_t* crow, const int64_t* col, int64_t n,
                            const int64_t* selected, int64_t s,
                            int64_t* new_crow, void* workspace,
                            size_t workspace_bytes, void* stream);
int as_induced_sample_fill(const int64_t* crow, const int64_t* col,
                           const float* val, int64_t n,
                           const int64_t* selected, int64_t s,
                           const int64_t* new_crow, int64_t* new_col,
                           float* new_val, const void* workspace,
                           size_t workspace_bytes, void* stream);

/* Structure check of a CSR graph (no reference counterpart: the reference
 * kernels trust their inputs).  ORs into *flags (device int32, zeroed by the
 * caller): 1 = crow[0] != 0, 2 = crow decreases somewhere, 4 = crow[n] != nnz,
 * 8 = a column outside [0, n_cols); and 16 = columns descend somewhere inside
 * a row, which is valid CSR but rules out as_spmm_csr_colslice_f32.  Reads
 * nothing out of bounds. */
int as_csr_validate(const int64_t* crow, const int64_t* col, int64_t n,
                    int64_t nnz, int64_t n_cols, int32_t* flags,
                    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AUTOSAGE_HIP_H */
