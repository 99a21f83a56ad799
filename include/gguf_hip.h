/* gguf_hip.h - C ABI of the MI355X (gfx950) GGUF quantized linear path.
 *
 * A drop-in for the out-of-tree vLLM GGUF plugin's linear path: the entry points below are
 * what that plugin's Python binds for (a) dequantize(W, type, shape), (b) the load-time tile
 * repack and grouped-layer preparation, and (c) the grouped matmul op called from
 * GGUFLinearMethod.apply(layer, x, bias).  Plain C: raw device pointers, sizes and a HIP stream
 * passed as void*.  No allocation happens inside any entry point: outputs, tiles and workspace
 * are owned by the caller (torch), and every launch goes on the caller's stream.
 *
 * Status: every int-returning function returns GQK_OK (0) or a negative GQK_ERR_* code;
 * gqk_last_error() returns a thread-local message for the last failure on the calling thread.
 */
#ifndef GGUF_HIP_H
#define GGUF_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GQK_OK 0
#define GQK_ERR_TYPE (-1)  /* GGML type without a kernel (reference: NotImplementedError,
                              gguf-plugin/gluon/interface.py:78-79) */
#define GQK_ERR_SHAPE (-2) /* shape / size / alignment contract broken (reference: AssertionError,
                              gguf-plugin/gluon/tiles_grouped.py:1211-1263) */
#define GQK_ERR_FORM (-3)  /* plan does not serve this launch (M outside the plan's range) */
#define GQK_ERR_HIP (-4)   /* HIP runtime error at launch */
#define GQK_ERR_ARG (-5)   /* null pointer or bad argument */

#define GQK_FORM_GEMV 1 /* M <= 32, every type: streaming forms over (tile, k-range) rows: the in-register
                           decode GEMV up to 16 rows (small shards up to 8 rows in its slab form,
                           plan bm = 2: a row per 32-row slab over the whole k-range), the mid form
                           (g = 8) for 17..32 (small shards at 9..32 rows in its slab form, bm = 2) */
#define GQK_FORM_GEMM 2 /* M > 32: LDS-dequant bf16 MFMA GEMM (any M) */

#define GQK_CTR_BYTES 262144 /* the arrival-counter region at the start of every workspace */

#define GQK_DTYPE_F32 0
#define GQK_DTYPE_BF16 1
#define GQK_DTYPE_F16 2

/* One shard of a grouped layer: its rows sit at byte `offset` of the packed tile buffer. */
typedef struct gqk_shard {
  int32_t ggml_type;
  int32_t reserved;
  int64_t n;      /* output rows */
  int64_t offset; /* byte offset of the shard's tiles in the packed buffer */
} gqk_shard;

/* Launch plan of a grouped layer for one batch-row bucket (filled by gqk_plan). */
typedef struct gqk_plan_info {
  int32_t form;       /* GQK_FORM_GEMV or GQK_FORM_GEMM */
  int32_t m_max;      /* largest batch rows M the plan serves (GEMV: 4 * g) */
  int32_t g;          /* GEMV: groups of 4 tokens (1, 2, 4; 8 = the mid form, 17..32 rows, or its slab
                         form from 9 rows) */
  int32_t bm;         /* GEMM: tokens per tile (64, 128, 256); GEMV (g <= 2): 1 when every wave streams
                         exactly one 256-weight record (the launch takes the pipeline-free kernel),
                         2 for the slab form (a workgroup per 32-row half tile over the whole k-range,
                         one wave per pair of super-blocks, no split-K partials; with g = 8 the mid
                         form's slab) */
  int32_t split;      /* GEMV: most workgroups sharing one tile (partials summed in split order in-kernel when > 1) */
  int32_t n_desc;     /* descriptor rows (workgroups along N x K) */
  int32_t types_mask; /* the GGML type of every shard, or 0 when the shards mix types */
  int32_t nb;         /* K / 256 */
  int32_t nw;         /* GEMV: waves per workgroup (they split the workgroup's k-range) */
  int32_t ctr_bytes;  /* bytes of arrival counters at the start of the workspace: GQK_CTR_BYTES in
                         every plan, so one workspace serves every layer and every M */
  int64_t n_total;    /* output columns: sum of the shards' rows */
  int64_t workspace_bytes; /* device workspace gqk_linear needs (any M <= m_max) */
} gqk_plan_info;

/* Last error message of the calling thread ("" when none). */
const char* gqk_last_error(void);

/* Library version: major * 10000 + minor * 100 + patch. */
int gqk_version(void);

/* Host-only metadata of a GGML type: info[0..3] = weights per block, bytes per block, bytes per
 * 256 weights, number of tile planes; planes (if not NULL, 6 ints per plane) = bytes per row,
 * segments, first raw offset, segment bytes, segment stride, column width of the tile layout.  Replaces the reference's tile
 * registry TILE_TYPES (gguf-plugin/gluon/tiles.py:24-36) and gguf.GGML_QUANT_SIZES. */
int gqk_type_info(int ggml_type, int32_t* info, int32_t* planes);

/* Dequantize n rows of K weights of `ggml_type` (raw GGUF blocks, row stride in bytes) into
 * out[n, ld_out] of out_dtype (GQK_DTYPE_*): fp32 bit-exact with gguf-py's dequantizer, bf16 /
 * fp16 the round-to-nearest-even of it.  Replaces ops.ggml_dequantize(W, type, m, n, dtype)
 * (gguf-plugin/patches/gguf-prefill-dispatch.patch:42-45, gguf-plugin/gluon/tiles.py:147-149). */
int gqk_dequantize(const void* W, int64_t w_row_stride, int ggml_type, int64_t n, int64_t K, void* out,
                   int64_t ld_out, int out_dtype, void* stream);

/* Dequantize n rows of K weights straight from the tile layout (gqk_repack's output) into
 * out[n, ld_out] of out_dtype, in one pass (no raw-row temporary); the same bits as
 * gqk_dequantize of the raw rows.  Replaces dequantize_tiles / dequantize_iq3s_tiles
 * (gguf-plugin/gluon/tiles.py:141-149, gguf-plugin/gluon/iq3s_tile_dequant.py:22-63). */
int gqk_dequantize_tiles(const void* tiles, int ggml_type, int64_t n, int64_t K, void* out, int64_t ld_out,
                         int out_dtype, void* stream);

/* Bytes of the tile layout of an n x K shard (< 0: error code).  K % 256 == 0. */
int64_t gqk_tiles_bytes(int ggml_type, int64_t n, int64_t K);

/* Raw GGUF rows -> CDNA4 plane-major tiles (64-row tiles x 256-weight super-blocks, rows past n
 * zero).  Replaces repack_tiles (gguf-plugin/gluon/tiles.py:128-130). */
int gqk_repack(const void* W, int64_t w_row_stride, int ggml_type, int64_t n, int64_t K, void* tiles, void* stream);

/* Tiles -> raw GGUF rows (bit-exact inverse of gqk_repack).  Replaces unrepack_tiles
 * (gguf-plugin/gluon/tiles.py:56-67). */
int gqk_unrepack(const void* tiles, int ggml_type, int64_t n, int64_t K, void* W, int64_t w_row_stride, void* stream);

/* Host code (no launch, no allocation): the launch plan of a grouped layer (shards packed back to
 * back, all of K columns) for batch rows M: fills *info and, if desc is not NULL and
 * desc_capacity (int32 words) is enough, the descriptor table (16 int32 per row) to upload to
 * the device.  cus: compute units of the device the plan is for (256 on MI355X); 0 asks the HIP
 * runtime for the current device's count (initialising the runtime; 256 when no device is
 * visible).  target_wgs > 0 overrides the GEMV heuristic's target of resident waves (0 = eight per
 * CU), from which the waves per workgroup and the split-K factor follow.  GEMM plans (M > 32)
 * take their tile form from M and, at 129..384 rows (129..768 for K <= 8192), from the layer's
 * size against the CU count.  Replaces prepare_grouped_layer / descriptors / grouped_split_for
 * (gguf-plugin/gluon/tiles_grouped.py:237-299). */
int gqk_plan(const gqk_shard* shards, int nshards, int64_t K, int M, int target_wgs, int cus, int32_t* desc,
             int64_t desc_capacity, gqk_plan_info* info);

/* Device workspace bytes gqk_linear needs for this plan at M batch rows (0: none; < 0: error).
 * GEMV plans with split-K need info->workspace_bytes; GEMM plans need room for their stream-K
 * partial tiles, which depends on M and on the current device's CU count.  Replaces the reference's transient split-K partials (gguf-plugin/gluon/tiles_grouped.py:1233-1238). */
int64_t gqk_linear_workspace_bytes(const gqk_plan_info* info, int M);

/* Workspace bytes that serve every GEMM plan at any M on the current device (< 0: error): one
 * buffer of this size (or of a layer's GEMV workspace_bytes, if larger) serves every layer on the
 * device, as calls on one stream never overlap.  No counterpart in the reference, whose split-K
 * partials are transient torch tensors (gguf-plugin/gluon/tiles_grouped.py:1233-1238). */
int64_t gqk_workspace_bytes_max(void);

/* Measurement only, no counterpart in the reference: a plain streaming read of `bytes` (a
 * multiple of 1 KiB, at most 2 GiB) at `buf` on `grid` workgroups of `waves` (1..16) waves, each
 * wave reading one contiguous share and writing one folded word to sink[wave] (grid * waves
 * uint32 words).  Timed over a shard's packed bytes on the shard's own grid it gives the memory
 * floor that bench.py reports beside each launch. */
int gqk_read_floor(const void* buf, int64_t bytes, int grid, int waves, void* sink, void* stream);

/* y[M, ldy] (bf16) = x[M, ldx] (bf16) @ W^T (+ bias) over the grouped layer's shards (columns in
 * shard order), on `stream`.  bias: NULL or bf16 [info->n_total] device memory, added in fp32
 * before the single rounding to bf16 (the reference adds it afterwards with out.add_(bias),
 * gguf-plugin/patches/gguf-tiles-grouped.patch:167-168).  desc_dev: the plan's descriptor table in device memory.  workspace: at
 * least gqk_linear_workspace_bytes(info, M) bytes of 256-byte aligned device memory (NULL when
 * that is 0) holding arrival counters (its first GQK_CTR_BYTES bytes) and fp32 partials (after
 * them); it must be zero-filled before its first use, every launch leaves the counters at zero
 * again, one workspace serves every plan of every layer (the counter region is the same in all
 * of them), and launches sharing one workspace must not overlap in time.  M must be <= info->m_max.  Replaces the grouped op
 * torch.ops.vllm._fused_mul_mat_gguf_tiles_grouped -> gluon_mul_mat_tiles_grouped
 * (gguf-plugin/patches/gguf-tiles-grouped.patch:28-72, gguf-plugin/gluon/interface.py:141-188). */
int gqk_linear(const void* packed, const int32_t* desc_dev, const gqk_plan_info* info, const void* x, int64_t ldx,
               int M, void* y, int64_t ldy, const void* bias, void* workspace, int64_t workspace_bytes, void* stream);

/* gqk_linear without a workspace argument, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart
 * in the reference.  The split-K / stream-K counters and partials live in a file-scope device
 * array of GQK_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends; its address is taken
 * once per device on the first call, which also clears its counters with a fill kernel on
 * `stream`).  Allocates nothing.  A plan that needs more workspace at this M is refused with
 * GQK_ERR_SHAPE: GEMM plans above 64 rows on large layers, and GEMV plans whose split-K partials
 * exceed the 32 MiB (those are 64 rows x m_max tokens x 4 bytes per partial slot: at most 4,096
 * slots at m_max = 32, 8,192 at 16, 32,768 at 4; e.g. a layer of 2,374 tiles at K = 16384 split 16
 * ways at M <= 4 needs ~39 MB).  Every call on one GPU shares that
 * GPU's array: calls that overlap in time on one GPU (other streams, other threads) race. */
#define GQK_NOALLOC_SCRATCH_BYTES (GQK_CTR_BYTES + 33554432)
int gqk_linear_noalloc(const void* packed, const int32_t* desc_dev, const gqk_plan_info* info, const void* x,
                       int64_t ldx, int M, void* y, int64_t ldy, const void* bias, void* stream);

/* ---- GGUF v3 files: the load path ----------------------------------------------------------
 * The reference's tensors come from vLLM's GGUF loader (gguf-py 0.17.1 GGUFReader,
 * gguf-plugin/requirements.txt:1) and are repacked at load time by _create_tiles
 * (gguf-plugin/patches/gguf-tiles-all-types.patch:59-131).  Here a C++ reader maps the file read
 * only; tensor data is never copied on the host. */
typedef struct gqk_gguf gqk_gguf; /* an open GGUF file (immutable: safe to share across threads) */

/* GGUF metadata value types */
#define GQK_GGUF_UINT8 0
#define GQK_GGUF_INT8 1
#define GQK_GGUF_UINT16 2
#define GQK_GGUF_INT16 3
#define GQK_GGUF_UINT32 4
#define GQK_GGUF_INT32 5
#define GQK_GGUF_FLOAT32 6
#define GQK_GGUF_BOOL 7
#define GQK_GGUF_STRING 8
#define GQK_GGUF_ARRAY 9
#define GQK_GGUF_UINT64 10
#define GQK_GGUF_INT64 11
#define GQK_GGUF_FLOAT64 12

typedef struct gqk_gguf_tensor {
  const char* name;   /* NUL-terminated, owned by the handle */
  int32_t ggml_type;
  int32_t n_dims;
  int64_t dims[4];    /* GGUF order: dims[0] = weights per row (K), dims[1] = rows (N); unused = 1 */
  int64_t offset;     /* absolute byte offset of the data in the file */
  int64_t nbytes;     /* packed bytes; -1 for a type without a fixed block size here */
  const void* data;   /* host pointer into the read-only mapping (NULL when nbytes < 0) */
} gqk_gguf_tensor;

typedef struct gqk_gguf_kv {
  const char* key;    /* NUL-terminated, owned by the handle */
  int32_t type;       /* GQK_GGUF_* */
  int32_t array_type; /* element type of an ARRAY */
  int64_t count;      /* 1 for a scalar, bytes of a STRING, elements of an ARRAY */
  int64_t i64;        /* integer and BOOL scalars (UINT64 as its bit pattern) */
  double f64;         /* FLOAT32 / FLOAT64 scalars */
  const void* data;   /* STRING bytes (not NUL-terminated) or the first ARRAY element (mapping) */
} gqk_gguf_kv;

/* (weights per block, bytes per block) of a GGML type: gguf.GGML_QUANT_SIZES
 * (gguf-plugin/patches/gguf-prefill-dispatch.patch:42-45 reads it for the dequant shape). */
int gqk_ggml_type_size(int ggml_type, int32_t* block, int32_t* bytes);

/* Map and parse a GGUF v3 file (GGUFReader(path) in gguf-py).  *out is NULL on failure. */
int gqk_gguf_open(const char* path, gqk_gguf** out);
void gqk_gguf_close(gqk_gguf* f);
/* Counts, alignment (general.alignment, default 32), data-section offset and version. */
int gqk_gguf_info(const gqk_gguf* f, int64_t* n_tensors, int64_t* n_kv, int64_t* alignment, int64_t* data_offset,
                  int32_t* version);
/* Tensor info i (GGUFReader.tensors[i]); index of a tensor by name, -1 when absent. */
int gqk_gguf_tensor_at(const gqk_gguf* f, int64_t i, gqk_gguf_tensor* out);
int64_t gqk_gguf_find_tensor(const gqk_gguf* f, const char* name);
/* Metadata key/value i (GGUFReader.fields); index of a key, -1 when absent; string j of a STRING
 * (j = 0) or of an ARRAY of strings. */
int gqk_gguf_kv_at(const gqk_gguf* f, int64_t i, gqk_gguf_kv* out);
int64_t gqk_gguf_find_kv(const gqk_gguf* f, const char* key);
int gqk_gguf_kv_string(const gqk_gguf* f, int64_t i, int64_t j, const char** s, int64_t* len);

/* Load path of one quantized matrix: its raw rows from the mapping into `staging` (device, at
 * least nbytes), then gqk_repack into `tiles` (gqk_tiles_bytes(type, dims[1], dims[0]) bytes), both
 * on `stream`.  The copy reads pageable host memory, so it returns once the rows are staged. */
int gqk_gguf_upload_tiles(const gqk_gguf* f, int64_t i, void* staging, int64_t staging_bytes, void* tiles,
                          void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GGUF_HIP_H */
