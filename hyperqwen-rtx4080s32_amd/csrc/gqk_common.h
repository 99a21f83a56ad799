// gqk_common.h - GGML block formats and the CDNA4 plane-major tile layout (host + device).
//
// Block formats (GGML type id, bytes per block) follow gguf-py's GGML_QUANT_SIZES; the field
// offsets are those the reference parses: Q8_0/Q3_K/Q5_K/Q6_K gguf-plugin/gluon/kq_ref.py:35-79,
// Q4_K gguf-plugin/gluon/q4k.py:5-20, Q2_K gguf-plugin/gluon/q2k.py:5-12, IQ4_XS
// gguf-plugin/gluon/iq4xs.py:5-11, IQ3_S gguf-plugin/test_gguf_rco_cpu.py:215-227.
// Q4_0 / Q5_0 / IQ4_NL follow the GGML block spec (the reference serves them only through the
// unvendored CUDA MMVQ, gguf-plugin/patches/gguf-mmvq-batched.patch:98-126,258-266).
//
// Tile layout.  A shard of n rows x K weights is cut into 64-row tiles and 256-weight
// super-blocks ("records": one K-quant / IQ block, or eight consecutive 32-weight blocks).
// The bytes of (tile t, super-block kb) form one contiguous chunk of 64 * REC bytes at
//     chunk(t, kb) = base + (t * nb + kb) * 64 * REC
// Inside a chunk the record is split into planes (quants, high bits, scales, d ...); plane p
// holds the p-th slice of all 64 rows, column-major in columns of W bytes (W = 16, or the
// largest power of two dividing the plane's bytes per row):
//     byte j of plane p of row r  at  chunk + 64 * plane_off[p] + ((j / W) * 64 + r) * W + j % W
// so a wavefront whose lane r reads row r issues one fully coalesced load per column
// (1 KiB per 16-byte load).  The layout holds exactly the GGUF bytes (no padding inside a
// chunk; rows past n are zero), which is why bandwidth is counted on raw block bytes.
#pragma once
#include <stdint.h>

#define GQK_Q4_0 2
#define GQK_Q5_0 6
#define GQK_Q8_0 8
#define GQK_Q2_K 10
#define GQK_Q3_K 11
#define GQK_Q4_K 12
#define GQK_Q5_K 13
#define GQK_Q6_K 14
#define GQK_IQ4_NL 20
#define GQK_IQ3_S 21
#define GQK_IQ4_XS 23

#define GQK_MAX_PLANES 5

struct gqk_plane {
  int size;        // bytes per row in this plane
  int nseg;        // source segments (raw-record byte ranges) concatenated into the plane
  int seg_off;     // first segment's raw offset
  int seg_len;     // bytes per segment
  int seg_stride;  // raw distance between segments
};

struct gqk_type {
  int id;
  int block_weights;   // 32 or 256
  int block_bytes;     // GGUF bytes per block
  int rec;             // GGUF bytes per 256 weights
  int nplanes;
  gqk_plane planes[GQK_MAX_PLANES];
};

// Plane tables.  Every plane is a strided gather of equal segments from the raw 256-weight
// record: segment i = raw[seg_off + i * seg_stride, + seg_len).
#define GQK_TYPES_TABLE                                                                              \
  X(GQK_Q4_0,   32, 18,  144, 2, {{128, 8, 2, 16, 18}, {16, 8, 0, 2, 18}})                            \
  X(GQK_Q5_0,   32, 22,  176, 3, {{128, 8, 6, 16, 22}, {32, 8, 2, 4, 22}, {16, 8, 0, 2, 22}})          \
  X(GQK_Q8_0,   32, 34,  272, 2, {{256, 8, 2, 32, 34}, {16, 8, 0, 2, 34}})                            \
  X(GQK_Q2_K,  256, 84,   84, 3, {{64, 1, 16, 64, 0}, {16, 1, 0, 16, 0}, {4, 1, 80, 4, 0}})            \
  X(GQK_Q3_K,  256, 110, 110, 4, {{64, 1, 32, 64, 0}, {32, 1, 0, 32, 0}, {12, 1, 96, 12, 0}, {2, 1, 108, 2, 0}}) \
  X(GQK_Q4_K,  256, 144, 144, 2, {{128, 1, 16, 128, 0}, {16, 1, 0, 16, 0}})                          \
  X(GQK_Q5_K,  256, 176, 176, 3, {{128, 1, 48, 128, 0}, {32, 1, 16, 32, 0}, {16, 1, 0, 16, 0}})        \
  X(GQK_Q6_K,  256, 210, 210, 3, {{192, 1, 0, 192, 0}, {16, 1, 192, 16, 0}, {2, 1, 208, 2, 0}})       \
  X(GQK_IQ4_NL, 32, 18,  144, 2, {{128, 8, 2, 16, 18}, {16, 8, 0, 2, 18}})                            \
  X(GQK_IQ3_S, 256, 110, 110, 5, {{64, 1, 2, 64, 0}, {32, 1, 74, 32, 0}, {8, 1, 66, 8, 0}, {4, 1, 106, 4, 0}, {2, 1, 0, 2, 0}}) \
  X(GQK_IQ4_XS, 256, 136, 136, 2, {{128, 1, 8, 128, 0}, {8, 1, 0, 8, 0}})

// Q6_K's first plane is not a byte gather: its 192 bytes per row (GGUF's ql[128] and qh[64]) hold
// the 256 six-bit values q = lo | hi << 4 re-packed per 16-weight scale group g, as three dwords
// P0..P2 whose bytes i carry q[16 g + 4 m + i] & 63 (dword m) in bits 0..5 and bits 2m, 2m + 1 of
// q[16 g + 12 + i] in bits 6..7.  A decoder takes four 6-bit values with one AND (P_m & 0x3F3F3F3F)
// and the last four from the three top-bit pairs.  The dwords of groups 4a .. 4a + 3 fill the
// plane's columns 3a .. 3a + 2: column 3a + m holds P_m of group 4a + d as its dword d.  The repack
// builds this from the raw record in LDS, and the unrepack / tile dequantizer invert it.
__host__ __device__ constexpr int gqk_q6_pos(int g, int m, int i) { return 16 * (3 * (g >> 2) + m) + 4 * (g & 3) + i; }

// The same table as compile-time constants per type (device code)
struct gqk_type_c {
  int rec, nplanes;
  gqk_plane planes[GQK_MAX_PLANES];
};
template <int T> struct gqk_planes;
#define X(ID, BW, BB, REC, NP, ...) \
  template <> struct gqk_planes<ID> { static constexpr gqk_type_c v = {REC, NP, __VA_ARGS__}; };
GQK_TYPES_TABLE
#undef X

// Column width of a plane of `size` bytes per row: 16, or the largest power of two dividing it.
__host__ __device__ constexpr int gqk_col_width(int size) {
  return size % 16 == 0 ? 16 : size % 8 == 0 ? 8 : size % 4 == 0 ? 4 : size % 2 == 0 ? 2 : 1;
}

// Host lookup of a type's table entry (nullptr for an unsupported id).
inline const gqk_type* gqk_type_get(int id) {
#define X(ID, BW, BB, REC, NP, ...) \
  if (id == ID) { static const gqk_type t = {ID, BW, BB, REC, NP, __VA_ARGS__}; return &t; }
  GQK_TYPES_TABLE
#undef X
  return nullptr;
}

// Compile-time plane offsets (bytes per row before plane p) for the kernels.
template <int T> struct gqk_layout;
#define GQK_LAYOUT(T, REC_, ...)                                \
  template <> struct gqk_layout<T> {                            \
    static constexpr int REC = REC_;                            \
    static constexpr int off[] = {__VA_ARGS__};                 \
  };
GQK_LAYOUT(GQK_Q4_0, 144, 0, 128)
GQK_LAYOUT(GQK_Q5_0, 176, 0, 128, 160)
GQK_LAYOUT(GQK_Q8_0, 272, 0, 256)
GQK_LAYOUT(GQK_Q2_K, 84, 0, 64, 80)
GQK_LAYOUT(GQK_Q3_K, 110, 0, 64, 96, 108)
GQK_LAYOUT(GQK_Q4_K, 144, 0, 128)
GQK_LAYOUT(GQK_Q5_K, 176, 0, 128, 160)
GQK_LAYOUT(GQK_Q6_K, 210, 0, 192, 208)
GQK_LAYOUT(GQK_IQ4_NL, 144, 0, 128)
GQK_LAYOUT(GQK_IQ3_S, 110, 0, 64, 96, 104, 108)
GQK_LAYOUT(GQK_IQ4_XS, 136, 0, 128)
#undef GQK_LAYOUT

// status codes (mirrored in include/gguf_hip.h)
#define GQK_OK 0
#define GQK_ERR_TYPE (-1)
#define GQK_ERR_SHAPE (-2)
#define GQK_ERR_FORM (-3)
#define GQK_ERR_HIP (-4)
#define GQK_ERR_ARG (-5)

// descriptor row of a grouped launch (int32 words)
#define GQK_DESC_WORDS 16
#define GQK_SPLIT_MAX 16   // split-K factor bound: the last workgroup loads every partial at once
#define GQK_GEMM_MAX_WGS 1024   // persistent GEMM workgroups (up to three per CU) a launch may use
// Arrival counters at the start of every workspace: one fixed region for every plan of every
// layer (GEMV split tiles and GEMM stream-K tiles each index below it), so that one workspace per
// device serves all layers and batch sizes: no plan's fp32 partials overlap another's counters.
#define GQK_CTR_BYTES 262144   // (mirrored in include/gguf_hip.h)
#define GQK_CTR_WORDS (GQK_CTR_BYTES / 4)
#define GQK_GEMV_MAX_M 32   // batch rows of the streaming forms (GEMV up to 16, mid form 17..32); GEMM above
#define GQK_GEMV_MAX_WAVES 8   // waves per GEMV workgroup (two per SIMD: no register bound below 256)
#define GQK_GEMV_SLAB 2        // plan bm of the GEMV slab form (M <= 8: a workgroup per 32-row slab, x in LDS)
#define GQK_SLAB_MAX_WAVES 12  // slab form: waves per workgroup (one per pair of super-blocks: nb <= 24)
#define GQK_SLAB_MAX_LDS 153600   // slab form: LDS bytes of x (+ the IQ tables) per workgroup
#define GQK_SLAB_SB_BYTES(mpad) (608 * (mpad))   // LDS bytes of one super-block's staged x (slots + sums)
#define GQK_GEMV_TAB_BYTES 9216  // LDS bytes of the IQ lookup tables
enum {
  D_TYPE = 0,     // GGML type of the row's shard
  D_OFF_LO = 1,   // byte offset of the shard's tiles in the packed buffer (low 32 bits)
  D_OFF_HI = 2,   //                                                      (high 32 bits)
  D_TILE0 = 3,    // first 64-row tile (within the shard) of this workgroup
  D_NTILES = 4,   // tiles of this workgroup (GEMV: one per wave, <= 4; GEMM: BN / 64)
  D_KB0 = 5,      // first super-block of the workgroup's k-range
  D_KB1 = 6,      // one past the last
  D_SPLIT = 7,    // split-K index (partials slice)
  D_COL0 = 8,     // output column of the first row of tile D_TILE0
  D_NVALID = 9,   // valid output rows from D_COL0 (the shard's last tile is partial)
  D_NB = 10,      // super-blocks per row (K / 256)
  D_CTR = 11,     // GEMV split-K: arrival counter of the row's tile (index into the counters)
  D_NC = 12,      // GEMV: workgroups (rows) sharing the row's tile; 1 = the row writes y itself
  D_SLOT0 = 13,   // GEMV split-K: first fp32 partial slot of the row's tile (slot D_SLOT0 + D_SPLIT)
};

#ifdef __cplusplus
// sets the calling thread's gqk_last_error() message (library-internal; defined in gqk_api.hip)
void gqk_set_last_error(const char* msg);
#endif

// forms of a grouped launch
#define GQK_FORM_GEMV 1   // M <= 32, descriptor rows of (tile, k-range): M <= 16 the GEMV (in-register
                          // decode, MFMA per scale group, fp32 epilogue); 17..32 the mid form (g = 8:
                          // weights decoded to bf16 in registers, MFMA 32x32x16)
#define GQK_FORM_GEMM 2   // M > 32: tile decoded to bf16 in LDS, MFMA 32x32x16
