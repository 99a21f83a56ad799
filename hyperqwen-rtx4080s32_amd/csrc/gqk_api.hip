// gqk_api.hip - the C ABI (include/gguf_hip.h): argument checks, the launch plans, errors.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <algorithm>
#include <mutex>
#include <string>
#include <vector>
#include "gguf_hip.h"
#include "gqk_common.h"
#include "gqk_internal.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(GQK_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return GQK_OK;
}

// GEMV wave target when the caller gives none: eight waves per CU of the plan's device (2048 on a
// 256-CU MI355X).  A workgroup takes one 64-row tile and up to four waves split its k-range
// (measured: more waves per workgroup, or more waves than stay resident at once, run slower);
// shards with too few tiles for the target also split K across workgroups (partials combined
// in-kernel).
constexpr int kWavesPerCu = 8;
constexpr int kGemvWaves = 4;

// CUs of the current device (256 when none is visible: the plan of a host without a GPU); only
// asked when the caller of gqk_plan passes cus = 0
static int current_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
    (void)hipGetLastError();   // leave no error behind for the next launch check
    cus = 256;
  }
  return cus;
}

// bytes of the fp32 split-K partials: [tile][split][64 rows][m_max tokens]
int64_t gqk_partial_bytes(int64_t tiles, int64_t split, int64_t m_max) { return tiles * split * 64 * m_max * 4; }

// ---- the no-allocation entry point's workspace -------------------------------------------------
// A file-scope device array, one copy per GPU the library runs on (held until the process ends):
// the arrival counters (GQK_CTR_BYTES, zero at rest) then room for the fp32 split-K / stream-K
// partials.  Host code never uses the array's name as an address: the per-device address comes
// from hipGetSymbolAddress, taken once per device with that device current.
constexpr int64_t kScratchBytes = GQK_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {nullptr};

__global__ void zero_words(uint32_t* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) p[i] = 0;
}

// The current device's scratch address; the first call on a device takes it and clears the
// counter region with a fill kernel on `st` (no memset: the call may be under graph capture, where
// the fill is recorded too and then zeroes counters that are zero at rest anyway).
int scratch_for_current_device(hipStream_t st, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(GQK_ERR_HIP, "linear_noalloc: no current HIP device (or device %d >= %d)", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return fail(GQK_ERR_HIP, "linear_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    if ((uintptr_t)ptr & 255) return fail(GQK_ERR_HIP, "linear_noalloc: scratch on device %d not 256-byte aligned", dev);
    hipLaunchKernelGGL(zero_words, dim3(64), dim3(256), 0, st, (uint32_t*)ptr, (int64_t)GQK_CTR_BYTES / 4);
    const hipError_t le = hipGetLastError();
    if (le != hipSuccess) return fail(GQK_ERR_HIP, "linear_noalloc: clearing the scratch counters: %s", hipGetErrorString(le));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return GQK_OK;
}

// The memory floor of a shard: a plain streaming read of its packed bytes on a given grid.  Wave
// w of W reads the 1 KiB units [w n / W, (w + 1) n / W) of the buffer, kFloorLoads units (one
// 16-byte buffer load per lane each) in flight per step, and folds them into one word per wave so
// the loads stay live.  Units past the wave's range read out of the buffer's bounds (zeros,
// no memory access).
constexpr int kFloorLoads = 16;
typedef uint32_t v4u_fl __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(1024) void read_floor_kernel(const uint8_t* buf, uint32_t units,
                                                                           uint32_t* sink) {
  const int lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  const uint64_t W = (uint64_t)gridDim.x * nw, w = (uint64_t)blockIdx.x * nw + (threadIdx.x >> 6);
  const uint32_t u0 = (uint32_t)(w * units / W), u1 = (uint32_t)((w + 1) * units / W);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)buf, 0, units * 1024u, 0x00020000);
  uint32_t acc = 0;
  for (uint32_t u = u0; u < u1; u += kFloorLoads) {
    v4u_fl v[kFloorLoads];
#pragma unroll
    for (int i = 0; i < kFloorLoads; ++i)
      v[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, u + i < u1 ? (u + i) * 1024u + lane * 16u : 0xFFFFFFF0u, 0, 0);
#pragma unroll
    for (int i = 0; i < kFloorLoads; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
  }
  for (int o = 32; o > 0; o >>= 1) acc ^= __shfl_xor(acc, o);
  if (lane == 0) sink[w] = acc;
}

}  // namespace

void gqk_set_last_error(const char* msg) { g_err = msg ? msg : ""; }

extern "C" {

const char* gqk_last_error(void) { return g_err.c_str(); }

int gqk_version(void) { return 200; }

int gqk_type_info(int ggml_type, int32_t* info, int32_t* planes) {
  const gqk_type* t = gqk_type_get(ggml_type);
  if (!t) return fail(GQK_ERR_TYPE, "unsupported GGML type %d", ggml_type);
  if (!info) return fail(GQK_ERR_ARG, "gqk_type_info: info is NULL");
  info[0] = t->block_weights;
  info[1] = t->block_bytes;
  info[2] = t->rec;
  info[3] = t->nplanes;
  if (planes)
    for (int p = 0; p < t->nplanes; ++p) {
      planes[6 * p + 0] = t->planes[p].size;
      planes[6 * p + 1] = t->planes[p].nseg;
      planes[6 * p + 2] = t->planes[p].seg_off;
      planes[6 * p + 3] = t->planes[p].seg_len;
      planes[6 * p + 4] = t->planes[p].seg_stride;
      planes[6 * p + 5] = gqk_col_width(t->planes[p].size);
    }
  return GQK_OK;
}

int gqk_dequantize(const void* W, int64_t w_row_stride, int ggml_type, int64_t n, int64_t K, void* out,
                   int64_t ld_out, int out_dtype, void* stream) {
  const gqk_type* t = gqk_type_get(ggml_type);
  if (!t) return fail(GQK_ERR_TYPE, "unsupported GGML type %d", ggml_type);
  if (n < 0 || K < 0 || K % t->block_weights != 0)
    return fail(GQK_ERR_SHAPE, "dequantize: K=%lld is not a multiple of the type's %d-weight block", (long long)K,
                t->block_weights);
  if (out_dtype < 0 || out_dtype > 2) return fail(GQK_ERR_ARG, "dequantize: out_dtype %d", out_dtype);
  if (n == 0 || K == 0) return GQK_OK;
  if (!W || !out) return fail(GQK_ERR_ARG, "dequantize: null pointer");
  if (w_row_stride < K / t->block_weights * t->block_bytes)
    return fail(GQK_ERR_SHAPE, "dequantize: row stride %lld < row bytes %lld", (long long)w_row_stride,
                (long long)(K / t->block_weights * t->block_bytes));
  if (ld_out < K) return fail(GQK_ERR_SHAPE, "dequantize: ld_out %lld < K %lld", (long long)ld_out, (long long)K);
  int rc = gqk::launch_dequant(ggml_type, W, w_row_stride, n, K, out, ld_out, out_dtype, (hipStream_t)stream);
  if (rc) return fail(rc, "dequantize: type %d", ggml_type);
  return check_launch("dequantize");
}

int gqk_dequantize_tiles(const void* tiles, int ggml_type, int64_t n, int64_t K, void* out, int64_t ld_out,
                         int out_dtype, void* stream) {
  const gqk_type* t = gqk_type_get(ggml_type);
  if (!t) return fail(GQK_ERR_TYPE, "unsupported GGML type %d", ggml_type);
  if (n < 0 || K < 0 || K % 256 != 0)
    return fail(GQK_ERR_SHAPE, "dequantize_tiles: K=%lld is not a multiple of 256", (long long)K);
  if (out_dtype < 0 || out_dtype > 2) return fail(GQK_ERR_ARG, "dequantize_tiles: out_dtype %d", out_dtype);
  if (n == 0 || K == 0) return GQK_OK;
  if (!tiles || !out) return fail(GQK_ERR_ARG, "dequantize_tiles: null pointer");
  if ((uintptr_t)tiles & 15) return fail(GQK_ERR_SHAPE, "dequantize_tiles: tiles must be 16-byte aligned");
  if (ld_out < K) return fail(GQK_ERR_SHAPE, "dequantize_tiles: ld_out %lld < K %lld", (long long)ld_out, (long long)K);
  int rc = gqk::launch_tile_dequant(ggml_type, tiles, n, K, out, ld_out, out_dtype, (hipStream_t)stream);
  if (rc) return fail(rc, "dequantize_tiles: type %d, %lld x %lld", ggml_type, (long long)n, (long long)K);
  return check_launch("dequantize_tiles");
}

int64_t gqk_tiles_bytes(int ggml_type, int64_t n, int64_t K) {
  const gqk_type* t = gqk_type_get(ggml_type);
  if (!t) return fail(GQK_ERR_TYPE, "unsupported GGML type %d", ggml_type);
  if (n < 0 || K < 0 || K % 256 != 0)
    return fail(GQK_ERR_SHAPE, "tiles: K=%lld is not a multiple of 256", (long long)K);
  return (n + 63) / 64 * 64 * (K / 256) * t->rec;
}

static int repack_common(const void* W, int64_t stride, int type, int64_t n, int64_t K, void* tiles, bool to_tiles,
                         void* stream) {
  const gqk_type* t = gqk_type_get(type);
  if (!t) return fail(GQK_ERR_TYPE, "unsupported GGML type %d", type);
  if (n < 0 || K < 0 || K % 256 != 0) return fail(GQK_ERR_SHAPE, "repack: K=%lld is not a multiple of 256", (long long)K);
  if (n == 0 || K == 0) return GQK_OK;
  if (!W || !tiles) return fail(GQK_ERR_ARG, "repack: null pointer");
  if ((uintptr_t)tiles & 15) return fail(GQK_ERR_SHAPE, "repack: tiles must be 16-byte aligned");
  if (stride < K / 256 * t->rec)
    return fail(GQK_ERR_SHAPE, "repack: row stride %lld < row bytes %lld", (long long)stride, (long long)(K / 256 * t->rec));
  int rc = gqk::launch_repack(type, W, stride, n, K, tiles, to_tiles, (hipStream_t)stream);
  if (rc) return fail(rc, "repack: type %d", type);
  return check_launch(to_tiles ? "repack" : "unrepack");
}

int gqk_repack(const void* W, int64_t w_row_stride, int ggml_type, int64_t n, int64_t K, void* tiles, void* stream) {
  return repack_common(W, w_row_stride, ggml_type, n, K, tiles, true, stream);
}

int gqk_unrepack(const void* tiles, int ggml_type, int64_t n, int64_t K, void* W, int64_t w_row_stride, void* stream) {
  return repack_common(W, w_row_stride, ggml_type, n, K, (void*)tiles, false, stream);
}

int gqk_plan(const gqk_shard* shards, int nshards, int64_t K, int M, int target_wgs, int cus, int32_t* desc,
             int64_t desc_capacity, gqk_plan_info* info) {
  if (!shards || nshards <= 0 || !info) return fail(GQK_ERR_ARG, "plan: no shards / info");
  if (cus < 0) return fail(GQK_ERR_ARG, "plan: cus=%d", cus);
  if (cus == 0) cus = current_cus();
  if (K <= 0 || K % 256 != 0) return fail(GQK_ERR_SHAPE, "plan: K=%lld is not a positive multiple of 256", (long long)K);
  if (M <= 0) return fail(GQK_ERR_SHAPE, "plan: M=%d", M);
  const int64_t nb = K / 256;
  if (nb > (1 << 30)) return fail(GQK_ERR_SHAPE, "plan: K too large");
  int64_t n_total = 0, expect_off = 0;
  int first_type = shards[0].ggml_type;
  bool mixed = false;
  for (int i = 0; i < nshards; ++i) {
    const gqk_type* t = gqk_type_get(shards[i].ggml_type);
    if (!t) return fail(GQK_ERR_TYPE, "plan: shard %d has unsupported GGML type %d", i, shards[i].ggml_type);
    if (shards[i].n <= 0) return fail(GQK_ERR_SHAPE, "plan: shard %d has %lld rows", i, (long long)shards[i].n);
    if (shards[i].offset != expect_off)
      return fail(GQK_ERR_SHAPE, "plan: shard %d at byte %lld, expected %lld (shards are packed back to back)", i,
                  (long long)shards[i].offset, (long long)expect_off);
    if (shards[i].offset % 16 != 0) return fail(GQK_ERR_SHAPE, "plan: shard %d offset not 16-byte aligned", i);
    expect_off += (shards[i].n + 63) / 64 * 64 * nb * t->rec;
    n_total += shards[i].n;
    mixed |= shards[i].ggml_type != first_type;
  }
  if (n_total >= (int64_t)1 << 31) return fail(GQK_ERR_SHAPE, "plan: %lld output columns", (long long)n_total);

  gqk_plan_info pi{};
  pi.types_mask = mixed ? 0 : first_type;
  pi.nb = (int32_t)nb;
  pi.n_total = n_total;
  std::vector<int32_t> rows;
  auto row = [&](int i, int64_t tile0, int ntiles, int64_t kb0, int64_t kb1, int split, int64_t col0, int64_t ctr,
                 int nc = 1, int64_t slot0 = 0) {
    int32_t r[GQK_DESC_WORDS] = {0};
    r[D_TYPE] = shards[i].ggml_type;
    r[D_OFF_LO] = (int32_t)(uint32_t)(shards[i].offset & 0xFFFFFFFF);
    r[D_OFF_HI] = (int32_t)(shards[i].offset >> 32);
    r[D_TILE0] = (int32_t)tile0;
    r[D_NTILES] = ntiles;
    r[D_KB0] = (int32_t)kb0;
    r[D_KB1] = (int32_t)kb1;
    r[D_SPLIT] = split;
    r[D_COL0] = (int32_t)(col0 + tile0 * 64);
    r[D_NVALID] = (int32_t)std::min<int64_t>((int64_t)ntiles * 64, shards[i].n - tile0 * 64);
    r[D_NB] = (int32_t)nb;
    r[D_CTR] = (int32_t)ctr;
    r[D_NC] = nc;
    r[D_SLOT0] = (int32_t)slot0;
    rows.insert(rows.end(), r, r + GQK_DESC_WORDS);
  };
  int64_t tiles = 0;
  for (int i = 0; i < nshards; ++i) tiles += (shards[i].n + 63) / 64;
  // The fixed counter region of every plan (the GEMV's split tiles and the GEMM's stream-K tiles
  // index below GQK_CTR_WORDS), so that one workspace serves every layer and every M.
  if (tiles > GQK_CTR_WORDS)
    return fail(GQK_ERR_SHAPE, "plan: %lld 64-row tiles (%lld rows) above the %d the counter region serves",
                (long long)tiles, (long long)(64 * tiles), GQK_CTR_WORDS);
  const int64_t ctr_bytes = GQK_CTR_BYTES;
  pi.ctr_bytes = (int32_t)ctr_bytes;
  // The GEMV serves up to 16 rows for every type (with its x operands broadcast from registers
  // the table types too beat the 32-row GEMM tile at 16 rows: IQ4_NL / IQ3_S / IQ4_XS 34816 x 5120
  // 41 / 43 / 42 us against 51 / 56 / 50 us, 5120 x 17408 26-28 us against 39-46 us), and the mid
  // form (g = 8) 17..32 rows with the same descriptor rows, split policy and exchange.
  if (M <= GQK_GEMV_MAX_M) {
    pi.form = GQK_FORM_GEMV;
    pi.g = M <= 4 ? 1 : M <= 8 ? 2 : M <= 16 ? 4 : 8;
    pi.m_max = 4 * pi.g;
    // The slab form (up to 8 rows): a workgroup per 32-row half of a tile over the whole k-range,
    // one wave per pair of super-blocks, each staging its own x in LDS; no split-K exchange.  One
    // workgroup per CU, so its time follows the slab's bytes, not the shard's: taken when the
    // slabs fill one round of the CUs, at least half of them.  Measured on 256 CUs against the
    // split-K plans (eight types, µs): qkv 7168 x 5120 (224 slabs) 0.3-1.7 faster at M = 1 / 4 and
    // 0.2-1.8 at M = 8; o_proj 5120 x 5120 (160 slabs) 0.3-0.6 faster at M = 1 / 4, and at M = 6 / 8
    // 0.1-0.7 faster for Q5_K, IQ4_XS, Q8_0, Q4_0, Q2_K, even for Q4_K, Q6_K, IQ3_S.
    //
    // From 17 rows the mid form's slab (32 x 32 MFMA blocks, x staged per step) replaces the mid
    // form's split-K exchange, whose 8 KiB of partials per workgroup cost ~30% of its launches
    // (eleven types at M = 17 / 32: qkv 5.6-9.8 us faster, o_proj 3.0-5.1; Q4_K qkv 20.7 -> 13.4 us
    // at 32).  At 9..16 rows it also beats the G = 4 GEMV when the slabs nearly fill the CUs (qkv,
    // 224 of 256: 1.0-3.5 us faster at 12, except IQ3_S, 0.6-0.8 slower); at 160 slabs (o_proj)
    // only for the types of the lightest decode (M = 9 / 12 / 16: Q8_0 1.4-1.9 us, Q4_K 1.0-1.4,
    // Q2_K 0.35-0.75, Q5_K 0.1-0.5 faster; Q3_K, Q6_K, IQ4_NL, IQ4_XS 0.3-1.3 and IQ3_S 2.5 slower).
    // Up to 8 rows the GEMV slab is 1.5-4.8 us faster than it.  `down` (68
    // super-blocks, 12 waves of ~6) measured 3-7 us slower than split-K at 24-32 rows.
    int64_t slabs = 0;
    bool any_iq = false, any_iq3s = false, light = true;
    for (int i = 0; i < nshards; ++i) {
      const int64_t rem = shards[i].n % 64;
      slabs += 2 * ((shards[i].n + 63) / 64) - (rem != 0 && rem <= 32 ? 1 : 0);
      const int t = shards[i].ggml_type;
      any_iq |= t == GQK_IQ4_NL || t == GQK_IQ4_XS || t == GQK_IQ3_S;
      any_iq3s |= t == GQK_IQ3_S;
      light &= t == GQK_Q8_0 || t == GQK_Q2_K || t == GQK_Q4_K || t == GQK_Q5_K;
    }
    const bool slab_fit =
        pi.g <= 2 ? nb * GQK_SLAB_SB_BYTES(pi.m_max) + (any_iq ? GQK_GEMV_TAB_BYTES : 0) <= GQK_SLAB_MAX_LDS
                  : pi.g == 8 || (8 * slabs >= 7 * cus && !any_iq3s) || light;
    const bool slab = target_wgs <= 0 && nb <= 2 * GQK_SLAB_MAX_WAVES && slab_fit && 2 * slabs >= cus && slabs <= cus;
    if (slab) {
      if (pi.g == 4) {   // served by the mid form's slab (x padded to 32 tokens)
        pi.g = 8;
        pi.m_max = 32;
      }
      pi.bm = GQK_GEMV_SLAB;
      pi.nw = (int32_t)((nb + 1) / 2);
      pi.split = 1;
      int64_t col0 = 0;
      for (int i = 0; i < nshards; ++i) {
        const int64_t ntile = (shards[i].n + 63) / 64;
        for (int64_t t0 = 0; t0 < ntile; ++t0)
          for (int h = 0; h < 2 && 64 * t0 + 32 * h < shards[i].n; ++h) row(i, t0, 1, 0, nb, h, col0, 0);
        col0 += shards[i].n;
      }
      pi.workspace_bytes = 0;
    } else {
      // waves per tile from the wave target; a workgroup's waves (at most nwmax: the x staging of
      // G >= 4 needs more LDS) split its k-range, and only when a tile wants more waves than one
      // workgroup holds does K split across workgroups.  Every wave keeps >= 1 super-block.
      // (Measured: a balanced stream that cuts the records into equal ranges per workgroup, so
      // that tile counts not a multiple of the CU count leave no tail, ran slower: its shared
      // tiles' partial exchange and shorter per-wave streams cost more than the tail.)
      int64_t target = target_wgs > 0 ? target_wgs : (int64_t)kWavesPerCu * cus;
      // Up to four rows (one token group), when every wave can hold exactly one record (k-range a
      // multiple of four super-blocks, at most GQK_SPLIT_MAX workgroups per tile): one record per
      // wave in short-lived workgroups.  Their loads all go out at once and the dispatcher balances
      // the CUs, which beats streaming waves there (gate_up 34816 x 5120 at M = 1: Q6_K 34.9 -> 32.5
      // us, Q5_K 31.4 -> 28.7, IQ4_XS 30.6 -> 29.1, Q5_0 31.4 -> 28.3; the others within 1 us); at 8 rows
      // the heavier per-record work makes the streaming plan the faster one for a single type.  A
      // mixed-type layer takes it up to eight rows: its streaming kernel holds the registers of its
      // costliest format (~235 VGPRs: two waves per SIMD) where the one-record kernel needs ~100
      // (a mixed stack's qkv + o_proj + gate_up launches at K = 5120, M = 8: 49.0 -> 43.2 us per layer; at 16
      // rows no gain, and splitting `down`'s 68 super-blocks 17 ways measured no better either).
      if (target_wgs <= 0 && (pi.g == 1 || (mixed && pi.g == 2)) && nb % kGemvWaves == 0 &&
          nb / kGemvWaves <= GQK_SPLIT_MAX)
        target = tiles * nb;
      const int64_t per_tile = std::max<int64_t>(1, (target + tiles - 1) / tiles);
      const int64_t nw = std::max<int64_t>(1, std::min({per_tile, nb, (int64_t)kGemvWaves}));
      const int64_t split =
          std::max<int64_t>(1, std::min({(per_tile + nw - 1) / nw, nb / nw, (int64_t)GQK_SPLIT_MAX}));
      // Tail: with whole tiles (split 1) in more than one round of resident workgroups (target / nw
      // of them, two per CU at the default target), a last round of r <= half the slots would put
      // a third whole tile on r CUs, which then finish last (gate_up's 544 tiles on 256 CUs: 28.5 us
      // against 22.2 us for 512).  Those r tiles split K instead, into workgroups of >= one record a
      // wave, so their work spreads over up to half the CUs as light extra workgroups.
      const int64_t slots = std::max<int64_t>(1, target / nw);
      int64_t tail = 0, split_tail = 1;
      if (split == 1 && tiles > slots) {
        const int64_t r = tiles % slots;
        if (r > 0 && 2 * r <= slots) split_tail = std::min<int64_t>({nb / nw, std::max<int64_t>(1, slots / 2 / r),
                                                                     (int64_t)GQK_SPLIT_MAX});
        if (split_tail > 1) tail = r;
      }
      pi.nw = (int32_t)nw;
      pi.split = (int32_t)std::max(split, split_tail);
      // One round of split tiles whose waves stream >= 2 records each: fill the resident slots
      // exactly (s0 or s0 + 1 rows per tile) rather than overshoot them and leave a few CUs a third
      // workgroup (down 5120 x 17408: 560 -> 512 workgroups, Q6_K M = 1 26.0 -> 21.3 us).  With one
      // record per wave (qkv, o_proj at K = 5120) the extra workgroups' memory parallelism wins.
      int64_t s0 = split, extra = 0;
      if (split > 1 && tiles <= slots && nb >= 2 * split * nw) {
        const int64_t smax = std::max<int64_t>(1, std::min<int64_t>(nb / nw, GQK_SPLIT_MAX));
        const int64_t total = std::min(slots, tiles * smax);
        s0 = std::max<int64_t>(1, total / tiles);
        extra = s0 < smax ? total - s0 * tiles : 0;
        pi.split = (int32_t)(s0 + (extra > 0));
      }
      int64_t col0 = 0, g = 0, ctr = 0, slot = 0;
      bool one_record = true;   // every wave of every row streams exactly one record
      for (int i = 0; i < nshards; ++i) {
        int64_t ntile = (shards[i].n + 63) / 64;
        for (int64_t t0 = 0; t0 < ntile; ++t0, ++g) {
          const int64_t sp = g >= tiles - tail ? split_tail : split > 1 ? s0 + (g < extra) : split;
          if (sp == 1) {
            row(i, t0, 1, 0, nb, 0, col0, 0);
            one_record &= nb == nw;
            continue;
          }
          for (int64_t s = 0; s < sp; ++s) {   // balanced partition: every split owns >= 1 super-block
            row(i, t0, 1, s * nb / sp, (s + 1) * nb / sp, (int)s, col0, ctr, (int)sp, slot);
            one_record &= (s + 1) * nb / sp - s * nb / sp == nw;
          }
          ++ctr;
          slot += sp;
        }
        col0 += shards[i].n;
      }
      // a plan whose waves all hold a single record launches the kernel built without the register
      // pipeline (fewer registers: more workgroups resident), flagged in the GEMM-only bm field
      pi.bm = one_record && pi.g <= 4 ? 1 : 0;
      // workspace: the counter region (one arrival counter per split tile; zero before the first
      // launch, left zero by each launch), then the fp32 partial slots [slot][64 rows][m_max tokens]
      pi.workspace_bytes = slot > 0 ? ctr_bytes + gqk_partial_bytes(slot, 1, pi.m_max) : 0;
    }
  } else {
    pi.form = GQK_FORM_GEMM;
    // 64 / 128 tokens x 128 rows per tile up to 128 tokens (one decode of each weight); 256 x 256 above.
    pi.bm = M <= 64 ? 64 : M <= 128 ? 128 : 256;
    // A layer with few 256-row groups keeps the 128 x 128 form up to 384 rows (768 for K up to
    // 8192) when the 256 x 256 form would have fewer tiles than a quarter of the CUs (one
    // workgroup each): its stream-K would leave most CUs idle and pad the last token block.
    // Measured on the 5120- and 7168-row shards (20 / 28 groups of 256 rows): 13-30% faster at
    // M = 129-384, 9-19% at 448-512 and (o_proj) 6-21% at 640-768 for K = 5120; qkv at 640-768
    // (above the quarter) even to 11% slower, `down` (K = 17408) 5-19% slower at 448-512, and
    // gate_up (136 groups) 6-22% slower at every M.
    if (pi.bm == 256 && (M <= 384 || (M <= 768 && nb <= 32))) {
      int64_t groups = 0;
      for (int i = 0; i < nshards; ++i) groups += ((shards[i].n + 63) / 64 + 3) / 4;
      if (groups * ((M + 255) / 256) * 4 < cus) pi.bm = 128;
    }
    pi.m_max = 1 << 30;
    pi.split = 1;
    const int64_t per = pi.bm == 256 ? 4 : 2;   // tiles per descriptor row
    int64_t col0 = 0;
    for (int i = 0; i < nshards; ++i) {
      int64_t ntile = (shards[i].n + 63) / 64;
      for (int64_t t0 = 0; t0 < ntile; t0 += per) row(i, t0, (int)std::min<int64_t>(per, ntile - t0), 0, nb, 0, col0, 0);
      col0 += shards[i].n;
    }
    pi.workspace_bytes = 0;
  }
  pi.n_desc = (int32_t)(rows.size() / GQK_DESC_WORDS);
  bool all_split = pi.form == GQK_FORM_GEMV;
  for (int64_t r = 0; all_split && r < pi.n_desc; ++r) all_split = rows[r * GQK_DESC_WORDS + D_NC] > 1;
  if (all_split) {
    // A plan whose tiles are all split (one record per wave; `down`): workgroup i runs on XCD
    // i % 8 (the dispatcher deals workgroups to the XCDs in turn), so the tiles go eight at a time
    // with their splits interleaved (workgroup 8 s + x = split s of the group's tile x): all
    // contributors of a tile share one XCD (for the exchange's round trips), and every XCD gets the
    // same work (qkv / o_proj 1.5-3.4% faster).  Plans with whole tiles keep their order (putting
    // their split tail first measured up to 6% slower).
    const int64_t n = pi.n_desc;
    std::vector<int32_t> out;
    out.reserve(rows.size());
    auto row_at = [&](int64_t r) { return rows.begin() + r * GQK_DESC_WORDS; };
    std::vector<std::pair<int64_t, int>> tiles_split;   // (first row, contributors)
    for (int64_t r = 0; r < n;) {
      const int nc = row_at(r)[D_NC];
      if (nc > 1) tiles_split.push_back({r, nc});
      r += nc;
    }
    for (size_t a = 0; a < tiles_split.size();) {
      size_t b = a;
      while (b < tiles_split.size() && b - a < 8 && tiles_split[b].second == tiles_split[a].second) ++b;
      for (int sidx = 0; sidx < tiles_split[a].second; ++sidx)
        for (size_t t = a; t < b; ++t) {
          auto it = row_at(tiles_split[t].first + sidx);
          out.insert(out.end(), it, it + GQK_DESC_WORDS);
        }
      a = b;
    }
    rows.swap(out);
  }
  *info = pi;
  if (desc) {
    if (desc_capacity < (int64_t)rows.size())
      return fail(GQK_ERR_ARG, "plan: descriptor capacity %lld < %lld words", (long long)desc_capacity,
                  (long long)rows.size());
    memcpy(desc, rows.data(), rows.size() * sizeof(int32_t));
  }
  return GQK_OK;
}

int64_t gqk_linear_workspace_bytes(const gqk_plan_info* info, int M) {
  if (!info) return fail(GQK_ERR_ARG, "linear_workspace_bytes: info is NULL");
  if (M <= 0) return 0;
  if (info->form == GQK_FORM_GEMV) return info->workspace_bytes;
  if (info->form == GQK_FORM_GEMM) {
    const int64_t n = gqk::gemm_workspace(info->bm, info->n_desc, M, info->nb, info->ctr_bytes);
    return n < 0 ? fail(GQK_ERR_HIP, "linear_workspace_bytes: no HIP device") : n;
  }
  return fail(GQK_ERR_FORM, "linear_workspace_bytes: unknown form %d", info->form);
}

int64_t gqk_workspace_bytes_max(void) {
  const int64_t n = gqk::gemm_workspace_max();
  return n < 0 ? fail(GQK_ERR_HIP, "workspace_bytes_max: no HIP device") : n;
}

int gqk_linear(const void* packed, const int32_t* desc_dev, const gqk_plan_info* info, const void* x, int64_t ldx,
               int M, void* y, int64_t ldy, const void* bias, void* workspace, int64_t workspace_bytes, void* stream) {
  if (!info) return fail(GQK_ERR_ARG, "linear: info is NULL");
  if (M < 0) return fail(GQK_ERR_SHAPE, "linear: M=%d", M);
  if (M == 0) return GQK_OK;
  if (!packed || !desc_dev || !x || !y) return fail(GQK_ERR_ARG, "linear: null pointer");
  const int64_t K = (int64_t)info->nb * 256;
  if (ldx < K || ldy < info->n_total)
    return fail(GQK_ERR_SHAPE, "linear: ldx %lld < K %lld or ldy %lld < columns %lld", (long long)ldx, (long long)K,
                (long long)ldy, (long long)info->n_total);
  if (((uintptr_t)x & 15) || (ldx & 7))
    return fail(GQK_ERR_SHAPE, "linear: x must be 16-byte aligned with a row stride that is a multiple of 8");
  if (info->form == GQK_FORM_GEMV) {
    if (M > info->m_max) return fail(GQK_ERR_FORM, "linear: M=%d above the GEMV plan's %d rows", M, info->m_max);
    if (info->g != 1 && info->g != 2 && info->g != 4 && info->g != 8) return fail(GQK_ERR_FORM, "linear: g=%d", info->g);
    int* counters = nullptr;
    float* partials = nullptr;
    if (info->workspace_bytes > 0) {
      // counters at the start (one per split tile, fewer than the descriptor rows), partial slots after
      const int64_t cb = info->ctr_bytes, need = info->workspace_bytes;
      if (cb != GQK_CTR_BYTES || need <= cb)
        return fail(GQK_ERR_FORM, "linear: counter region %lld / workspace %lld bytes", (long long)cb, (long long)need);
      if (!workspace || workspace_bytes < need)
        return fail(GQK_ERR_SHAPE, "linear: workspace %lld bytes < %lld", (long long)workspace_bytes, (long long)need);
      if ((uintptr_t)workspace & 255) return fail(GQK_ERR_SHAPE, "linear: workspace not 256-byte aligned");
      counters = (int*)workspace;
      partials = (float*)((char*)workspace + cb);
    }
    int rc = gqk::launch_gemv((const uint8_t*)packed, desc_dev, info->n_desc, info->types_mask, x, ldx, M, info->g, info->nw,
                              info->bm, info->nb, y, ldy, bias, partials, counters, (hipStream_t)stream);
    if (rc) return fail(rc, "linear: GEMV launch form");
    return check_launch("linear (GEMV)");
  }
  if (info->form == GQK_FORM_GEMM) {
    if ((int64_t)M * ldx >= ((int64_t)1 << 40)) return fail(GQK_ERR_SHAPE, "linear: x too large");
    int rc = gqk::launch_gemm((const uint8_t*)packed, desc_dev, info->n_desc, info->types_mask, x, ldx, M, K, y, ldy,
                              bias, info->bm, info->ctr_bytes, workspace, workspace_bytes, (hipStream_t)stream);
    if (rc == GQK_ERR_SHAPE)
      return fail(rc, "linear: GEMM workspace %lld bytes < %lld (or not 256-byte aligned)", (long long)workspace_bytes,
                  (long long)gqk::gemm_workspace(info->bm, info->n_desc, M, info->nb, info->ctr_bytes));
    if (rc == GQK_ERR_FORM)
      return fail(rc, "linear: %d-byte counter region below the device's persistent GEMM workgroups", info->ctr_bytes);
    if (rc) return fail(rc, "linear: GEMM launch form bm=%d", info->bm);
    return check_launch("linear (GEMM)");
  }
  return fail(GQK_ERR_FORM, "linear: unknown form %d", info->form);
}

int gqk_linear_noalloc(const void* packed, const int32_t* desc_dev, const gqk_plan_info* info, const void* x,
                       int64_t ldx, int M, void* y, int64_t ldy, const void* bias, void* stream) {
  if (!info) return fail(GQK_ERR_ARG, "linear_noalloc: info is NULL");
  if (M < 0) return fail(GQK_ERR_SHAPE, "linear_noalloc: M=%d", M);
  if (M == 0) return GQK_OK;
  const int64_t need = gqk_linear_workspace_bytes(info, M);
  if (need < 0) return (int)need;
  if (need > kScratchBytes)
    return fail(GQK_ERR_SHAPE,
                "linear_noalloc: this plan needs %lld workspace bytes at M=%d, above the %lld-byte scratch of the "
                "no-allocation entry point (use gqk_linear with a caller workspace)",
                (long long)need, M, (long long)kScratchBytes);
  void* ws = nullptr;
  int rc = scratch_for_current_device((hipStream_t)stream, &ws);
  if (rc) return rc;
  return gqk_linear(packed, desc_dev, info, x, ldx, M, y, ldy, bias, need > 0 ? ws : nullptr, need > 0 ? kScratchBytes : 0,
                    stream);
}

int gqk_read_floor(const void* buf, int64_t bytes, int grid, int waves, void* sink, void* stream) {
  if (!buf || !sink) return fail(GQK_ERR_ARG, "read_floor: null pointer");
  if (bytes < 1024 || bytes % 1024 || bytes > ((int64_t)1 << 31))
    return fail(GQK_ERR_SHAPE, "read_floor: %lld bytes (a multiple of 1 KiB, at most 2 GiB)", (long long)bytes);
  if (grid < 1 || waves < 1 || waves > 16)
    return fail(GQK_ERR_SHAPE, "read_floor: grid %d x %d waves (1..16 waves)", grid, waves);
  hipLaunchKernelGGL(read_floor_kernel, dim3(grid), dim3(64 * waves), 0, (hipStream_t)stream, (const uint8_t*)buf,
                     (uint32_t)(bytes / 1024), (uint32_t*)sink);
  return check_launch("read_floor");
}

}  // extern "C"
