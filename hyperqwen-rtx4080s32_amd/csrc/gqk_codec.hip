// gqk_codec.hip - GGML block decode to fp32 (the dequantize API) and the tile repack.
//
// dequantize: every weight is computed as gguf-py computes it (gguf.quants.dequantize, the
// reference dequantizer of this path: gguf-plugin/patches/gguf-prefill-dispatch.patch:42-45,
// gguf-plugin/gluon/tiles.py:141-149): (d * sc) * q - dmin * m in fp32.  d * sc * q is exact in
// fp32 for every type (<= 24 significant bits), so only the K-quant min subtraction rounds,
// once; bf16 / fp16 outputs are the round-to-nearest-even of that fp32 value.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include "gqk_common.h"
#include "gqk_internal.h"

namespace gqk {

__device__ __forceinline__ float f16_at(const uint8_t* p) {
  uint16_t b = (uint16_t)p[0] | ((uint16_t)p[1] << 8);
  return (float)__builtin_bit_cast(_Float16, b);
}

__device__ __forceinline__ void scale_min_k4(const uint8_t* s, int j, int& sc, int& m) {
  // gguf-plugin/gluon/kq_ref.py:17-27
  if (j < 4) {
    sc = s[j] & 63;
    m = s[j + 4] & 63;
  } else {
    sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
    m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
}

// The 32 fp32 weights of group g (0..7) of the raw 256-weight record at rec.
template <int T> __device__ void deq32(const uint8_t* rec, int g, float* w);

template <> __device__ void deq32<GQK_Q4_0>(const uint8_t* rec, int g, float* w) {
  const uint8_t* b = rec + 18 * g;
  float d = f16_at(b);
  for (int j = 0; j < 16; ++j) {
    w[j] = d * (float)((int)(b[2 + j] & 0xF) - 8);
    w[j + 16] = d * (float)((int)(b[2 + j] >> 4) - 8);
  }
}

template <> __device__ void deq32<GQK_IQ4_NL>(const uint8_t* rec, int g, float* w) {
  const uint8_t* b = rec + 18 * g;
  float d = f16_at(b);
  for (int j = 0; j < 16; ++j) {
    w[j] = d * (float)c_kvalues[b[2 + j] & 0xF];
    w[j + 16] = d * (float)c_kvalues[b[2 + j] >> 4];
  }
}

template <> __device__ void deq32<GQK_Q5_0>(const uint8_t* rec, int g, float* w) {
  const uint8_t* b = rec + 22 * g;
  float d = f16_at(b);
  uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
  for (int j = 0; j < 16; ++j) {
    int lo = (b[6 + j] & 0xF) | (((qh >> j) & 1) << 4);
    int hi = (b[6 + j] >> 4) | (((qh >> (j + 16)) & 1) << 4);
    w[j] = d * (float)(lo - 16);
    w[j + 16] = d * (float)(hi - 16);
  }
}

template <> __device__ void deq32<GQK_Q8_0>(const uint8_t* rec, int g, float* w) {
  const uint8_t* b = rec + 34 * g;
  float d = f16_at(b);
  for (int j = 0; j < 32; ++j) w[j] = d * (float)(int8_t)b[2 + j];
}

template <> __device__ void deq32<GQK_Q2_K>(const uint8_t* rec, int g, float* w) {
  // scales[16] | qs[64] | d | dmin; weight 128 h + 32 t + l = bits 2t of byte 32 h + l
  float d = f16_at(rec + 80), dmin = f16_at(rec + 82);
  int h = g >> 2, t = g & 3;
  for (int hf = 0; hf < 2; ++hf) {
    int sc = rec[8 * h + 2 * t + hf];
    float dl = d * (float)(sc & 0xF), ml = dmin * (float)(sc >> 4);
    for (int j = 0; j < 16; ++j) {
      int l = 16 * hf + j;
      int q = (rec[16 + 32 * h + l] >> (2 * t)) & 3;
      w[l] = dl * (float)q - ml;
    }
  }
}

template <> __device__ void deq32<GQK_Q3_K>(const uint8_t* rec, int g, float* w) {
  // hmask[32] | qs[64] | scales[12] | d   (kq_ref.py:40-56)
  float d = f16_at(rec + 108);
  const uint8_t* s = rec + 96;
  int h = g >> 2, jj = g & 3;
  for (int hf = 0; hf < 2; ++hf) {
    int i = 2 * g + hf;
    int lo = (s[i % 8] >> (4 * (i / 8))) & 0xF;
    int hi = (s[8 + i % 4] >> (2 * (i / 4))) & 3;
    float dl = d * (float)((lo | (hi << 4)) - 32);
    for (int j = 0; j < 16; ++j) {
      int l = 16 * hf + j;
      int hb = (rec[l] >> (4 * h + jj)) & 1;
      int q = ((rec[32 + 32 * h + l] >> (2 * jj)) & 3) - (hb ? 0 : 4);
      w[l] = dl * (float)q;
    }
  }
}

template <int T> __device__ __forceinline__ void deq32_q45k(const uint8_t* rec, int g, float* w) {
  // d | dmin | scales[12] | (qh[32]) | qs[128]   (q4k.py:5-20, kq_ref.py:57-68)
  float d = f16_at(rec), dmin = f16_at(rec + 2);
  int sc, m;
  scale_min_k4(rec + 4, g, sc, m);
  float dl = d * (float)sc, ml = dmin * (float)m;
  const uint8_t* qs = rec + (T == GQK_Q4_K ? 16 : 48);
  for (int p = 0; p < 32; ++p) {
    int q = (qs[32 * (g >> 1) + p] >> (4 * (g & 1))) & 0xF;
    if (T == GQK_Q5_K) q |= ((rec[16 + p] >> g) & 1) << 4;
    w[p] = dl * (float)q - ml;
  }
}
template <> __device__ void deq32<GQK_Q4_K>(const uint8_t* rec, int g, float* w) { deq32_q45k<GQK_Q4_K>(rec, g, w); }
template <> __device__ void deq32<GQK_Q5_K>(const uint8_t* rec, int g, float* w) { deq32_q45k<GQK_Q5_K>(rec, g, w); }

template <> __device__ void deq32<GQK_Q6_K>(const uint8_t* rec, int g, float* w) {
  // ql[128] | qh[64] | int8 scales[16] | d   (kq_ref.py:69-79)
  float d = f16_at(rec + 208);
  int h = g >> 2, t = g & 3;
  for (int hf = 0; hf < 2; ++hf) {
    float dl = d * (float)(int8_t)rec[192 + 8 * h + 2 * t + hf];
    for (int j = 0; j < 16; ++j) {
      int p = 16 * hf + j;
      int lo = (rec[64 * h + 32 * (t & 1) + p] >> (4 * (t >> 1))) & 0xF;
      int hi = (rec[128 + 32 * h + p] >> (2 * t)) & 3;
      w[p] = dl * (float)((lo | (hi << 4)) - 32);
    }
  }
}

template <> __device__ void deq32<GQK_IQ4_XS>(const uint8_t* rec, int g, float* w) {
  // d | scales_h u16 | scales_l[4] | qs[128]   (iq4xs.py:5-11)
  float d = f16_at(rec);
  int sh = rec[2] | (rec[3] << 8);
  int ls = ((rec[4 + g / 2] >> (4 * (g % 2))) & 0xF) | (((sh >> (2 * g)) & 3) << 4);
  float dl = d * (float)(ls - 32);
  const uint8_t* qs = rec + 8 + 16 * g;
  for (int j = 0; j < 16; ++j) {
    w[j] = dl * (float)c_kvalues[qs[j] & 0xF];
    w[j + 16] = dl * (float)c_kvalues[qs[j] >> 4];
  }
}

template <> __device__ void deq32<GQK_IQ3_S>(const uint8_t* rec, int g, float* w) {
  // d | qs[64] | qh[8] | signs[32] | scales[4]   (iq3s_tile_dequant.py:30-53)
  float d = f16_at(rec);
  int s = (rec[106 + g / 2] >> (4 * (g % 2))) & 0xF;
  float dl = d * (float)(1 + 2 * s);
  int qh = rec[66 + g];
  for (int l = 0; l < 4; ++l) {
    int sg = rec[74 + 4 * g + l];
    for (int half = 0; half < 2; ++half) {
      int idx = rec[2 + 8 * g + 2 * l + half] | ((qh << (8 - 2 * l - half)) & 256);
      uint32_t gw = c_iq3s_grid[idx];
      for (int k4 = 0; k4 < 4; ++k4) {
        int jj = 4 * half + k4;
        float v = dl * (float)((gw >> (8 * k4)) & 0xFF);
        w[8 * l + jj] = ((sg >> jj) & 1) ? -v : v;
      }
    }
  }
}

template <typename O> __device__ __forceinline__ O cvt_out(float v);
template <> __device__ __forceinline__ float cvt_out<float>(float v) { return v; }
// The fp32 value is made opaque before the narrowing conversion: otherwise the compiler may fuse
// the last multiply into the conversion (v_fma_mixlo_f16(a, b, +0)), which turns a -0.0 product
// (negative scale x zero quant, kept by gguf-py) into +0.0.
template <> __device__ __forceinline__ __bf16 cvt_out<__bf16>(float v) {
  asm volatile("" : "+v"(v));
  return (__bf16)v;
}
template <> __device__ __forceinline__ _Float16 cvt_out<_Float16>(float v) {
  asm volatile("" : "+v"(v));
  return (_Float16)v;
}

// One thread per (row, group of 32 weights).  VEC: the output rows are 16-byte aligned, so the
// 32 values go out as 16-byte stores (64 or 128 contiguous bytes per thread).
template <int T, typename O, bool VEC>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ W, int64_t stride, int64_t n,
                                                      int64_t K, O* __restrict__ out, int64_t ldo, int rec) {
  int64_t ng = K / 32;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n * ng) return;
  int64_t row = i / ng, gg = i % ng;
  int64_t kb = gg / 8;
  int g = (int)(gg % 8);
  const uint8_t* recp = W + row * stride + kb * rec;
  float w[32];
  deq32<T>(recp, g, w);
  O* o = out + row * ldo + gg * 32;
  if constexpr (VEC) {
    constexpr int PER = 16 / sizeof(O);   // values per 16-byte store
    uint4* ov = (uint4*)o;
#pragma unroll
    for (int v = 0; v < 32 / PER; ++v) {
      O c[PER];
#pragma unroll
      for (int j = 0; j < PER; ++j) c[j] = cvt_out<O>(w[v * PER + j]);
      ov[v] = __builtin_bit_cast(uint4, c);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 32; ++j) o[j] = cvt_out<O>(w[j]);
  }
}

template <int T>
static int launch_dequant_t(const void* W, int64_t stride, int64_t n, int64_t K, void* out, int64_t ldo, int dtype,
                            hipStream_t st) {
  const int rec = gqk_layout<T>::REC;
  int64_t total = n * (K / 32);
  dim3 grid((unsigned)((total + 255) / 256)), block(256);
  const int esz = dtype == 0 ? 4 : 2;
  const bool vec = ((uintptr_t)out % 16 == 0) && ((ldo * esz) % 16 == 0);
#define L(O, V) hipLaunchKernelGGL((dequant_kernel<T, O, V>), grid, block, 0, st, (const uint8_t*)W, stride, n, K, (O*)out, ldo, rec)
  if (dtype == 0) {
    if (vec) L(float, true); else L(float, false);
  } else if (dtype == 1) {
    if (vec) L(__bf16, true); else L(__bf16, false);
  } else {
    if (vec) L(_Float16, true); else L(_Float16, false);
  }
#undef L
  return GQK_OK;
}

int launch_dequant(int type, const void* W, int64_t stride, int64_t n, int64_t K, void* out, int64_t ldo, int dtype,
                   hipStream_t st) {
  switch (type) {
#define C(T) case T: return launch_dequant_t<T>(W, stride, n, K, out, ldo, dtype, st);
    C(GQK_Q4_0) C(GQK_Q5_0) C(GQK_Q8_0) C(GQK_Q2_K) C(GQK_Q3_K) C(GQK_Q4_K) C(GQK_Q5_K) C(GQK_Q6_K)
    C(GQK_IQ4_NL) C(GQK_IQ3_S) C(GQK_IQ4_XS)
#undef C
  }
  return GQK_ERR_TYPE;
}

// ---------------------------------------------------------------------------------------------
// Repack raw rows <-> tiles.  One workgroup per chunk (tile t, super-block kb): 64 rows x REC bytes.
// Repack stages the chunk's 64 raw records in LDS (2-byte loads along each row when the rows are
// 2-byte aligned, REC being even) and writes the chunk plane-major with 16-byte stores; unrepack
// loads the chunk with 16-byte loads, scatters it into the 64 raw records in LDS and writes them
// back row by row.  Rows past n are zeros in the tiles (repack) and are not written (unrepack).
// Each byte crosses HBM once in each direction.  The plane table is a compile-time constant per
// type, so the index arithmetic folds to shifts and multiplies by constants.

// raw byte of byte j of plane p (segments of equal length concatenated)
template <int T, int P>
__device__ __forceinline__ int raw_of(int j) {
  constexpr gqk_plane pl = gqk_planes<T>::v.planes[P];
  return pl.seg_off + (j / pl.seg_len) * pl.seg_stride + j % pl.seg_len;
}

template <int T, int P>
__device__ __forceinline__ constexpr int plane_off() {
  int o = 0;
  for (int p = 0; p < P; ++p) o += gqk_planes<T>::v.planes[p].size;
  return o;
}

// visits the 16-byte words of plane P of a chunk: f(word index in the chunk, row of byte i, raw
// byte of byte i) for i = 0..15 through g(i) -> (r, b)
template <int T, int P, class F>
__device__ __forceinline__ void plane_words(int tid, F&& f) {
  constexpr gqk_plane pl = gqk_planes<T>::v.planes[P];
  constexpr int W = gqk_col_width(pl.size), poff = plane_off<T, P>();
  for (int w = tid; w < 4 * pl.size; w += 256) {     // 64 rows * size bytes / 16
    const int x = 16 * w, col = x / (64 * W), rem = x % (64 * W);
    f(4 * poff + w, [&](int i, int& r, int& b) {
      r = (rem + i) / W;
      b = raw_of<T, P>(col * W + (rem + i) % W);
    });
  }
}

template <int T, int P = 0, class F>
__device__ __forceinline__ void every_plane_word(int tid, F&& f) {
  if constexpr (P < gqk_planes<T>::v.nplanes) {
    plane_words<T, P>(tid, f);
    every_plane_word<T, P + 1>(tid, f);
  }
}

// ---- Q6_K: the six-bit values re-packed per scale group (gqk_q6_pos) <-> GGUF's ql / qh ----------
// q of weight k of a raw record (ql[128] | qh[64], kq_ref.py:69-79): 4 low bits from ql, 2 from qh
__device__ __forceinline__ uint32_t q6_raw(const uint8_t* rec, int k) {
  const int hh = k >> 7, l = k & 127;
  const uint32_t lo = (rec[64 * hh + (l & 63)] >> (4 * (l >> 6))) & 0xF;
  const uint32_t hi = (rec[128 + 32 * hh + (l & 31)] >> (2 * (l >> 5))) & 3;
  return lo | (hi << 4);
}
// q of weight k of a re-packed record
__device__ __forceinline__ uint32_t q6_packed(const uint8_t* rec, int k) {
  const int g = k >> 4, j = k & 15;
  if (j < 12) return rec[gqk_q6_pos(g, j >> 2, j & 3)] & 63;
  uint32_t v = 0;
#pragma unroll
  for (int m = 0; m < 3; ++m) v |= (uint32_t)(rec[gqk_q6_pos(g, m, j - 12)] >> 6) << (2 * m);
  return v;
}
// In place on the chunk's 64 records in LDS (raw[row][REC]): TO_PACKED re-packs bytes 0..191 of
// every record, else restores GGUF's ql / qh.  Every thread computes its share into registers
// before any is written (barriers between), so the pass reads only the old layout.
template <bool TO_PACKED>
__device__ __forceinline__ void q6_convert(uint8_t* raw, int tid) {
  constexpr int REC = 210, PER = 64 * 48 / 256;   // 48 dwords of 192 bytes per row, 12 per thread
  uint32_t v[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int it = tid + 256 * k, r = it / 48, w = it % 48;
    const uint8_t* rec = raw + r * REC;
    uint32_t d = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int b = 4 * w + i;   // output byte
      uint32_t byte;
      if (TO_PACKED) {             // byte b = gqk_q6_pos(g, m, i'): low 6 bits of q[16 g + 4 m + i'], top 2 of q[16 g + 12 + i']
        const int col = b >> 4, a = col / 3, m = col % 3, g = 4 * a + ((b >> 2) & 3), ii = b & 3;
        byte = (q6_raw(rec, 16 * g + 4 * m + ii) & 63) | (((q6_raw(rec, 16 * g + 12 + ii) >> (2 * m)) & 3) << 6);
      } else if (b < 128) {        // ql byte b: low nibbles of weights 128 hh + p and 128 hh + 64 + p
        const int hh = b >> 6, p = b & 63;
        byte = (q6_packed(rec, 128 * hh + p) & 15) | ((q6_packed(rec, 128 * hh + 64 + p) & 15) << 4);
      } else {                     // qh byte: the high pairs of weights 128 hh + p + 32 t
        const int hh = (b - 128) >> 5, p = (b - 128) & 31;
        byte = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) byte |= (q6_packed(rec, 128 * hh + p + 32 * t) >> 4) << (2 * t);
      }
      d |= byte << (8 * i);
    }
    v[k] = d;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int it = tid + 256 * k, r = it / 48, w = it % 48;
    uint8_t* rec = raw + r * REC;
#pragma unroll
    for (int i = 0; i < 4; ++i) rec[4 * w + i] = (uint8_t)(v[k] >> (8 * i));
  }
  __syncthreads();
}

// The 64 raw records of a chunk from its plane-major words (16-byte loads), into raw[row][REC] in
// LDS (Q6_K's six-bit values converted back to ql / qh before the function returns, unless
// Q6_PACKED: then its first 192 bytes stay in the re-packed order).
template <int T, bool Q6_PACKED = false>
__device__ __forceinline__ void chunk_to_raw(const uint4* __restrict__ in, uint8_t* raw, int tid) {
  constexpr int REC = gqk_planes<T>::v.rec;
  auto scatter = [&](int wi, auto&& at) {
    const uint4 q = in[wi];
    const uint32_t v[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      int r, b;
      at(i, r, b);
      raw[r * REC + b] = (uint8_t)(v[i >> 2] >> (8 * (i & 3)));
    }
  };
  every_plane_word<T>(tid, scatter);
  if constexpr (T == GQK_Q6_K && !Q6_PACKED) {
    __syncthreads();
    q6_convert<false>(raw, tid);
  }
}

// deq32<Q6_K> on a record whose six-bit values are in the re-packed order (gqk_q6_pos): the same
// weights and the same fp32 bits, without restoring ql / qh first.
__device__ __forceinline__ void deq32_q6_packed(const uint8_t* rec, int g, float* w) {
  const float d = f16_at(rec + 208);
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const int g16 = 2 * g + hf;
    const float dl = d * (float)(int8_t)rec[192 + g16];
    uint32_t top[4] = {0, 0, 0, 0};
#pragma unroll
    for (int m = 0; m < 3; ++m)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t b = rec[gqk_q6_pos(g16, m, i)];
        w[16 * hf + 4 * m + i] = dl * (float)((int)(b & 63) - 32);
        top[i] |= (b >> 6) << (2 * m);
      }
#pragma unroll
    for (int i = 0; i < 4; ++i) w[16 * hf + 12 + i] = dl * (float)((int)top[i] - 32);
  }
}

template <int T, bool TO_TILES, bool WIDE>
__global__ __launch_bounds__(256) void repack_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                     int64_t stride, int64_t n, int64_t nb) {
  constexpr gqk_type_c ty = gqk_planes<T>::v;
  constexpr int REC = ty.rec, CB = 64 * REC;          // chunk bytes (a multiple of 64)
  __shared__ __attribute__((aligned(16))) uint8_t raw[CB + 16];   // the 64 raw records, [row][REC]
  const int tid = threadIdx.x;
  const int64_t chunk = blockIdx.x, kb = chunk % nb, tile = chunk / nb;
  const int64_t row0 = tile * 64;
  if (TO_TILES) {
    const uint8_t* rows = src + row0 * stride + kb * REC;
    if (WIDE) {
      for (int i = tid; i < CB / 2; i += 256) {
        const int r = i / (REC / 2), h = i % (REC / 2);
        const uint16_t v = row0 + r < n ? *(const uint16_t*)(rows + r * stride + 2 * h) : (uint16_t)0;
        *(uint16_t*)(raw + r * REC + 2 * h) = v;
      }
    } else {
      for (int i = tid; i < CB; i += 256) {
        const int r = i / REC, b = i % REC;
        raw[i] = row0 + r < n ? rows[r * stride + b] : (uint8_t)0;
      }
    }
    __syncthreads();
    if constexpr (T == GQK_Q6_K) q6_convert<true>(raw, tid);
    uint4* out = (uint4*)(dst + chunk * CB);
    auto gather = [&](int wi, auto&& at) {
      uint32_t v[4] = {0, 0, 0, 0};
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        int r, b;
        at(i, r, b);
        v[i >> 2] |= (uint32_t)raw[r * REC + b] << (8 * (i & 3));
      }
      out[wi] = make_uint4(v[0], v[1], v[2], v[3]);
    };
    every_plane_word<T>(tid, gather);
  } else {
    chunk_to_raw<T>((const uint4*)(src + chunk * CB), raw, tid);
    __syncthreads();
    uint8_t* rows = dst + row0 * stride + kb * REC;
    if (WIDE) {
      for (int i = tid; i < CB / 2; i += 256) {
        const int r = i / (REC / 2), h = i % (REC / 2);
        if (row0 + r < n) *(uint16_t*)(rows + r * stride + 2 * h) = *(const uint16_t*)(raw + r * REC + 2 * h);
      }
    } else {
      for (int i = tid; i < CB; i += 256) {
        const int r = i / REC, b = i % REC;
        if (row0 + r < n) rows[r * stride + b] = raw[i];
      }
    }
  }
}

template <int T>
static void launch_repack_t(bool to_tiles, bool wide, dim3 grid, hipStream_t st, const uint8_t* s, uint8_t* d,
                            int64_t stride, int64_t n, int64_t nb) {
  const dim3 block(256);
  if (to_tiles) {
    if (wide) hipLaunchKernelGGL((repack_kernel<T, true, true>), grid, block, 0, st, s, d, stride, n, nb);
    else hipLaunchKernelGGL((repack_kernel<T, true, false>), grid, block, 0, st, s, d, stride, n, nb);
  } else {
    if (wide) hipLaunchKernelGGL((repack_kernel<T, false, true>), grid, block, 0, st, s, d, stride, n, nb);
    else hipLaunchKernelGGL((repack_kernel<T, false, false>), grid, block, 0, st, s, d, stride, n, nb);
  }
}

int launch_repack(int type, const void* W, int64_t stride, int64_t n, int64_t K, void* tiles, bool to_tiles,
                  hipStream_t st) {
  const gqk_type* t = gqk_type_get(type);
  if (!t) return GQK_ERR_TYPE;
  const int64_t nb = K / 256, ntiles = (n + 63) / 64;
  const int64_t chunks = ntiles * nb;
  if (chunks == 0) return GQK_OK;
  if (chunks >= ((int64_t)1 << 31)) return GQK_ERR_SHAPE;
  // 2-byte accesses along the raw rows when every row starts 2-byte aligned (every REC is even)
  const bool wide = (t->rec % 2 == 0) && (stride % 2 == 0) && ((uintptr_t)W % 2 == 0);
  const dim3 grid((unsigned)chunks);
  const uint8_t* s = (const uint8_t*)(to_tiles ? W : tiles);
  uint8_t* d = (uint8_t*)(to_tiles ? tiles : W);
  switch (type) {
#define C(T) case T: launch_repack_t<T>(to_tiles, wide, grid, st, s, d, stride, n, nb); return GQK_OK;
    C(GQK_Q4_0) C(GQK_Q5_0) C(GQK_Q8_0) C(GQK_Q2_K) C(GQK_Q3_K) C(GQK_Q4_K) C(GQK_Q5_K) C(GQK_Q6_K)
    C(GQK_IQ4_NL) C(GQK_IQ3_S) C(GQK_IQ4_XS)
#undef C
  }
  return GQK_ERR_TYPE;
}

// ---------------------------------------------------------------------------------------------
// Dequantize straight from the tiles: one workgroup per chunk (tile t, super-block kb) gathers the
// chunk's planes back into its 64 raw records in LDS (as the unrepack does), then every thread
// decodes (row, 32-weight group) items from LDS with the same deq32 as the raw-row dequantizer
// and writes them to the output row: each tile byte is read once, no raw-row temporary.
template <int T, typename O, bool VEC>
__global__ __launch_bounds__(256) void tile_dequant_kernel(const uint8_t* __restrict__ tiles, int64_t n, int64_t nb,
                                                           O* __restrict__ out, int64_t ldo) {
  constexpr int REC = gqk_planes<T>::v.rec, CB = 64 * REC;
  __shared__ __attribute__((aligned(16))) uint8_t raw[CB + 16];
  const int tid = threadIdx.x;
  const int64_t chunk = blockIdx.x, kb = chunk % nb, tile = chunk / nb;
  chunk_to_raw<T, true>((const uint4*)(tiles + chunk * CB), raw, tid);
  __syncthreads();
  for (int it = tid; it < 64 * 8; it += 256) {   // consecutive threads: consecutive groups of a row
    const int r = it >> 3, g = it & 7;
    const int64_t row = tile * 64 + r;
    if (row >= n) continue;
    float w[32];
    if constexpr (T == GQK_Q6_K) deq32_q6_packed(raw + r * REC, g, w);
    else deq32<T>(raw + r * REC, g, w);
    O* o = out + row * ldo + kb * 256 + g * 32;
    if constexpr (VEC) {
      constexpr int PER = 16 / sizeof(O);
      uint4* ov = (uint4*)o;
#pragma unroll
      for (int v = 0; v < 32 / PER; ++v) {
        O c[PER];
#pragma unroll
        for (int j = 0; j < PER; ++j) c[j] = cvt_out<O>(w[v * PER + j]);
        ov[v] = __builtin_bit_cast(uint4, c);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 32; ++j) o[j] = cvt_out<O>(w[j]);
    }
  }
}

template <int T>
static int launch_tile_dequant_t(const void* tiles, int64_t n, int64_t K, void* out, int64_t ldo, int dtype,
                                 hipStream_t st) {
  const int64_t nb = K / 256, chunks = (n + 63) / 64 * nb;
  if (chunks == 0) return GQK_OK;
  if (chunks >= ((int64_t)1 << 31)) return GQK_ERR_SHAPE;
  const dim3 grid((unsigned)chunks), block(256);
  const int esz = dtype == 0 ? 4 : 2;
  const bool vec = ((uintptr_t)out % 16 == 0) && ((ldo * esz) % 16 == 0);
  const uint8_t* t = (const uint8_t*)tiles;
#define L(O, V) hipLaunchKernelGGL((tile_dequant_kernel<T, O, V>), grid, block, 0, st, t, n, nb, (O*)out, ldo)
  if (dtype == 0) {
    if (vec) L(float, true); else L(float, false);
  } else if (dtype == 1) {
    if (vec) L(__bf16, true); else L(__bf16, false);
  } else {
    if (vec) L(_Float16, true); else L(_Float16, false);
  }
#undef L
  return GQK_OK;
}

int launch_tile_dequant(int type, const void* tiles, int64_t n, int64_t K, void* out, int64_t ldo, int dtype,
                        hipStream_t st) {
  switch (type) {
#define C(T) case T: return launch_tile_dequant_t<T>(tiles, n, K, out, ldo, dtype, st);
    C(GQK_Q4_0) C(GQK_Q5_0) C(GQK_Q8_0) C(GQK_Q2_K) C(GQK_Q3_K) C(GQK_Q4_K) C(GQK_Q5_K) C(GQK_Q6_K)
    C(GQK_IQ4_NL) C(GQK_IQ3_S) C(GQK_IQ4_XS)
#undef C
  }
  return GQK_ERR_TYPE;
}

}  // namespace gqk
