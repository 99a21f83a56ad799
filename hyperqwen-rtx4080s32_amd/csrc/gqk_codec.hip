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

// One thread per (row, group of 32 weights).
template <int T, typename O>
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
#pragma unroll
  for (int j = 0; j < 32; ++j) o[j] = cvt_out<O>(w[j]);
}

template <int T>
static int launch_dequant_t(const void* W, int64_t stride, int64_t n, int64_t K, void* out, int64_t ldo, int dtype,
                            hipStream_t st) {
  const int rec = gqk_layout<T>::REC;
  int64_t total = n * (K / 32);
  dim3 grid((unsigned)((total + 255) / 256)), block(256);
  if (dtype == 0)
    hipLaunchKernelGGL((dequant_kernel<T, float>), grid, block, 0, st, (const uint8_t*)W, stride, n, K, (float*)out, ldo, rec);
  else if (dtype == 1)
    hipLaunchKernelGGL((dequant_kernel<T, __bf16>), grid, block, 0, st, (const uint8_t*)W, stride, n, K, (__bf16*)out, ldo, rec);
  else
    hipLaunchKernelGGL((dequant_kernel<T, _Float16>), grid, block, 0, st, (const uint8_t*)W, stride, n, K, (_Float16*)out, ldo, rec);
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
// Repack raw rows <-> tiles.  One thread per (tile row, super-block): the record's bytes are
// moved plane by plane; rows past n are written as zeros (repack) or skipped (unrepack).

struct PlaneArgs {
  int nplanes;
  int size[GQK_MAX_PLANES];
  int nseg[GQK_MAX_PLANES];
  int seg_off[GQK_MAX_PLANES];
  int seg_len[GQK_MAX_PLANES];
  int seg_stride[GQK_MAX_PLANES];
};

template <bool TO_TILES>
__global__ __launch_bounds__(256) void repack_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                     int64_t stride, int64_t n, int64_t nb, int rec, PlaneArgs pa) {
  int64_t ntiles = (n + 63) / 64;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= ntiles * 64 * nb) return;
  // i = ((tile * nb) + kb) * 64 + r: consecutive threads take consecutive rows of one chunk
  int r = (int)(i % 64);
  int64_t chunk = i / 64;
  int64_t kb = chunk % nb, tile = chunk / nb;
  int64_t row = tile * 64 + r;
  uint8_t* tbase = (uint8_t*)(TO_TILES ? dst : src) + chunk * 64 * rec;
  bool valid = row < n;
  const uint8_t* rrec = (TO_TILES ? src : dst) + row * stride + kb * rec;
  int poff = 0;
  for (int p = 0; p < pa.nplanes; ++p) {
    const int W = gqk_col_width(pa.size[p]);
    uint8_t* tp = tbase + 64 * poff + r * W;     // byte j of the row: tp + (j / W) * 64 * W + j % W
    int j = 0;
    for (int sgi = 0; sgi < pa.nseg[p]; ++sgi) {
      int so = pa.seg_off[p] + sgi * pa.seg_stride[p];
      for (int b = 0; b < pa.seg_len[p]; ++b, ++j) {
        uint8_t* tj = tp + (j / W) * 64 * W + j % W;
        if (TO_TILES)
          *tj = valid ? rrec[so + b] : (uint8_t)0;
        else if (valid)
          ((uint8_t*)rrec)[so + b] = *tj;
      }
    }
    poff += pa.size[p];
  }
}

int launch_repack(int type, const void* W, int64_t stride, int64_t n, int64_t K, void* tiles, bool to_tiles,
                  hipStream_t st) {
  const gqk_type* t = gqk_type_get(type);
  if (!t) return GQK_ERR_TYPE;
  PlaneArgs pa{};
  pa.nplanes = t->nplanes;
  for (int p = 0; p < t->nplanes; ++p) {
    pa.size[p] = t->planes[p].size;
    pa.nseg[p] = t->planes[p].nseg;
    pa.seg_off[p] = t->planes[p].seg_off;
    pa.seg_len[p] = t->planes[p].seg_len;
    pa.seg_stride[p] = t->planes[p].seg_stride;
  }
  int64_t nb = K / 256, ntiles = (n + 63) / 64;
  int64_t total = ntiles * 64 * nb;
  if (total == 0) return GQK_OK;
  dim3 grid((unsigned)((total + 255) / 256)), block(256);
  if (to_tiles)
    hipLaunchKernelGGL(repack_kernel<true>, grid, block, 0, st, (const uint8_t*)W, (uint8_t*)tiles, stride, n, nb, t->rec, pa);
  else
    hipLaunchKernelGGL(repack_kernel<false>, grid, block, 0, st, (const uint8_t*)tiles, (uint8_t*)W, stride, n, nb, t->rec, pa);
  return GQK_OK;
}

}  // namespace gqk
