// gqk_gemm.hip - the grouped dequant-GEMM (batch rows M > 32, the prefill regime).
//
// Replaces the reference's prefill paths: the wide int8 forms of the grouped kernel and, for
// Q4_K / Q5_K, dequantize_tiles + cuBLAS bf16 (gguf-plugin/gluon/interface.py:159-188,
// gguf-plugin/gluon/tiles.py:141-149).  Here one kernel does both: each workgroup owns a
// BM x 128 output tile (BM tokens, two 64-row weight tiles of one shard), walks K in steps of
// 64, decodes the step's weights to bf16 in LDS (bf16 = round-to-nearest-even of the exact
// fp32 gguf-py value), stages the activations beside them, and runs v_mfma_f32_32x32x16_bf16
// with fp32 accumulation.  Global loads of step s+1 are in flight while step s multiplies.
#include <hip/hip_runtime.h>
#include "gqk_common.h"
#include "gqk_internal.h"

namespace gqk {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float g_h2f(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits16 & 0xFFFF));
}
__device__ __forceinline__ uint32_t g_bf16x2(float lo, float hi) {
  typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
  v2bf p;
  p[0] = (__bf16)lo;
  p[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, p);
}
__device__ __forceinline__ uint32_t g_byte(const uint32_t* w, int b) { return (w[b >> 2] >> (8 * (b & 3))) & 0xFF; }

template <int N>
__device__ __forceinline__ void gld(uint32_t* dst, const uint8_t* p) {
  if constexpr (N % 16 == 0) {
#pragma unroll
    for (int i = 0; i < N / 16; ++i) {
      uint4 v = *(const uint4*)(p + 16 * i);
      dst[4 * i] = v.x; dst[4 * i + 1] = v.y; dst[4 * i + 2] = v.z; dst[4 * i + 3] = v.w;
    }
  } else if constexpr (N == 8) {
    uint2 v = *(const uint2*)p;
    dst[0] = v.x; dst[1] = v.y;
  } else if constexpr (N == 4) {
    dst[0] = *(const uint32_t*)p;
  } else if constexpr (N == 12) {
    const uint32_t* q = (const uint32_t*)p;
    dst[0] = q[0]; dst[1] = q[1]; dst[2] = q[2];
  } else {
    static_assert(N == 2, "plane slice size");
    dst[0] = *(const uint16_t*)p;
  }
}

// 16-byte column `col` of row r in a plane with 16-byte columns (column-major: (col * 64 + r) * 16)
__device__ __forceinline__ const uint8_t* col16(const uint8_t* plane, int r, int col) { return plane + (col * 64 + r) * 16; }

// Per-type decode of one group of 32 consecutive weights (g = 0..7 of a super-block) of row r
// to 16 dwords of bf16 pairs in natural k order.  load() issues the global loads, out() decodes.
template <int T> struct GDec;

template <> struct GDec<GQK_Q4_0> {
  uint32_t qs[4], d;
  __device__ void load(const uint8_t* c, int r, int g) { gld<16>(qs, col16(c, r, g)); gld<2>(&d, c + 64 * 128 + r * 16 + 2 * g); }
  __device__ void out(uint32_t* o) const {
    float dd = g_h2f(d);
#pragma unroll
    for (int j = 0; j < 16; j += 2) {
      uint32_t b0 = g_byte(qs, j), b1 = g_byte(qs, j + 1);
      o[j / 2] = g_bf16x2(dd * (float)((int)(b0 & 0xF) - 8), dd * (float)((int)(b1 & 0xF) - 8));
      o[8 + j / 2] = g_bf16x2(dd * (float)((int)(b0 >> 4) - 8), dd * (float)((int)(b1 >> 4) - 8));
    }
  }
};

template <> struct GDec<GQK_IQ4_NL> {
  uint32_t qs[4], d;
  __device__ void load(const uint8_t* c, int r, int g) { gld<16>(qs, col16(c, r, g)); gld<2>(&d, c + 64 * 128 + r * 16 + 2 * g); }
  __device__ void out(uint32_t* o) const {
    float dd = g_h2f(d);
#pragma unroll
    for (int j = 0; j < 16; j += 2) {
      uint32_t b0 = g_byte(qs, j), b1 = g_byte(qs, j + 1);
      o[j / 2] = g_bf16x2(dd * (float)c_kvalues[b0 & 0xF], dd * (float)c_kvalues[b1 & 0xF]);
      o[8 + j / 2] = g_bf16x2(dd * (float)c_kvalues[b0 >> 4], dd * (float)c_kvalues[b1 >> 4]);
    }
  }
};

template <> struct GDec<GQK_Q5_0> {
  uint32_t qs[4], qh, d;
  __device__ void load(const uint8_t* c, int r, int g) {
    gld<16>(qs, col16(c, r, g)); gld<4>(&qh, col16(c + 64 * 128, r, g >> 2) + 4 * (g & 3)); gld<2>(&d, c + 64 * 160 + r * 16 + 2 * g);
  }
  __device__ void out(uint32_t* o) const {
    float dd = g_h2f(d);
#pragma unroll
    for (int j = 0; j < 16; j += 2) {
      uint32_t b0 = g_byte(qs, j), b1 = g_byte(qs, j + 1);
      int l0 = (b0 & 0xF) | (((qh >> j) & 1) << 4), l1 = (b1 & 0xF) | (((qh >> (j + 1)) & 1) << 4);
      int h0 = (b0 >> 4) | (((qh >> (j + 16)) & 1) << 4), h1 = (b1 >> 4) | (((qh >> (j + 17)) & 1) << 4);
      o[j / 2] = g_bf16x2(dd * (float)(l0 - 16), dd * (float)(l1 - 16));
      o[8 + j / 2] = g_bf16x2(dd * (float)(h0 - 16), dd * (float)(h1 - 16));
    }
  }
};

template <> struct GDec<GQK_Q8_0> {
  uint32_t qs[8], d;
  __device__ void load(const uint8_t* c, int r, int g) { gld<16>(qs, col16(c, r, 2 * g)); gld<16>(qs + 4, col16(c, r, 2 * g + 1)); gld<2>(&d, c + 64 * 256 + r * 16 + 2 * g); }
  __device__ void out(uint32_t* o) const {
    float dd = g_h2f(d);
#pragma unroll
    for (int j = 0; j < 32; j += 2)
      o[j / 2] = g_bf16x2(dd * (float)(int8_t)g_byte(qs, j), dd * (float)(int8_t)g_byte(qs, j + 1));
  }
};

template <> struct GDec<GQK_Q2_K> {
  uint32_t qs[8], sc, dd;
  int t;
  __device__ void load(const uint8_t* c, int r, int g) {
    int h = g >> 2;
    t = g & 3;
    gld<16>(qs, col16(c, r, 2 * h));
    gld<16>(qs + 4, col16(c, r, 2 * h + 1));
    gld<2>(&sc, c + 64 * 64 + r * 16 + 2 * g);
    gld<4>(&dd, c + 64 * 80 + r * 4);
  }
  __device__ void out(uint32_t* o) const {
    float d = g_h2f(dd), dmin = g_h2f(dd >> 16);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      uint32_t sb = (sc >> (8 * hf)) & 0xFF;
      float dl = d * (float)(sb & 0xF), ml = dmin * (float)(sb >> 4);
#pragma unroll
      for (int j = 0; j < 16; j += 2) {
        int l = 16 * hf + j;
        float w0 = dl * (float)((g_byte(qs, l) >> (2 * t)) & 3) - ml;
        float w1 = dl * (float)((g_byte(qs, l + 1) >> (2 * t)) & 3) - ml;
        o[l / 2] = g_bf16x2(w0, w1);
      }
    }
  }
};

template <> struct GDec<GQK_Q3_K> {
  uint32_t qs[8], hm[8], sb[3], d;
  int g;
  __device__ void load(const uint8_t* c, int r, int g_) {
    g = g_;
    gld<16>(qs, col16(c, r, 2 * (g >> 2)));
    gld<16>(qs + 4, col16(c, r, 2 * (g >> 2) + 1));
    gld<16>(hm, col16(c + 64 * 64, r, 0));
    gld<16>(hm + 4, col16(c + 64 * 64, r, 1));
    const uint32_t* p = (const uint32_t*)(c + 64 * 96);   // three 4-byte columns
    sb[0] = p[r]; sb[1] = p[64 + r]; sb[2] = p[128 + r];
    gld<2>(&d, c + 64 * 108 + r * 2);
  }
  __device__ void out(uint32_t* o) const {
    int n = g >> 2, jj = g & 3;
    float dd = g_h2f(d);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      int i = 2 * g + hf;
      int lo = (g_byte(sb, i % 8) >> (4 * (i / 8))) & 0xF;
      int hi = (g_byte(sb, 8 + i % 4) >> (2 * (i / 4))) & 3;
      float dl = dd * (float)((lo | (hi << 4)) - 32);
#pragma unroll
      for (int j = 0; j < 16; j += 2) {
        int l = 16 * hf + j;
        int q0 = ((g_byte(qs, l) >> (2 * jj)) & 3) - (((g_byte(hm, l) >> (4 * n + jj)) & 1) ? 0 : 4);
        int q1 = ((g_byte(qs, l + 1) >> (2 * jj)) & 3) - (((g_byte(hm, l + 1) >> (4 * n + jj)) & 1) ? 0 : 4);
        o[l / 2] = g_bf16x2(dl * (float)q0, dl * (float)q1);
      }
    }
  }
};

__device__ __forceinline__ void g_scale_min_k4(const uint32_t* S, int j, int& sc, int& m) {
  if (j < 4) {
    sc = g_byte(S, j) & 63;
    m = g_byte(S, j + 4) & 63;
  } else {
    sc = (g_byte(S, j + 4) & 0xF) | ((g_byte(S, j - 4) >> 6) << 4);
    m = (g_byte(S, j + 4) >> 4) | ((g_byte(S, j) >> 6) << 4);
  }
}

template <> struct GDec<GQK_Q4_K> {
  uint32_t qs[8], hdr[4];
  int g;
  __device__ void load(const uint8_t* c, int r, int g_) {
    g = g_;
    gld<16>(qs, col16(c, r, 2 * (g >> 1)));
    gld<16>(qs + 4, col16(c, r, 2 * (g >> 1) + 1));
    gld<16>(hdr, c + 64 * 128 + r * 16);
  }
  __device__ void out(uint32_t* o) const {
    int sc, m;
    g_scale_min_k4(hdr + 1, g, sc, m);
    float dl = g_h2f(hdr[0]) * (float)sc, ml = g_h2f(hdr[0] >> 16) * (float)m;
    const int sh = 4 * (g & 1);
#pragma unroll
    for (int p = 0; p < 32; p += 2)
      o[p / 2] = g_bf16x2(dl * (float)((g_byte(qs, p) >> sh) & 0xF) - ml, dl * (float)((g_byte(qs, p + 1) >> sh) & 0xF) - ml);
  }
};

template <> struct GDec<GQK_Q5_K> {
  uint32_t qs[8], qh[8], hdr[4];
  int g;
  __device__ void load(const uint8_t* c, int r, int g_) {
    g = g_;
    gld<16>(qs, col16(c, r, 2 * (g >> 1)));
    gld<16>(qs + 4, col16(c, r, 2 * (g >> 1) + 1));
    gld<16>(qh, col16(c + 64 * 128, r, 0));
    gld<16>(qh + 4, col16(c + 64 * 128, r, 1));
    gld<16>(hdr, c + 64 * 160 + r * 16);
  }
  __device__ void out(uint32_t* o) const {
    int sc, m;
    g_scale_min_k4(hdr + 1, g, sc, m);
    float dl = g_h2f(hdr[0]) * (float)sc, ml = g_h2f(hdr[0] >> 16) * (float)m;
    const int sh = 4 * (g & 1);
#pragma unroll
    for (int p = 0; p < 32; p += 2) {
      int q0 = ((g_byte(qs, p) >> sh) & 0xF) | (((g_byte(qh, p) >> g) & 1) << 4);
      int q1 = ((g_byte(qs, p + 1) >> sh) & 0xF) | (((g_byte(qh, p + 1) >> g) & 1) << 4);
      o[p / 2] = g_bf16x2(dl * (float)q0 - ml, dl * (float)q1 - ml);
    }
  }
};

template <> struct GDec<GQK_Q6_K> {
  uint32_t ql[8], qh[8], sc, d;
  int g;
  __device__ void load(const uint8_t* c, int r, int g_) {
    g = g_;
    int h = g >> 2, t = g & 3;
    gld<16>(ql, col16(c, r, 4 * h + 2 * (t & 1)));
    gld<16>(ql + 4, col16(c, r, 4 * h + 2 * (t & 1) + 1));
    gld<16>(qh, col16(c + 64 * 128, r, 2 * h));
    gld<16>(qh + 4, col16(c + 64 * 128, r, 2 * h + 1));
    gld<2>(&sc, c + 64 * 192 + r * 16 + 2 * g);
    gld<2>(&d, c + 64 * 208 + r * 2);
  }
  __device__ void out(uint32_t* o) const {
    int t = g & 3;
    float dd = g_h2f(d);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      float dl = dd * (float)(int8_t)((sc >> (8 * hf)) & 0xFF);
#pragma unroll
      for (int j = 0; j < 16; j += 2) {
        int p = 16 * hf + j;
        int q0 = (((g_byte(ql, p) >> (4 * (t >> 1))) & 0xF) | (((g_byte(qh, p) >> (2 * t)) & 3) << 4)) - 32;
        int q1 = (((g_byte(ql, p + 1) >> (4 * (t >> 1))) & 0xF) | (((g_byte(qh, p + 1) >> (2 * t)) & 3) << 4)) - 32;
        o[p / 2] = g_bf16x2(dl * (float)q0, dl * (float)q1);
      }
    }
  }
};

template <> struct GDec<GQK_IQ4_XS> {
  uint32_t qs[4], hdr[2];
  int g;
  __device__ void load(const uint8_t* c, int r, int g_) {
    g = g_;
    gld<16>(qs, col16(c, r, g));
    gld<8>(hdr, c + 64 * 128 + r * 8);
  }
  __device__ void out(uint32_t* o) const {
    int ls = ((hdr[1] >> (4 * g)) & 0xF) | (((hdr[0] >> (16 + 2 * g)) & 3) << 4);
    float dl = g_h2f(hdr[0]) * (float)(ls - 32);
#pragma unroll
    for (int j = 0; j < 16; j += 2) {
      uint32_t b0 = g_byte(qs, j), b1 = g_byte(qs, j + 1);
      o[j / 2] = g_bf16x2(dl * (float)c_kvalues[b0 & 0xF], dl * (float)c_kvalues[b1 & 0xF]);
      o[8 + j / 2] = g_bf16x2(dl * (float)c_kvalues[b0 >> 4], dl * (float)c_kvalues[b1 >> 4]);
    }
  }
};

template <> struct GDec<GQK_IQ3_S> {
  uint32_t qs[2], sg, qh[2], scb, d;
  int g;
  __device__ void load(const uint8_t* c, int r, int g_) {
    g = g_;
    gld<8>(qs, col16(c, r, g >> 1) + 8 * (g & 1));
    gld<4>(&sg, col16(c + 64 * 64, r, g >> 2) + 4 * (g & 3));
    gld<8>(qh, c + 64 * 96 + r * 8);
    gld<4>(&scb, c + 64 * 104 + r * 4);
    gld<2>(&d, c + 64 * 108 + r * 2);
  }
  __device__ void out(uint32_t* o) const {
    float dl = g_h2f(d) * (float)(1 + 2 * (int)((scb >> (4 * g)) & 0xF));
    uint32_t qhb = g_byte(qh, g);
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      uint32_t sb = (sg >> (8 * l)) & 0xFF;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        uint32_t idx = g_byte(qs, 2 * l + half) | ((qhb << (8 - 2 * l - half)) & 256);
        uint32_t gw = c_iq3s_grid[idx];
        float v[4];
#pragma unroll
        for (int k4 = 0; k4 < 4; ++k4) {
          float a = dl * (float)((gw >> (8 * k4)) & 0xFF);
          v[k4] = ((sb >> (4 * half + k4)) & 1) ? -a : a;
        }
        o[4 * l + 2 * half] = g_bf16x2(v[0], v[1]);
        o[4 * l + 2 * half + 1] = g_bf16x2(v[2], v[3]);
      }
    }
  }
};

#define GEMM_BN 128
#define GEMM_BK 64
#define GEMM_LDK (GEMM_BK + 8)   // LDS row stride in bf16 (16 B pad)

template <int BM, int T>
__device__ __forceinline__ void gemm_tile(const uint8_t* __restrict__ packed, const int32_t* __restrict__ dsc,
                                          const uint16_t* __restrict__ x, int64_t ldx, int M, uint16_t* __restrict__ y,
                                          int64_t ldy, uint16_t* As, uint16_t* Bs) {
  constexpr int WM = BM / 2;              // tokens per wave (2 x 2 waves)
  constexpr int MB = WM / 32;             // 32-token MFMA blocks per wave
  constexpr int AV = BM * GEMM_BK / 8 / 256;   // uint4 of x per thread per step
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int nb = dsc[D_NB];
  const int ntiles = dsc[D_NTILES];
  const int64_t off = (int64_t)(uint32_t)dsc[D_OFF_LO] | ((int64_t)dsc[D_OFF_HI] << 32);
  const int64_t tile0 = dsc[D_TILE0];
  const int m0 = blockIdx.y * BM;
  constexpr int REC = gqk_layout<T>::REC;

  // B-decode role: thread -> (weight row br = tid / 2 in the 128-row block, 32-weight half bh)
  const int br = tid >> 1, bh = tid & 1;
  const int btile = br >> 6, brow = br & 63;
  const bool bvalid = btile < ntiles;
  const uint8_t* bbase = packed + off + (tile0 + (bvalid ? btile : 0)) * nb * (int64_t)(64 * REC);

  v16f acc[MB][2];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int nsteps = nb * 4;
  uint4 areg[AV];
  GDec<T> breg;

  auto gload = [&](int step) {
    const int kb = step >> 2, kq = step & 3;
#pragma unroll
    for (int a = 0; a < AV; ++a) {
      int e = tid + 256 * a;          // uint4 index in the BM x 64 tile: row e / 8, col 8 * (e % 8)
      int row = e >> 3, c8 = e & 7;
      int t = m0 + row;
      areg[a] = t < M ? *(const uint4*)(x + (int64_t)t * ldx + (int64_t)step * GEMM_BK + 8 * c8) : make_uint4(0, 0, 0, 0);
    }
    breg.load(bbase + (int64_t)kb * 64 * REC, brow, 2 * kq + bh);
  };
  auto lstore = [&](int buf) {
    uint16_t* as = As + buf * BM * GEMM_LDK;
    uint16_t* bs = Bs + buf * GEMM_BN * GEMM_LDK;
#pragma unroll
    for (int a = 0; a < AV; ++a) {
      int e = tid + 256 * a;
      int row = e >> 3, c8 = e & 7;
      *(uint4*)(as + row * GEMM_LDK + 8 * c8) = areg[a];
    }
    uint32_t o[16];
    if (bvalid) breg.out(o);
    else
#pragma unroll
      for (int i = 0; i < 16; ++i) o[i] = 0;
    uint4* dst = (uint4*)(bs + br * GEMM_LDK + 32 * bh);
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
  };

  gload(0);
  lstore(0);
  __syncthreads();
  for (int step = 0; step < nsteps; ++step) {
    const int buf = step & 1;
    if (step + 1 < nsteps) gload(step + 1);
    const uint16_t* as = As + buf * BM * GEMM_LDK;
    const uint16_t* bs = Bs + buf * GEMM_BN * GEMM_LDK;
#pragma unroll
    for (int kk = 0; kk < GEMM_BK; kk += 16) {
      const int kl = kk + 8 * (lane >> 5);
      v8bf bf[2];
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bf[j] = *(const v8bf*)(bs + (wn * 64 + 32 * j + (lane & 31)) * GEMM_LDK + kl);
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        v8bf af = *(const v8bf*)(as + (wm * WM + 32 * i + (lane & 31)) * GEMM_LDK + kl);
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, bf[j], acc[i][j], 0, 0, 0);
      }
    }
    if (step + 1 < nsteps) lstore(buf ^ 1);
    __syncthreads();
  }

  // C block (i, j): lane -> weight row 32 j + (lane & 31), tokens 8 (v / 4) + 4 (lane / 32) + v % 4
  const int nvalid = dsc[D_NVALID];
  const int64_t col0 = dsc[D_COL0];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int r = wn * 64 + 32 * j + (lane & 31);
    if (r >= nvalid) continue;
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int t = m0 + wm * WM + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (t < M) y[(int64_t)t * ldy + col0 + r] = __builtin_bit_cast(uint16_t, (__bf16)acc[i][j][v]);
      }
  }
}

template <int BM, int ONLY>
__global__ __launch_bounds__(256) void gemm_kernel(const uint8_t* __restrict__ packed, const int32_t* __restrict__ desc,
                                                   const uint16_t* __restrict__ x, int64_t ldx, int M,
                                                   uint16_t* __restrict__ y, int64_t ldy) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2 * BM * GEMM_LDK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2 * GEMM_BN * GEMM_LDK];
  const int32_t* dsc = desc + (int64_t)blockIdx.x * GQK_DESC_WORDS;
  const int type = dsc[D_TYPE];
#define RUN(T) if ((ONLY == 0 || ONLY == T) && type == T) gemm_tile<BM, T>(packed, dsc, x, ldx, M, y, ldy, As, Bs);
  RUN(GQK_Q4_0) RUN(GQK_Q5_0) RUN(GQK_Q8_0) RUN(GQK_Q2_K) RUN(GQK_Q3_K) RUN(GQK_Q4_K) RUN(GQK_Q5_K) RUN(GQK_Q6_K)
  RUN(GQK_IQ4_NL) RUN(GQK_IQ3_S) RUN(GQK_IQ4_XS)
#undef RUN
}

template <int BM>
static void launch_bm(int only, dim3 grid, hipStream_t st, const uint8_t* packed, const int32_t* desc, const uint16_t* x,
                      int64_t ldx, int M, uint16_t* y, int64_t ldy) {
  switch (only) {
#define C(T) case T: hipLaunchKernelGGL((gemm_kernel<BM, T>), grid, dim3(256), 0, st, packed, desc, x, ldx, M, y, ldy); return;
    C(GQK_Q4_0) C(GQK_Q5_0) C(GQK_Q8_0) C(GQK_Q2_K) C(GQK_Q3_K) C(GQK_Q4_K) C(GQK_Q5_K) C(GQK_Q6_K)
    C(GQK_IQ4_NL) C(GQK_IQ3_S) C(GQK_IQ4_XS)
#undef C
    default:
      hipLaunchKernelGGL((gemm_kernel<BM, 0>), grid, dim3(256), 0, st, packed, desc, x, ldx, M, y, ldy);
  }
}

int launch_gemm(const uint8_t* packed, const int32_t* desc, int n_desc, int types_mask, const void* x, int64_t ldx,
                int M, int64_t K, void* y, int64_t ldy, int bm, hipStream_t st) {
  (void)K;
  dim3 grid(n_desc, (M + bm - 1) / bm);
  if (bm == 128)
    launch_bm<128>(types_mask, grid, st, packed, desc, (const uint16_t*)x, ldx, M, (uint16_t*)y, ldy);
  else if (bm == 64)
    launch_bm<64>(types_mask, grid, st, packed, desc, (const uint16_t*)x, ldx, M, (uint16_t*)y, ldy);
  else
    return GQK_ERR_FORM;
  return GQK_OK;
}

}  // namespace gqk
