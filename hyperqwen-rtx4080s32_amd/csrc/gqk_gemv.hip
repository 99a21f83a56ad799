// gqk_gemv.hip - the grouped decode GEMV (batch rows M <= 32) over mixed-type tile shards.
//
// Replaces the reference's grouped Gluon kernel for decode (tiles_grouped_kernel / _run /
// grouped_gemm, gguf-plugin/gluon/tiles_grouped.py:304-1275, dispatched for M <= 32 by
// gluon_mul_mat_tiles_grouped, gguf-plugin/gluon/interface.py:169-182), with bf16 activations
// in place of its int8 ones.
//
// Work split.  One workgroup (4 waves) per descriptor row: the row names a shard, up to four
// consecutive 64-row tiles of it (one per wave) and a k-range of 256-weight super-blocks.  The
// type is uniform per workgroup.  Lane r of a wave owns weight row r of its tile and streams
// that row's record planes with 16-byte loads (one coalesced 1 KiB access per plane slice).
//
// Arithmetic.  Every format's weight is w = d * sc * q - dmin * m with q a small integer.  The
// lane decodes q + c (c = 128, or 0 for the table formats) straight into bf16 bit patterns
// (0x4300 | u is exactly 128 + u for u < 128; table formats look up exact bf16 values) and
// feeds them as the B operand of v_mfma_f32_4x4x4_16b_bf16 (16 blocks of 4 weight rows x 4
// tokens x 4 k).  One chain of MFMAs covers one scale group (16 or 32 weights); the epilogue
// applies it in fp32:  y += (d * sc) * C - (c * d * sc + dmin * m) * sum(x over the group).
// The group sums of x are computed once per workgroup when x is staged into LDS.  Products
// bf16 x exact-integer are exact in the MFMA, accumulation is fp32, so the result equals an
// fp32 matmul of the gguf-py weights up to summation order.
//
// Split-K: with more than one k-range per tile the workgroups write fp32 partials
// [split][M][n_total] that gemv_reduce sums in a fixed order (deterministic), as the
// reference's sum_partials does (gguf-plugin/gluon/tiles_grouped.py:142-162).
#include <hip/hip_runtime.h>
#include "gqk_common.h"
#include "gqk_internal.h"

namespace gqk {

typedef short v4s __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

#define MAGIC 0x43004300u   // bf16 128.0 in both halves

enum { FAM_NAT = 0, FAM_SWAP = 1, FAM_IQ4 = 2 };

struct Tabs {
  const uint32_t* iq4;    // [256] bf16x2 (kv[b & 15], kv[b >> 4])
  const uint2* iq3g;      // [512] bf16 x 4 grid magnitudes
  const uint4* iq3s;      // [256] sign masks: bit 15 / 31 of pair dwords for 8 weights
};

__device__ __forceinline__ float h2f(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits16 & 0xFFFF));
}
__device__ __forceinline__ uint32_t bf16x2(float lo, float hi) {
  typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
  v2bf p;
  p[0] = (__bf16)lo;
  p[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, p);
}
__device__ __forceinline__ uint32_t byte_of(const uint32_t* w, int b) { return (w[b >> 2] >> (8 * (b & 3))) & 0xFF; }

template <int N>
__device__ __forceinline__ void ld16(uint32_t* dst, const uint8_t* p) {
#pragma unroll
  for (int i = 0; i < N / 16; ++i) {
    uint4 v = *(const uint4*)(p + 16 * i);
    dst[4 * i] = v.x; dst[4 * i + 1] = v.y; dst[4 * i + 2] = v.z; dst[4 * i + 3] = v.w;
  }
}

// ---- per-type decoders: load(chunk, r) pulls row r's record planes; scales(s) gives the fp32
// scale and bias of scale group s; pair(s, m) gives the two bf16x2 B dwords of MFMA m of group s.

template <int T> struct Dec;

template <> struct Dec<GQK_Q4_0> {
  static constexpr int SUB = 32, FAM = FAM_SWAP, REC = 144;
  uint32_t qs[32], dw[4];
  __device__ void load(const uint8_t* c, int r) { ld16<128>(qs, c + r * 128); ld16<16>(dw, c + 64 * 128 + r * 16); }
  __device__ void scales(int s, float& sc, float& b) const { float d = h2f(dw[s >> 1] >> (16 * (s & 1))); sc = d; b = 136.f * d; }
  __device__ void pair(int s, int m, uint32_t& b0, uint32_t& b1, const Tabs&) const {
    uint32_t w = qs[4 * s + (m & 3)];
    if (m >= 4) w >>= 4;
    b0 = (w & 0x000F000Fu) | MAGIC;
    b1 = ((w >> 8) & 0x000F000Fu) | MAGIC;
  }
};

template <> struct Dec<GQK_Q5_0> {
  static constexpr int SUB = 32, FAM = FAM_SWAP, REC = 176;
  uint32_t qs[32], qh[8], dw[4];
  __device__ void load(const uint8_t* c, int r) {
    ld16<128>(qs, c + r * 128); ld16<32>(qh, c + 64 * 128 + r * 32); ld16<16>(dw, c + 64 * 160 + r * 16);
  }
  __device__ void scales(int s, float& sc, float& b) const { float d = h2f(dw[s >> 1] >> (16 * (s & 1))); sc = d; b = 144.f * d; }
  __device__ void pair(int s, int m, uint32_t& b0, uint32_t& b1, const Tabs&) const {
    uint32_t w = qs[4 * s + (m & 3)];
    if (m >= 4) w >>= 4;
    uint32_t h4 = (qh[s] >> (4 * m)) & 0xFu;
    uint32_t hb = ((h4 * 0x00204081u) & 0x01010101u) << 4;   // bit i of h4 -> bit 4 of byte i
    uint32_t u = (w & 0x0F0F0F0Fu) | hb;
    b0 = (u & 0x00FF00FFu) | MAGIC;
    b1 = ((u >> 8) & 0x00FF00FFu) | MAGIC;
  }
};

template <> struct Dec<GQK_Q8_0> {
  static constexpr int SUB = 32, FAM = FAM_NAT, REC = 272;
  uint32_t qs[64], dw[4];
  __device__ void load(const uint8_t* c, int r) { ld16<256>(qs, c + r * 256); ld16<16>(dw, c + 64 * 256 + r * 16); }
  __device__ void scales(int s, float& sc, float& b) const { float d = h2f(dw[s >> 1] >> (16 * (s & 1))); sc = d; b = 128.f * d; }
  __device__ void pair(int s, int m, uint32_t& b0, uint32_t& b1, const Tabs&) const {
    uint32_t w = qs[8 * s + m] ^ 0x80808080u;   // int8 q -> q + 128 as unsigned bytes
    b0 = bf16x2((float)(w & 0xFF), (float)((w >> 8) & 0xFF));
    b1 = bf16x2((float)((w >> 16) & 0xFF), (float)(w >> 24));
  }
};

template <> struct Dec<GQK_Q2_K> {
  static constexpr int SUB = 16, FAM = FAM_SWAP, REC = 84;
  uint32_t qs[16], sc[4], dd;
  __device__ void load(const uint8_t* c, int r) {
    ld16<64>(qs, c + r * 64); ld16<16>(sc, c + 64 * 64 + r * 16); dd = *(const uint32_t*)(c + 64 * 80 + r * 4);
  }
  __device__ void scales(int s, float& scale, float& b) const {
    uint32_t sb = byte_of(sc, s);
    float d = h2f(dd), dmin = h2f(dd >> 16);
    scale = d * (float)(sb & 0xF);
    b = 128.f * scale + dmin * (float)(sb >> 4);
  }
  __device__ void pair(int s, int m, uint32_t& b0, uint32_t& b1, const Tabs&) const {
    int h = s >> 3, t = (s >> 1) & 3, hf = s & 1;
    uint32_t w = qs[8 * h + 4 * hf + m] >> (2 * t);
    b0 = (w & 0x00030003u) | MAGIC;
    b1 = ((w >> 8) & 0x00030003u) | MAGIC;
  }
};

template <> struct Dec<GQK_Q3_K> {
  static constexpr int SUB = 16, FAM = FAM_SWAP, REC = 110;
  uint32_t qs[16], hm[8], sb[3], d16;
  __device__ void load(const uint8_t* c, int r) {
    ld16<64>(qs, c + r * 64);
    ld16<32>(hm, c + 64 * 64 + r * 32);
    const uint32_t* p = (const uint32_t*)(c + 64 * 96 + r * 12);
    sb[0] = p[0]; sb[1] = p[1]; sb[2] = p[2];
    d16 = *(const uint16_t*)(c + 64 * 108 + r * 2);
  }
  __device__ void scales(int s, float& scale, float& b) const {
    int lo = (byte_of(sb, s % 8) >> (4 * (s / 8))) & 0xF;
    int hi = (byte_of(sb, 8 + s % 4) >> (2 * (s / 4))) & 3;
    scale = h2f(d16) * (float)((lo | (hi << 4)) - 32);
    b = 132.f * scale;
  }
  __device__ void pair(int s, int m, uint32_t& b0, uint32_t& b1, const Tabs&) const {
    int n = s >> 3, j = (s >> 1) & 3, hf = s & 1;
    uint32_t q = (qs[8 * n + 4 * hf + m] >> (2 * j)) & 0x03030303u;
    uint32_t h = (hm[4 * hf + m] >> (4 * n + j)) & 0x01010101u;
    uint32_t u = q | (h << 2);
    b0 = (u & 0x00FF00FFu) | MAGIC;
    b1 = ((u >> 8) & 0x00FF00FFu) | MAGIC;
  }
};

__device__ __forceinline__ void scale_min_k4w(const uint32_t* S, int j, int& sc, int& m) {
  if (j < 4) {
    sc = byte_of(S, j) & 63;
    m = byte_of(S, j + 4) & 63;
  } else {
    sc = (byte_of(S, j + 4) & 0xF) | ((byte_of(S, j - 4) >> 6) << 4);
    m = (byte_of(S, j + 4) >> 4) | ((byte_of(S, j) >> 6) << 4);
  }
}

template <> struct Dec<GQK_Q4_K> {
  static constexpr int SUB = 32, FAM = FAM_SWAP, REC = 144;
  uint32_t qs[32], hdr[4];
  __device__ void load(const uint8_t* c, int r) { ld16<128>(qs, c + r * 128); ld16<16>(hdr, c + 64 * 128 + r * 16); }
  __device__ void scales(int s, float& scale, float& b) const {
    int sc, m;
    scale_min_k4w(hdr + 1, s, sc, m);
    scale = h2f(hdr[0]) * (float)sc;
    b = 128.f * scale + h2f(hdr[0] >> 16) * (float)m;
  }
  __device__ void pair(int s, int m, uint32_t& b0, uint32_t& b1, const Tabs&) const {
    uint32_t w = qs[8 * (s >> 1) + m] >> (4 * (s & 1));
    b0 = (w & 0x000F000Fu) | MAGIC;
    b1 = ((w >> 8) & 0x000F000Fu) | MAGIC;
  }
};

template <> struct Dec<GQK_Q5_K> {
  static constexpr int SUB = 32, FAM = FAM_SWAP, REC = 176;
  uint32_t qs[32], qh[8], hdr[4];
  __device__ void load(const uint8_t* c, int r) {
    ld16<128>(qs, c + r * 128); ld16<32>(qh, c + 64 * 128 + r * 32); ld16<16>(hdr, c + 64 * 160 + r * 16);
  }
  __device__ void scales(int s, float& scale, float& b) const {
    int sc, m;
    scale_min_k4w(hdr + 1, s, sc, m);
    scale = h2f(hdr[0]) * (float)sc;
    b = 128.f * scale + h2f(hdr[0] >> 16) * (float)m;
  }
  __device__ void pair(int s, int m, uint32_t& b0, uint32_t& b1, const Tabs&) const {
    uint32_t w = (qs[8 * (s >> 1) + m] >> (4 * (s & 1))) & 0x0F0F0F0Fu;
    uint32_t u = w | (((qh[m] >> s) & 0x01010101u) << 4);
    b0 = (u & 0x00FF00FFu) | MAGIC;
    b1 = ((u >> 8) & 0x00FF00FFu) | MAGIC;
  }
};

template <> struct Dec<GQK_Q6_K> {
  static constexpr int SUB = 16, FAM = FAM_SWAP, REC = 210;
  uint32_t ql[32], qh[16], sc[4], d16;
  __device__ void load(const uint8_t* c, int r) {
    ld16<128>(ql, c + r * 128); ld16<64>(qh, c + 64 * 128 + r * 64); ld16<16>(sc, c + 64 * 192 + r * 16);
    d16 = *(const uint16_t*)(c + 64 * 208 + r * 2);
  }
  __device__ void scales(int s, float& scale, float& b) const {
    scale = h2f(d16) * (float)(int8_t)byte_of(sc, s);
    b = 160.f * scale;
  }
  __device__ void pair(int s, int m, uint32_t& b0, uint32_t& b1, const Tabs&) const {
    int h = s >> 3, t = (s >> 1) & 3, hf = s & 1;
    uint32_t lo = (ql[16 * h + 8 * (t & 1) + 4 * hf + m] >> (4 * (t >> 1))) & 0x0F0F0F0Fu;
    uint32_t hi = (qh[8 * h + 4 * hf + m] >> (2 * t)) & 0x03030303u;
    uint32_t u = lo | (hi << 4);
    b0 = (u & 0x00FF00FFu) | MAGIC;
    b1 = ((u >> 8) & 0x00FF00FFu) | MAGIC;
  }
};

template <> struct Dec<GQK_IQ4_NL> {
  static constexpr int SUB = 32, FAM = FAM_IQ4, REC = 144;
  uint32_t qs[32], dw[4];
  __device__ void load(const uint8_t* c, int r) { ld16<128>(qs, c + r * 128); ld16<16>(dw, c + 64 * 128 + r * 16); }
  __device__ void scales(int s, float& sc, float& b) const { sc = h2f(dw[s >> 1] >> (16 * (s & 1))); b = 0.f; }
  __device__ void pair(int s, int m, uint32_t& b0, uint32_t& b1, const Tabs& tb) const {
    uint32_t w = qs[4 * s + (m >> 1)] >> (16 * (m & 1));
    b0 = tb.iq4[w & 0xFF];
    b1 = tb.iq4[(w >> 8) & 0xFF];
  }
};

template <> struct Dec<GQK_IQ4_XS> {
  static constexpr int SUB = 32, FAM = FAM_IQ4, REC = 136;
  uint32_t qs[32], hdr[2];
  __device__ void load(const uint8_t* c, int r) {
    ld16<128>(qs, c + r * 128);
    uint2 h = *(const uint2*)(c + 64 * 128 + r * 8);
    hdr[0] = h.x; hdr[1] = h.y;
  }
  __device__ void scales(int s, float& sc, float& b) const {
    int ls = ((hdr[1] >> (4 * s)) & 0xF) | (((hdr[0] >> (16 + 2 * s)) & 3) << 4);
    sc = h2f(hdr[0]) * (float)(ls - 32);
    b = 0.f;
  }
  __device__ void pair(int s, int m, uint32_t& b0, uint32_t& b1, const Tabs& tb) const {
    uint32_t w = qs[4 * s + (m >> 1)] >> (16 * (m & 1));
    b0 = tb.iq4[w & 0xFF];
    b1 = tb.iq4[(w >> 8) & 0xFF];
  }
};

template <> struct Dec<GQK_IQ3_S> {
  static constexpr int SUB = 32, FAM = FAM_NAT, REC = 110;
  uint32_t qs[16], sg[8], qh[2], scb, d16;
  __device__ void load(const uint8_t* c, int r) {
    ld16<64>(qs, c + r * 64);
    ld16<32>(sg, c + 64 * 64 + r * 32);
    uint2 h = *(const uint2*)(c + 64 * 96 + r * 8);
    qh[0] = h.x; qh[1] = h.y;
    scb = *(const uint32_t*)(c + 64 * 104 + r * 4);
    d16 = *(const uint16_t*)(c + 64 * 108 + r * 2);
  }
  __device__ void scales(int s, float& sc, float& b) const {
    sc = h2f(d16) * (float)(1 + 2 * (int)((scb >> (4 * s)) & 0xF));
    b = 0.f;
  }
  __device__ void pair(int s, int m, uint32_t& b0, uint32_t& b1, const Tabs& tb) const {
    int l = m >> 1, half = m & 1;
    uint32_t qsb = (qs[2 * s + (l >> 1)] >> (8 * (2 * (l & 1) + half))) & 0xFF;
    uint32_t qhb = byte_of(qh, s);
    uint32_t idx = qsb | ((qhb << (8 - 2 * l - half)) & 256);
    uint2 mag = tb.iq3g[idx];
    uint4 msk = tb.iq3s[(sg[s] >> (8 * l)) & 0xFF];
    b0 = mag.x ^ (half ? msk.z : msk.x);
    b1 = mag.y ^ (half ? msk.w : msk.y);
  }
};

// ---- x staging: slot (k / 4 in the decoder's order) x token, 4 bf16 each.
// FAM_NAT: slot q holds k = 4q .. 4q+3; FAM_SWAP: (4q, 4q+2, 4q+1, 4q+3);
// FAM_IQ4: slot q = 8s + m holds (32s + 2m, 32s + 2m + 16, 32s + 2m + 1, 32s + 2m + 17).
template <int FAM>
__device__ __forceinline__ uint2 stage_slot(const uint16_t* xr, int q) {
  if (FAM == FAM_IQ4) {
    int s = q >> 3, m = q & 7;
    uint32_t a = *(const uint32_t*)(xr + 32 * s + 2 * m);
    uint32_t c = *(const uint32_t*)(xr + 32 * s + 2 * m + 16);
    return make_uint2((a & 0xFFFFu) | (c << 16), (a >> 16) | (c & 0xFFFF0000u));
  } else {
    uint2 v = *(const uint2*)(xr + 4 * q);
    if (FAM == FAM_SWAP) {
      return make_uint2((v.x & 0xFFFFu) | (v.y << 16), (v.x >> 16) | (v.y & 0xFFFF0000u));
    }
    return v;
  }
}

__device__ __forceinline__ float bf2f(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

// LDS budget: x chunk 16 KiB (CH super-blocks x 64 slots x MPAD tokens x 8 B with CH * MPAD = 32),
// group sums 3 KiB, tables 9 KiB.
#define GEMV_XCH_SLOTS 2048   // CH * 64 * MPAD
#define GEMV_LDS_X (GEMV_XCH_SLOTS * 8)
#define GEMV_LDS_SUM (32 * 24 * 4)

template <int G, int T>
__device__ __forceinline__ void gemv_tile(const uint8_t* __restrict__ packed, const int32_t* __restrict__ dsc,
                                          const uint16_t* __restrict__ x, int64_t ldx, int M, uint8_t* lds,
                                          const Tabs& tb, v4f (&acc)[G]) {
  typedef Dec<T> D;
  constexpr int MPAD = 4 * G, CH = 32 / MPAD, MPS = D::SUB / 4, NSUB = 256 / D::SUB;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kb0 = dsc[D_KB0], kb1 = dsc[D_KB1], nb = dsc[D_NB];
  const int ntiles = dsc[D_NTILES];
  const int64_t off = (int64_t)(uint32_t)dsc[D_OFF_LO] | ((int64_t)dsc[D_OFF_HI] << 32);
  const int64_t tile = dsc[D_TILE0] + wave;
  const bool active = wave < ntiles;
  const uint8_t* tbase = packed + off + tile * nb * (int64_t)(64 * D::REC);
  uint2* xs = (uint2*)lds;
  float* xsum16 = (float*)(lds + GEMV_LDS_X);
  float* xsum32 = xsum16 + CH * 16 * MPAD;

  for (int kc = kb0; kc < kb1; kc += CH) {
    const int nch = min(CH, kb1 - kc);
    __syncthreads();
    // stage x[:, kc*256 .. (kc+nch)*256) in the decoder's slot order, zero for tokens >= M
    for (int it = tid; it < nch * 64 * MPAD; it += 256) {
      int t = it % MPAD, q = it / MPAD;   // q = kbl * 64 + slot
      uint2 v = make_uint2(0, 0);
      if (t < M) v = stage_slot<D::FAM>(x + t * ldx + (int64_t)(kc + (q >> 6)) * 256, q & 63);
      xs[it] = v;
    }
    for (int it = tid; it < nch * 8 * MPAD; it += 256) {
      int t = it % MPAD, q = it / MPAD;   // q = kbl * 8 + s32
      float a = 0.f, b = 0.f;
      if (t < M) {
        const uint16_t* xr = x + t * ldx + (int64_t)(kc + (q >> 3)) * 256 + 32 * (q & 7);
#pragma unroll
        for (int j = 0; j < 16; ++j) a += bf2f(xr[j]);
#pragma unroll
        for (int j = 0; j < 16; ++j) b += bf2f(xr[16 + j]);
      }
      int kbl = q >> 3, s = q & 7;
      xsum16[(kbl * 16 + 2 * s) * MPAD + t] = a;
      xsum16[(kbl * 16 + 2 * s + 1) * MPAD + t] = b;
      xsum32[(kbl * 8 + s) * MPAD + t] = a + b;
    }
    __syncthreads();
    if (!active) continue;

    D cur;
    cur.load(tbase + (int64_t)kc * 64 * D::REC, lane);
    for (int kbl = 0; kbl < nch; ++kbl) {
      D nxt;
      if (kbl + 1 < nch) nxt.load(tbase + (int64_t)(kc + kbl + 1) * 64 * D::REC, lane);
#pragma unroll
      for (int s = 0; s < NSUB; ++s) {
        float scale, bias;
        cur.scales(s, scale, bias);
        v4f C[G];
#pragma unroll
        for (int g = 0; g < G; ++g) C[g] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < MPS; ++m) {
          uint32_t b0, b1;
          cur.pair(s, m, b0, b1, tb);
          v4s B = __builtin_bit_cast(v4s, make_uint2(b0, b1));
          const int slot = s * MPS + m;
#pragma unroll
          for (int g = 0; g < G; ++g) {
            v4s A = __builtin_bit_cast(v4s, xs[(kbl * 64 + slot) * MPAD + 4 * g + (lane & 3)]);
            C[g] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(A, B, C[g], 0, 0, 0);
          }
        }
        const float* xsm = (D::SUB == 16 ? xsum16 + (kbl * 16 + s) * MPAD : xsum32 + (kbl * 8 + s) * MPAD);
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float4 sx = *(const float4*)(xsm + 4 * g);
          acc[g][0] += scale * C[g][0] - bias * sx.x;
          acc[g][1] += scale * C[g][1] - bias * sx.y;
          acc[g][2] += scale * C[g][2] - bias * sx.z;
          acc[g][3] += scale * C[g][3] - bias * sx.w;
        }
      }
      cur = nxt;
    }
  }
}

__device__ void build_tables(uint8_t* lds_tab, int type) {
  const int tid = threadIdx.x;
  if (type == GQK_IQ4_NL || type == GQK_IQ4_XS) {
    uint32_t* t4 = (uint32_t*)lds_tab;
    t4[tid] = bf16x2((float)c_kvalues[tid & 15], (float)c_kvalues[tid >> 4]);
  } else if (type == GQK_IQ3_S) {
    uint2* tg = (uint2*)lds_tab;
    uint4* ts = (uint4*)(lds_tab + 512 * 8);
    for (int i = tid; i < 512; i += 256) {
      uint32_t gw = c_iq3s_grid[i];
      tg[i] = make_uint2(bf16x2((float)(gw & 0xFF), (float)((gw >> 8) & 0xFF)),
                         bf16x2((float)((gw >> 16) & 0xFF), (float)(gw >> 24)));
    }
    uint32_t m[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) m[p] = (((tid >> (2 * p)) & 1) << 15) | (((tid >> (2 * p + 1)) & 1) << 31);
    ts[tid] = make_uint4(m[0], m[1], m[2], m[3]);
  }
}

template <int G, int ONLY>
__global__ __launch_bounds__(256) void gemv_kernel(const uint8_t* __restrict__ packed, const int32_t* __restrict__ desc,
                                                   const uint16_t* __restrict__ x, int64_t ldx, int M,
                                                   uint16_t* __restrict__ y, int64_t ldy, float* __restrict__ part,
                                                   int64_t n_total) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[GEMV_LDS_X + GEMV_LDS_SUM + 9216];
  const int32_t* dsc = desc + (int64_t)blockIdx.x * GQK_DESC_WORDS;
  const int type = dsc[D_TYPE];
  uint8_t* lds_tab = lds + GEMV_LDS_X + GEMV_LDS_SUM;
  Tabs tb{(const uint32_t*)lds_tab, (const uint2*)lds_tab, (const uint4*)(lds_tab + 4096)};
  build_tables(lds_tab, type);   // made visible by the first barrier of the staging loop
  v4f acc[G];
#pragma unroll
  for (int g = 0; g < G; ++g) acc[g] = v4f{0.f, 0.f, 0.f, 0.f};

#define RUN(T) if ((ONLY == 0 || ONLY == T) && type == T) gemv_tile<G, T>(packed, dsc, x, ldx, M, lds, tb, acc);
  RUN(GQK_Q4_0) RUN(GQK_Q5_0) RUN(GQK_Q8_0) RUN(GQK_Q2_K) RUN(GQK_Q3_K) RUN(GQK_Q4_K) RUN(GQK_Q5_K) RUN(GQK_Q6_K)
  RUN(GQK_IQ4_NL) RUN(GQK_IQ3_S) RUN(GQK_IQ4_XS)
#undef RUN

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (wave >= dsc[D_NTILES]) return;
  const int r = wave * 64 + lane;
  if (r >= dsc[D_NVALID]) return;
  const int64_t col = (int64_t)dsc[D_COL0] + r;
  if (part == nullptr) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        int t = 4 * g + i;
        if (t < M) y[t * ldy + col] = __builtin_bit_cast(uint16_t, (__bf16)acc[g][i]);
      }
  } else {
    float* p = part + (int64_t)dsc[D_SPLIT] * M * n_total;
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        int t = 4 * g + i;
        if (t < M) p[t * n_total + col] = acc[g][i];
      }
  }
}

// y[t, c] = bf16( sum_s part[s, t, c] ), s = 0 .. S-1 in order
__global__ __launch_bounds__(256) void gemv_reduce(const float* __restrict__ part, int S, int M, int64_t n_total,
                                                   uint16_t* __restrict__ y, int64_t ldy) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)M * n_total) return;
  int64_t t = i / n_total, c = i % n_total;
  float a = 0.f;
  for (int s = 0; s < S; ++s) a += part[(int64_t)s * M * n_total + i];
  y[t * ldy + c] = __builtin_bit_cast(uint16_t, (__bf16)a);
}

template <int G>
static void launch_g(int only, dim3 grid, hipStream_t st, const uint8_t* packed, const int32_t* desc, const uint16_t* x,
                     int64_t ldx, int M, uint16_t* y, int64_t ldy, float* part, int64_t n_total) {
  switch (only) {
#define C(T) case T: hipLaunchKernelGGL((gemv_kernel<G, T>), grid, dim3(256), 0, st, packed, desc, x, ldx, M, y, ldy, part, n_total); return;
    C(GQK_Q4_0) C(GQK_Q5_0) C(GQK_Q8_0) C(GQK_Q2_K) C(GQK_Q3_K) C(GQK_Q4_K) C(GQK_Q5_K) C(GQK_Q6_K)
    C(GQK_IQ4_NL) C(GQK_IQ3_S) C(GQK_IQ4_XS)
#undef C
    default:
      hipLaunchKernelGGL((gemv_kernel<G, 0>), grid, dim3(256), 0, st, packed, desc, x, ldx, M, y, ldy, part, n_total);
  }
}

// types_mask: the single type of every row (> 0) or 0 for a mixed launch
int launch_gemv(const uint8_t* packed, const int32_t* desc, int n_desc, int types_mask, const void* x, int64_t ldx,
                int M, int G, void* y, int64_t ldy, float* partials, int split, int64_t n_total, hipStream_t st) {
  dim3 grid(n_desc);
  float* part = split > 1 ? partials : nullptr;
  const uint16_t* xx = (const uint16_t*)x;
  uint16_t* yy = (uint16_t*)y;
  switch (G) {
    case 1: launch_g<1>(types_mask, grid, st, packed, desc, xx, ldx, M, yy, ldy, part, n_total); break;
    case 2: launch_g<2>(types_mask, grid, st, packed, desc, xx, ldx, M, yy, ldy, part, n_total); break;
    case 4: launch_g<4>(types_mask, grid, st, packed, desc, xx, ldx, M, yy, ldy, part, n_total); break;
    case 8: launch_g<8>(types_mask, grid, st, packed, desc, xx, ldx, M, yy, ldy, part, n_total); break;
    default: return GQK_ERR_FORM;
  }
  if (split > 1) {
    int64_t total = (int64_t)M * n_total;
    hipLaunchKernelGGL(gemv_reduce, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, partials, split, M, n_total,
                       yy, ldy);
  }
  return GQK_OK;
}

}  // namespace gqk
