// gqk_gemv.hip - the grouped decode GEMV (batch rows M <= 16) over mixed-type tile shards.
//
// Replaces the reference's grouped Gluon kernel for decode (tiles_grouped_kernel / _run /
// grouped_gemm, gguf-plugin/gluon/tiles_grouped.py:304-1275, dispatched for M <= 32 by
// gluon_mul_mat_tiles_grouped, gguf-plugin/gluon/interface.py:169-182), with bf16 activations
// in place of its int8 ones.  Here it serves M <= 16; the GEMM form is faster from 17 rows.
//
// Work split.  One workgroup (nw waves, chosen by the planner) per descriptor row: the row names
// a shard, one 64-row tile of it and a k-range of 256-weight super-blocks, which the waves split
// evenly.  The type is uniform per workgroup.  Lane r of a wave owns weight row r of the tile
// and streams that row's record planes with 16-byte loads (one coalesced 1 KiB access per plane
// column); each wave stages its own slice of x in a private LDS region, so the main loop has no
// workgroup barrier.
//
// Arithmetic.  Every format's weight is w = d * sc * q - dmin * m with q a small integer.  The
// lane decodes q + c (c = 128, or 0 for the table formats) straight into bf16 bit patterns
// (0x4300 | u is exactly 128 + u for u < 128; table formats look up exact bf16 values) and
// feeds them as the B operand of v_mfma_f32_4x4x4_16b_bf16 (16 blocks of 4 weight rows x 4
// tokens x 4 k).  One chain of MFMAs covers one scale group (16 or 32 weights); the epilogue
// applies it in fp32:  y += (d * sc) * C - (c * d * sc + dmin * m) * sum(x over the group), the
// second term as one v_mfma_f32_4x4x1f32 outer product (token sums x row biases) per group.
// The x operands (A) and the group sums of x are computed once per record when the wave stages
// its x slice into LDS; the MFMAs then take them from registers through the block broadcast
// (CBSZ / ABID), one LDS read per 16 slots.  Products bf16 x exact-integer are exact in the
// MFMA, accumulation is fp32, so the result equals an fp32 matmul of the gguf-py weights up to
// summation order.
//
// Split-K: a tile shared by several workgroups (k-ranges) gets fp32 partial slots
// [slot][row][token]; the last workgroup of the tile to arrive sums them in split order
// (deterministic, one rounding to bf16), the reference's sum_partials
// (gguf-plugin/gluon/tiles_grouped.py:142-162) fused into the same launch.
#include <hip/hip_runtime.h>
#include "gqk_common.h"
#include "gqk_internal.h"

namespace gqk {

typedef short v4s __attribute__((ext_vector_type(4)));
// buffer resource word 3 (raw untyped dword access) and the device-scope cache policy (sc1)
#define GQK_BUF_WORD3 0x00020000
#define GQK_CPOL_SC1 16
typedef float v4f __attribute__((ext_vector_type(4)));


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

// Opaque constants for the decode: gfx9 VOP3 takes no literal, so with the masks held in SGPRs
// and the bf16 exponent pattern (0x4300 = 128.0 in each half) in a VGPR, (a & m) | o is a single
// v_and_or_b32.  The values are hidden from constant folding by empty asm statements (no
// instruction is emitted), so the compiler still schedules the ALU ops and their MFMA hazards.
struct Masks {
  // 0x000F000F, 0x00FF00FF, 0x00030003, 0x000C000C, 0x00300030 (SGPRs); 0x43004300, 0x43434343 (VGPRs)
  uint32_t f, ff, t3, t3b, t3c, mg, m43;
};
__device__ __forceinline__ Masks make_masks() {
  Masks k{0x000F000Fu, 0x00FF00FFu, 0x00030003u, 0x000C000Cu, 0x00300030u, 0x43004300u, 0x43434343u};
  asm volatile("" : "+s"(k.f));
  asm volatile("" : "+s"(k.ff));
  asm volatile("" : "+s"(k.t3));
  asm volatile("" : "+s"(k.t3b));
  asm volatile("" : "+s"(k.t3c));
  asm volatile("" : "+v"(k.mg));
  asm volatile("" : "+v"(k.m43));
  return k;
}
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) { return (a & m) | o; }
// Four byte values u0..u3 < 128 -> the two B dwords {128 + u0, 128 + u2} and {128 + u1, 128 + u3}
// as bf16 pairs (the FAM_SWAP order): one v_perm_b32 each, placing a 0x43 exponent byte above
// every value byte (v_perm selector bytes 0-3 pick bytes of the second source, 4-7 of the first).
__device__ __forceinline__ void split_bytes(uint32_t u, const Masks& k, uint32_t& b0, uint32_t& b1) {
  b0 = __builtin_amdgcn_perm(k.m43, u, 0x04020400u);
  b1 = __builtin_amdgcn_perm(k.m43, u, 0x04030401u);
}

// Row r's slice of a plane of N bytes per row (N a multiple of 16).  Planes are column-major in
// 16-byte columns: column i of row r sits at (i * 64 + r) * 16, so load i of a wave is one
// contiguous 1 KiB access.  The lane's offset enters as an unsigned 32-bit add to the column's
// base, which lets the columns past the 4 KiB immediate range share the lane's offset register
// (a signed (i * 64 + r) * 16 gave each such column a 64-bit address of its own, and Q6_K's
// twelve columns spilled at three waves per SIMD).
template <int N>
__device__ __forceinline__ void ldp(uint32_t* dst, const uint8_t* plane, int r) {
#pragma unroll
  for (int i = 0; i < N / 16; ++i) {
    uint4 v = *(const uint4*)(plane + i * 1024 + (uint32_t)(r * 16));
    dst[4 * i] = v.x; dst[4 * i + 1] = v.y; dst[4 * i + 2] = v.z; dst[4 * i + 3] = v.w;
  }
}

// ---- per-type decoders: load(chunk, r) pulls row r's record planes; scales(s) gives the fp32
// scale and bias of scale group s; pair(s, m) gives the two bf16x2 B dwords of MFMA m of group s.

template <int T> struct Dec;

template <> struct Dec<GQK_Q4_0> {
  static constexpr int SUB = 32, FAM = FAM_SWAP, REC = 144;
  uint32_t qs[32], dw[4];
  __device__ void load(const uint8_t* c, int r) { ldp<128>(qs, c, r); ldp<16>(dw, c + 64 * 128, r); }
  __device__ void scales(int s, float& sc, float& b) const { float d = h2f(dw[s >> 1] >> (16 * (s & 1))); sc = d; b = 136.f * d; }
  __device__ void pair(int s, int m, uint32_t& b0, uint32_t& b1, const Tabs&, const Masks& k) const {
    uint32_t w = qs[4 * s + (m & 3)];
    if (m >= 4) w >>= 4;
    b0 = and_or(w, k.f, k.mg);
    b1 = and_or(w >> 8, k.f, k.mg);
  }
};

template <> struct Dec<GQK_Q5_0> {
  static constexpr int SUB = 32, FAM = FAM_SWAP, REC = 176;
  uint32_t qs[32], qh[8], dw[4];
  __device__ void load(const uint8_t* c, int r) {
    ldp<128>(qs, c, r); ldp<32>(qh, c + 64 * 128, r); ldp<16>(dw, c + 64 * 160, r);
  }
  __device__ void scales(int s, float& sc, float& b) const { float d = h2f(dw[s >> 1] >> (16 * (s & 1))); sc = d; b = 144.f * d; }
  __device__ void pair(int s, int m, uint32_t& b0, uint32_t& b1, const Tabs&, const Masks& k) const {
    uint32_t w = qs[4 * s + (m & 3)];
    if (m >= 4) w >>= 4;
    uint32_t h4 = (qh[s] >> (4 * m)) & 0xFu;
    uint32_t hb = ((h4 * 0x00204081u) & 0x01010101u) << 4;   // bit i of h4 -> bit 4 of byte i
    uint32_t u = (w & 0x0F0F0F0Fu) | hb;
    split_bytes(u, k, b0, b1);
  }
};

template <> struct Dec<GQK_Q8_0> {
  static constexpr int SUB = 32, FAM = FAM_NAT, REC = 272;
  uint32_t qs[64], dw[4];
  __device__ void load(const uint8_t* c, int r) { ldp<256>(qs, c, r); ldp<16>(dw, c + 64 * 256, r); }
  __device__ void scales(int s, float& sc, float& b) const { float d = h2f(dw[s >> 1] >> (16 * (s & 1))); sc = d; b = 128.f * d; }
  __device__ void pair(int s, int m, uint32_t& b0, uint32_t& b1, const Tabs&, const Masks& k) const {
    uint32_t w = qs[8 * s + m] ^ 0x80808080u;   // int8 q -> q + 128 as unsigned bytes
    b0 = bf16x2((float)(w & 0xFF), (float)((w >> 8) & 0xFF));
    b1 = bf16x2((float)((w >> 16) & 0xFF), (float)(w >> 24));
  }
};

// Q2_K / Q3_K: the 2-bit field of scale group s sits at bits 2t .. 2t + 1 of each byte (t =
// (s >> 1) & 3).  It is masked where it sits rather than shifted down: the bf16 pattern
// 0x4300 | (u << p) is exactly 128 + 2^p u while bit p + 2 (Q3_K: p + 3) stays below the
// exponent, and the group's scale is divided by 2^p (exact).  p = 2t for t <= 2; the t = 3 field
// is shifted down to p = 2 (Q2_K) or p = 4 (Q3_K, whose third bit needs room above it).
__device__ constexpr float q2_inv(int t) { return t == 0 ? 1.f : t == 2 ? 0.0625f : 0.25f; }
__device__ constexpr float q3_inv(int t) { return t == 0 ? 1.f : t == 1 ? 0.25f : 0.0625f; }

template <> struct Dec<GQK_Q2_K> {
  static constexpr int SUB = 16, FAM = FAM_SWAP, REC = 84;
  uint32_t qs[16], sc[4], dd;
  __device__ void load(const uint8_t* c, int r) {
    ldp<64>(qs, c, r); ldp<16>(sc, c + 64 * 64, r); dd = *(const uint32_t*)(c + 64 * 80 + r * 4);
  }
  __device__ void scales(int s, float& scale, float& b) const {
    uint32_t sb = byte_of(sc, s);
    const float d = h2f(dd), dmin = h2f(dd >> 16);
    scale = (d * q2_inv((s >> 1) & 3)) * (float)(sb & 0xF);   // d 2^-p: one product per p (exact)
    b = 128.f * scale + dmin * (float)(sb >> 4);
  }
  __device__ void pair(int s, int m, uint32_t& b0, uint32_t& b1, const Tabs&, const Masks& k) const {
    int h = s >> 3, t = (s >> 1) & 3, hf = s & 1;
    const uint32_t w = qs[8 * h + 4 * hf + m];
    const uint32_t v = t == 3 ? w >> 4 : w;
    const uint32_t msk = t == 0 ? k.t3 : t == 2 ? k.t3c : k.t3b;
    b0 = and_or(v, msk, k.mg);
    b1 = and_or(v >> 8, msk, k.mg);
  }
};

template <> struct Dec<GQK_Q3_K> {
  static constexpr int SUB = 16, FAM = FAM_SWAP, REC = 110;
  uint32_t qs[16], hm[8], sb[3], d16;
  __device__ void load(const uint8_t* c, int r) {
    ldp<64>(qs, c, r);
    ldp<32>(hm, c + 64 * 64, r);
    const uint32_t* p = (const uint32_t*)(c + 64 * 96);   // 12-byte plane: three 4-byte columns
    sb[0] = p[r]; sb[1] = p[64 + r]; sb[2] = p[128 + r];
    d16 = *(const uint16_t*)(c + 64 * 108 + r * 2);
  }
  __device__ void scales(int s, float& scale, float& b) const {
    int lo = (byte_of(sb, s % 8) >> (4 * (s / 8))) & 0xF;
    int hi = (byte_of(sb, 8 + s % 4) >> (2 * (s / 4))) & 3;
    const float inv = q3_inv((s >> 1) & 3);
    scale = (h2f(d16) * inv) * (float)((lo | (hi << 4)) - 32);   // d 2^-p: one product per p (exact)
    b = (128.f + 4.f / inv) * scale;                              // 128 2^-p d sc + 4 d sc, exact
  }
  __device__ void pair(int s, int m, uint32_t& b0, uint32_t& b1, const Tabs&, const Masks& k) const {
    int n = s >> 3, j = (s >> 1) & 3, hf = s & 1;
    const int p = j == 3 ? 4 : 2 * j;                        // where the 3-bit value lands
    const uint32_t qd = qs[8 * n + 4 * hf + m];
    const uint32_t q = (j == 3 ? qd >> 2 : qd) & (0x03030303u << p);
    const int hs = 4 * n + j - (p + 2);                      // the hmask bit (4n + j) -> bit p + 2
    const uint32_t hd = hm[4 * hf + m];
    const uint32_t h = hs >= 0 ? hd >> hs : hd << -hs;
    const uint32_t u = and_or(h, 0x04040404u << p, q);
    split_bytes(u, k, b0, b1);
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
  __device__ void load(const uint8_t* c, int r) { ldp<128>(qs, c, r); ldp<16>(hdr, c + 64 * 128, r); }
  __device__ void scales(int s, float& scale, float& b) const {
    int sc, m;
    scale_min_k4w(hdr + 1, s, sc, m);
    scale = h2f(hdr[0]) * (float)sc;
    b = 128.f * scale + h2f(hdr[0] >> 16) * (float)m;
  }
  __device__ void pair(int s, int m, uint32_t& b0, uint32_t& b1, const Tabs&, const Masks& k) const {
    uint32_t w = qs[8 * (s >> 1) + m] >> (4 * (s & 1));
    b0 = and_or(w, k.f, k.mg);
    b1 = and_or(w >> 8, k.f, k.mg);
  }
};

template <> struct Dec<GQK_Q5_K> {
  static constexpr int SUB = 32, FAM = FAM_SWAP, REC = 176;
  uint32_t qs[32], qh[8], hdr[4];
  __device__ void load(const uint8_t* c, int r) {
    ldp<128>(qs, c, r); ldp<32>(qh, c + 64 * 128, r); ldp<16>(hdr, c + 64 * 160, r);
  }
  __device__ void scales(int s, float& scale, float& b) const {
    int sc, m;
    scale_min_k4w(hdr + 1, s, sc, m);
    scale = h2f(hdr[0]) * (float)sc;
    b = 128.f * scale + h2f(hdr[0] >> 16) * (float)m;
  }
  __device__ void pair(int s, int m, uint32_t& b0, uint32_t& b1, const Tabs&, const Masks& k) const {
    uint32_t w = (qs[8 * (s >> 1) + m] >> (4 * (s & 1))) & 0x0F0F0F0Fu;
    uint32_t u = w | (((qh[m] >> s) & 0x01010101u) << 4);
    split_bytes(u, k, b0, b1);
  }
};

// Q6_K from the re-packed six-bit plane (gqk_q6_pos): group s's dwords P0..P2 sit at column
// 3 (s / 4) + m, dword s % 4.  Weights 4m .. 4m + 3 of the group are one AND away (m < 3); the last
// four gather their three top-bit pairs (measured against the GGUF ql / qh planes, whose merge
// costs two to three more VALU per four weights: Q6_K gate_up at M = 8 6% faster at equal registers).
template <> struct Dec<GQK_Q6_K> {
  static constexpr int SUB = 16, FAM = FAM_SWAP, REC = 210;
  uint32_t q6[48], sc[4], d16;
  __device__ void load(const uint8_t* c, int r) {
    ldp<192>(q6, c, r); ldp<16>(sc, c + 64 * 192, r);
    d16 = *(const uint16_t*)(c + 64 * 208 + r * 2);
  }
  __device__ void scales(int s, float& scale, float& b) const {
    scale = h2f(d16) * (float)(int8_t)byte_of(sc, s);
    b = 160.f * scale;
  }
  __device__ void pair(int s, int m, uint32_t& b0, uint32_t& b1, const Tabs&, const Masks& k) const {
    const uint32_t* P = q6 + 12 * (s >> 2) + (s & 3);   // P_j = P[4 j]
    const uint32_t u = m < 3 ? P[4 * m] & 0x3F3F3F3Fu
                             : and_or(P[8] >> 2, 0x30303030u, and_or(P[4] >> 4, 0x0C0C0C0Cu, (P[0] >> 6) & 0x03030303u));
    split_bytes(u, k, b0, b1);
  }
};

template <> struct Dec<GQK_IQ4_NL> {
  static constexpr int SUB = 32, FAM = FAM_IQ4, REC = 144;
  uint32_t qs[32], dw[4];
  __device__ void load(const uint8_t* c, int r) { ldp<128>(qs, c, r); ldp<16>(dw, c + 64 * 128, r); }
  __device__ void scales(int s, float& sc, float& b) const { sc = h2f(dw[s >> 1] >> (16 * (s & 1))); b = 0.f; }
  __device__ void pair(int s, int m, uint32_t& b0, uint32_t& b1, const Tabs& tb, const Masks&) const {
    uint32_t w = qs[4 * s + (m >> 1)] >> (16 * (m & 1));
    b0 = tb.iq4[w & 0xFF];
    b1 = tb.iq4[(w >> 8) & 0xFF];
  }
};

template <> struct Dec<GQK_IQ4_XS> {
  static constexpr int SUB = 32, FAM = FAM_IQ4, REC = 136;
  uint32_t qs[32], hdr[2];
  __device__ void load(const uint8_t* c, int r) {
    ldp<128>(qs, c, r);
    uint2 h = *(const uint2*)(c + 64 * 128 + r * 8);
    hdr[0] = h.x; hdr[1] = h.y;
  }
  __device__ void scales(int s, float& sc, float& b) const {
    int ls = ((hdr[1] >> (4 * s)) & 0xF) | (((hdr[0] >> (16 + 2 * s)) & 3) << 4);
    sc = h2f(hdr[0]) * (float)(ls - 32);
    b = 0.f;
  }
  __device__ void pair(int s, int m, uint32_t& b0, uint32_t& b1, const Tabs& tb, const Masks&) const {
    uint32_t w = qs[4 * s + (m >> 1)] >> (16 * (m & 1));
    b0 = tb.iq4[w & 0xFF];
    b1 = tb.iq4[(w >> 8) & 0xFF];
  }
};

template <> struct Dec<GQK_IQ3_S> {
  static constexpr int SUB = 32, FAM = FAM_NAT, REC = 110;
  uint32_t qs[16], sg[8], qh[2], scb, d16;
  __device__ void load(const uint8_t* c, int r) {
    ldp<64>(qs, c, r);
    ldp<32>(sg, c + 64 * 64, r);
    uint2 h = *(const uint2*)(c + 64 * 96 + r * 8);
    qh[0] = h.x; qh[1] = h.y;
    scb = *(const uint32_t*)(c + 64 * 104 + r * 4);
    d16 = *(const uint16_t*)(c + 64 * 108 + r * 2);
  }
  __device__ void scales(int s, float& sc, float& b) const {
    sc = h2f(d16) * (float)(1 + 2 * (int)((scb >> (4 * s)) & 0xF));
    b = 0.f;
  }
  __device__ void pair(int s, int m, uint32_t& b0, uint32_t& b1, const Tabs& tb, const Masks&) const {
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

__device__ __forceinline__ float bf2f(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

// ---- x staging: wave-private, one super-block at a time.  An item is (token t, 32-weight group
// s32): 64 bytes of x loaded with four 16-byte loads, rearranged into the decoder's 8 slots and
// summed (two 16-sums and their 32-sum for the bias terms).
template <int FAM>
__device__ __forceinline__ void slots_of_group(const uint4 (&v)[4], uint2 (&o)[8]) {
  const uint32_t w[16] = {v[0].x, v[0].y, v[0].z, v[0].w, v[1].x, v[1].y, v[1].z, v[1].w,
                          v[2].x, v[2].y, v[2].z, v[2].w, v[3].x, v[3].y, v[3].z, v[3].w};   // k pairs (2j, 2j+1)
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    if (FAM == FAM_NAT) {
      o[m] = make_uint2(w[2 * m], w[2 * m + 1]);
    } else if (FAM == FAM_SWAP) {                  // (4m, 4m+2, 4m+1, 4m+3)
      const uint32_t a = w[2 * m], c = w[2 * m + 1];
      o[m] = make_uint2((a & 0xFFFFu) | (c << 16), (a >> 16) | (c & 0xFFFF0000u));
    } else {                                       // (2m, 2m+16, 2m+1, 2m+17)
      const uint32_t a = w[m], c = w[m + 8];
      o[m] = make_uint2((a & 0xFFFFu) | (c << 16), (a >> 16) | (c & 0xFFFF0000u));
    }
  }
}

// The 4 x 4 x 4 (16 blocks) MFMA with block ab's A operand broadcast to every block (CBSZ = 4,
// ABID = ab), and the 4 x 4 x 1 fp32 one likewise.  ab must fold to a constant (unrolled loops).
#define GQK_AB_CASES(F) F(0) F(1) F(2) F(3) F(4) F(5) F(6) F(7) F(8) F(9) F(10) F(11) F(12) F(13) F(14) F(15)
__device__ __forceinline__ v4f mfma4_bcast(int ab, v4s a, v4s b, v4f c) {
  switch (ab) {
#define GQK_CASE(k) case k: return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(a, b, c, 4, k, 0);
    GQK_AB_CASES(GQK_CASE)
#undef GQK_CASE
  }
  return c;
}
__device__ __forceinline__ v4f mfma1_bcast(int ab, float a, float b, v4f c) {
  switch (ab) {
#define GQK_CASE(k) case k: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, k, 0);
    GQK_AB_CASES(GQK_CASE)
#undef GQK_CASE
  }
  return c;
}
// The same within each half of the wave (CBSZ = 3: blocks 0-7 and 8-15 each take block ab of their
// own half), for the slab form whose lane halves multiply different super-blocks.
#define GQK_AB8_CASES(F) F(0) F(1) F(2) F(3) F(4) F(5) F(6) F(7)
__device__ __forceinline__ v4f mfma4_bcast8(int ab, v4s a, v4s b, v4f c) {
  switch (ab) {
#define GQK_CASE(k) case k: return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(a, b, c, 3, k, 0);
    GQK_AB8_CASES(GQK_CASE)
#undef GQK_CASE
  }
  return c;
}
__device__ __forceinline__ v4f mfma1_bcast8(int ab, float a, float b, v4f c) {
  switch (ab) {
#define GQK_CASE(k) case k: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 3, k, 0);
    GQK_AB8_CASES(GQK_CASE)
#undef GQK_CASE
  }
  return c;
}

// Which x operands a kernel broadcasts from registers (the MFMA operands, the group sums).  Every
// kernel broadcasts both but Q6_K's one-record kernel at G = 2, which keeps both in LDS (0.2 us
// faster on qkv than either; broadcasting both there measured -0.6..+1.5% on qkv / o_proj).  Q6_K's
// streaming kernel at G = 2 takes both in 136 VGPRs (three waves per SIMD, no scratch): gate_up at
// M = 6 / 8 2.4% and down 0.7% faster than with the sums from LDS.
template <int G, int T, bool ONE>
constexpr bool x_broadcast() { return !(G == 2 && T == GQK_Q6_K && ONE); }
template <int G, int T, bool ONE>
constexpr bool xq_broadcast() { return x_broadcast<G, T, ONE>(); }

template <int MPAD>
struct WaveX {            // per-wave LDS: 64 slots x MPAD tokens x 8 B, then 16 + 8 group sums x MPAD
  static constexpr int X = 64 * MPAD * 8;
  static constexpr int BYTES = X + 24 * MPAD * 4;
};

// Order of the x slots in LDS.  Lane 4b + i reads the 8 bytes of token 4g + i at a slot (once per
// 16 slots with the broadcast operands, once per MFMA without).  The orders were chosen when every
// MFMA read its operand from LDS; measured then:  Groups adjacent ([slot][i][g]): the G groups' operands of a lane are
// one 8 G-byte run, a single ds_read_b128 at G = 2 (M = 8: IQ types 7-9% faster, Q4_K 3%, Q5_K 2%;
// M = 16: up to 5%).  Tokens in order ([slot][t]): two 8-byte reads 32 bytes apart (ds_read2_b64);
// kept for Q8_0 and Q5_0, whose one-record kernels measured 4-8% slower with the adjacent order
// (more registers), and for Q6_K, whose G = 2 kernel sits at the three-waves register bound and
// spilled with it.
template <int T>
constexpr bool x_groups_adjacent() { return T != GQK_Q8_0 && T != GQK_Q5_0 && T != GQK_Q6_K; }

// G = 1 has a single group: there the adjacent pair is two consecutive slots of a token
// ([slot / 2][t][slot % 2]), so two MFMAs' operands are one ds_read_b128 (M = 1-4: IQ types 5-9%
// faster, Q4_K 2%).
template <int MPAD, bool XG>
__device__ __forceinline__ int x_slot(int slot, int t) {
  if (XG && MPAD == 4) return ((slot >> 1) * 4 + t) * 2 + (slot & 1);
  return XG ? (slot * 4 + (t & 3)) * (MPAD / 4) + (t >> 2) : slot * MPAD + t;
}

// Issue the loads of super-block kb's x items (clamped addresses; masked when written).
template <int MPAD>
__device__ __forceinline__ void stage_load(const uint16_t* __restrict__ x, int64_t ldx, int M, int kb, int lane,
                                           uint4 (&v)[(8 * MPAD + 63) / 64][4]) {
  constexpr int NI = (8 * MPAD + 63) / 64;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int it = min(lane + 64 * i, 8 * MPAD - 1), t = it % MPAD, s32 = it / MPAD;
    const uint4* p = (const uint4*)(x + min(t, M - 1) * ldx + (int64_t)kb * 256 + 32 * s32);
#pragma unroll
    for (int j = 0; j < 4; ++j) v[i][j] = p[j];
  }
}

// Tokens t >= M hold clamped copies of row M - 1 (stage_load): their slots and sums reach only
// outputs of those tokens, which are never stored, so nothing is masked here.
template <int MPAD, int FAM, bool XG>
__device__ __forceinline__ void stage_store(uint8_t* wl, int lane, const uint4 (&v)[(8 * MPAD + 63) / 64][4]) {
  constexpr int NI = (8 * MPAD + 63) / 64;
  uint2* xs = (uint2*)wl;
  float* xsum16 = (float*)(wl + WaveX<MPAD>::X);
  float* xsum32 = xsum16 + 16 * MPAD;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int it = lane + 64 * i, t = it % MPAD, s32 = it / MPAD;
    if (it < 8 * MPAD) {
      uint2 o[8];
      slots_of_group<FAM>(v[i], o);
      float a = 0.f, b = 0.f;
      const uint32_t* w = (const uint32_t*)&v[i][0];
#pragma unroll
      for (int j = 0; j < 8; ++j) a += bf2f(w[j] & 0xFFFF) + bf2f(w[j] >> 16);
#pragma unroll
      for (int j = 8; j < 16; ++j) b += bf2f(w[j] & 0xFFFF) + bf2f(w[j] >> 16);
#pragma unroll
      for (int m = 0; m < 8; ++m) xs[x_slot<MPAD, XG>(s32 * 8 + m, t)] = o[m];
      xsum16[(2 * s32) * MPAD + t] = a;
      xsum16[(2 * s32 + 1) * MPAD + t] = b;
      xsum32[s32 * MPAD + t] = a + b;
    }
  }
}

template <int G, int T, class P>
__device__ __forceinline__ void gemv_pipeline(const uint8_t* __restrict__ tbase, const uint16_t* __restrict__ x,
                                              int64_t ldx, int M, int kw0, int kw1, uint8_t* wl, int lane,
                                              const P& process);

// One wave: weight rows of tile `tile`, super-blocks [kw0, kw1), accumulating into acc.  ONE: the
// launch guarantees kw1 - kw0 == 1 for every wave (only the pipeline-free path is compiled).
template <int G, int T, bool ONE>
__device__ __forceinline__ void gemv_wave(const uint8_t* __restrict__ tbase, const uint16_t* __restrict__ x,
                                          int64_t ldx, int M, int kw0, int kw1, uint8_t* wl, const Tabs& tb,
                                          const Masks& mk, v4f (&acc)[G]) {
  typedef Dec<T> D;
  constexpr int MPAD = 4 * G, MPS = D::SUB / 4, NSUB = 256 / D::SUB, NI = (8 * MPAD + 63) / 64;
  constexpr bool BIAS = !(T == GQK_IQ4_NL || T == GQK_IQ4_XS || T == GQK_IQ3_S);
  const int lane = threadIdx.x & 63, li = lane & 3;
  const uint2* xs = (const uint2*)wl;
  const float* xsum16 = (const float*)(wl + WaveX<MPAD>::X);
  const float* xsum32 = xsum16 + 16 * MPAD;
  if (kw0 >= kw1) return;

  // The x operands come from registers, 16 slots per register pair: lane 4b + i holds token
  // 4g + i's x at slot 16j + b, and each MFMA broadcasts block (slot % 16)'s operand to all 16
  // blocks (CBSZ = 4, ABID = slot % 16), so a wave reads each slot's x from LDS once instead of
  // once per MFMA.  The group sums likewise: lane 4b + i holds token 4g + i's sum of group b.
  constexpr bool XB = x_broadcast<G, T, ONE>(), XQ = xq_broadcast<G, T, ONE>();
  const int bl = lane >> 2;
  // one record (super-block) of the lane's row: MFMA chains per scale group, fp32 epilogue
  auto process = [&](const D& rec) {
    const float* xsm = (D::SUB == 16 ? xsum16 : xsum32) + (XQ ? min(bl, NSUB - 1) * MPAD : 0);
    float xq[G];
    if constexpr (XQ)
#pragma unroll
      for (int g = 0; g < G; ++g) xq[g] = xsm[4 * g + li];
    uint2 xa[G];
#pragma unroll
    for (int s = 0; s < NSUB; ++s) {
      float scale, bias;
      rec.scales(s, scale, bias);
      v4f C[G];
#pragma unroll
      for (int g = 0; g < G; ++g) C[g] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < MPS; ++m) {
        uint32_t b0, b1;
        rec.pair(s, m, b0, b1, tb, mk);
        v4s B = __builtin_bit_cast(v4s, make_uint2(b0, b1));
        const int slot = s * MPS + m;
        if constexpr (XB) {
          if (slot % 16 == 0)
#pragma unroll
            for (int g = 0; g < G; ++g) xa[g] = xs[x_slot<MPAD, x_groups_adjacent<T>()>(slot + bl, 4 * g + li)];
#pragma unroll
          for (int g = 0; g < G; ++g) C[g] = mfma4_bcast(slot % 16, __builtin_bit_cast(v4s, xa[g]), B, C[g]);
        } else {
#pragma unroll
          for (int g = 0; g < G; ++g) {
            v4s A = __builtin_bit_cast(v4s, xs[x_slot<MPAD, x_groups_adjacent<T>()>(slot, 4 * g + li)]);
            C[g] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(A, B, C[g], 0, 0, 0);
          }
        }
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        if constexpr (BIAS) {
          // acc[i][row] -= sum_x[token i] * bias[row]: an fp32 outer product per 4x4 block
          if constexpr (XQ) acc[g] = mfma1_bcast(s, xq[g], -bias, acc[g]);
          else acc[g] = __builtin_amdgcn_mfma_f32_4x4x1f32(xsm[s * MPAD + 4 * g + li], -bias, acc[g], 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[g][i] = __builtin_fmaf(scale, C[g][i], acc[g][i]);
      }
    }
  };

  if (ONE || (G <= 2 && kw1 - kw0 == 1)) {
    // a single record: no pipeline, so no clamped follow-up loads for the workgroup barrier's
    // vmcnt(0) to wait on (the waves of the K = 5120 shards split 5 ways hold one record each)
    uint4 xs[NI][4];
    D r;
    stage_load<MPAD>(x, ldx, M, kw0, lane, xs);
    r.load(tbase + (int64_t)kw0 * (64 * D::REC), lane);
    stage_store<MPAD, D::FAM, x_groups_adjacent<T>()>(wl, lane, xs);
    process(r);
    return;
  }
  if constexpr (!ONE) gemv_pipeline<G, T>(tbase, x, ldx, M, kw0, kw1, wl, lane, process);
}

// The register pipeline of a wave with two or more records, two super-blocks deep: while record
// kb is decoded, the record (and the x slice) of kb+1 is in flight.  Each step issues x(kb+2) and
// then the record kb+2, so every wait (x of a step before its LDS write, the record before its
// decode) covers exactly the loads it needs under the in-order vmcnt count.  Every load is
// unconditional (addresses clamped to the wave's last super-block, so the tail re-reads it from
// L2) and the buffers rotate by code position, never by copy.  (A third record in flight costs a
// wave per SIMD of occupancy and measured slower for every format; one x buffer, reloaded at the
// start of each step, freed 16 VGPRs at G = 2 and measured 0-9% slower.)
template <int G, int T, class P>
__device__ __forceinline__ void gemv_pipeline(const uint8_t* __restrict__ tbase, const uint16_t* __restrict__ x,
                                              int64_t ldx, int M, int kw0, int kw1, uint8_t* wl, int lane,
                                              const P& process) {
  typedef Dec<T> D;
  constexpr int MPAD = 4 * G, NI = (8 * MPAD + 63) / 64;
  // the wave's record count in a scalar register: the loop's bound and the clamp of its follow-up
  // loads take no VGPR (a VGPR bound spilled here, and its reload's vmcnt(0) at every back edge
  // drained the loads in flight)
  const int n = __builtin_amdgcn_readfirstlane(kw1 - kw0);
  const uint8_t* tw = tbase + (int64_t)kw0 * (64 * D::REC);
  const uint16_t* xw = x + (int64_t)kw0 * 256;
  auto rec = [&](int i) { return tw + (int64_t)min(i, n - 1) * (64 * D::REC); };
  uint4 x0[NI][4], x1[NI][4];
  D r0, r1;
  stage_load<MPAD>(xw, ldx, M, 0, lane, x0);
  r0.load(rec(0), lane);
  stage_load<MPAD>(xw, ldx, M, min(1, n - 1), lane, x1);
  r1.load(rec(1), lane);
  auto step = [&](D& r, uint4 (&xv)[NI][4], int i) {
    stage_store<MPAD, D::FAM, x_groups_adjacent<T>()>(wl, lane, xv);
    process(r);
    stage_load<MPAD>(xw, ldx, M, min(i + 2, n - 1), lane, xv);
    r.load(rec(i + 2), lane);
  };
  for (int i = 0;; i += 2) {
    step(r0, x0, i);
    if (i + 1 >= n) break;
    step(r1, x1, i + 1);
    if (i + 2 >= n) break;
  }
}

// The IQ lookup tables in LDS, built by all blockDim.x threads (any workgroup size).
__device__ void build_tables(uint8_t* lds_tab, int type) {
  const int nt = blockDim.x;
  if (type == GQK_IQ4_NL || type == GQK_IQ4_XS) {
    uint32_t* t4 = (uint32_t*)lds_tab;                    // [256] bf16 pairs (kv[b & 15], kv[b >> 4])
    for (int i = threadIdx.x; i < 256; i += nt) t4[i] = bf16x2((float)c_kvalues[i & 15], (float)c_kvalues[i >> 4]);
  } else if (type == GQK_IQ3_S) {
    uint2* tg = (uint2*)lds_tab;                          // [512] grid magnitudes as bf16 x 4
    uint4* ts = (uint4*)(lds_tab + 512 * 8);              // [256] sign masks of a sign byte
    for (int i = threadIdx.x; i < 512; i += nt) {
      uint32_t gw = c_iq3s_grid[i];
      tg[i] = make_uint2(bf16x2((float)(gw & 0xFF), (float)((gw >> 8) & 0xFF)),
                         bf16x2((float)((gw >> 16) & 0xFF), (float)(gw >> 24)));
    }
    for (int i = threadIdx.x; i < 256; i += nt) {
      uint32_t m[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) m[p] = (((i >> (2 * p)) & 1) << 15) | (((i >> (2 * p + 1)) & 1) << 31);
      ts[i] = make_uint4(m[0], m[1], m[2], m[3]);
    }
  }
}

#define GEMV_TAB_BYTES 9216

// Dynamic LDS of a workgroup of nw waves: nw wave-private x regions, then the IQ tables.
template <int G>
__host__ __device__ constexpr int gemv_lds_bytes(int nw, bool tables) {
  return nw * WaveX<4 * G>::BYTES + (tables ? GEMV_TAB_BYTES : 0);
}

// One workgroup of nw waves (blockDim.x / 64, at most GQK_GEMV_MAX_WAVES) per descriptor row: one
// 64-row tile, its k-range split evenly over the waves, the waves' sums combined through LDS in
// a fixed order.  A tile covered by one row (D_NC = 1) is written to y; a tile shared by D_NC rows
// (split-K) sends its fp32 partial to slot D_SLOT0 + D_SPLIT, and the last workgroup of the tile
// to arrive (counter ctr[D_CTR]) sums the partials in split order, writes y and resets the counter.
typedef __bf16 v8bf_t __attribute__((ext_vector_type(8)));
typedef unsigned v2u_t __attribute__((ext_vector_type(2)));
typedef unsigned v4u_t __attribute__((ext_vector_type(4)));
// 4 x 4 transpose of 16-lane groups across four registers: out[b] at lane 16 c + r = in[c] at
// lane 16 b + r (v_permlane32_swap, then v_permlane16_swap).
__device__ __forceinline__ void xpose4(uint32_t& a0, uint32_t& a1, uint32_t& a2, uint32_t& a3) {
  const v2u_t p = __builtin_amdgcn_permlane32_swap(a0, a2, false, false);
  const v2u_t q = __builtin_amdgcn_permlane32_swap(a1, a3, false, false);
  const v2u_t u = __builtin_amdgcn_permlane16_swap(p[0], q[0], false, false);
  const v2u_t w = __builtin_amdgcn_permlane16_swap(p[1], q[1], false, false);
  a0 = u[0]; a1 = u[1]; a2 = w[0]; a3 = w[1];
}
__device__ __forceinline__ void xpose4f(float& a0, float& a1, float& a2, float& a3) {
  uint32_t b0 = __builtin_bit_cast(uint32_t, a0), b1 = __builtin_bit_cast(uint32_t, a1);
  uint32_t b2 = __builtin_bit_cast(uint32_t, a2), b3 = __builtin_bit_cast(uint32_t, a3);
  xpose4(b0, b1, b2, b3);
  a0 = __builtin_bit_cast(float, b0); a1 = __builtin_bit_cast(float, b1);
  a2 = __builtin_bit_cast(float, b2); a3 = __builtin_bit_cast(float, b3);
}
// Types that take the 16 x 16 x 32 form at G = 4 (9-16 rows).  Measured against the 4 x 4 x 4 form
// on gate_up, down, qkv and o_proj at M = 12 / 16 (three rotating copies): IQ4_NL 8-14% faster,
// IQ4_XS 1-16%, IQ3_S 0-13%, Q8_0 0-8%, Q4_0 3-5% and Q5_0 -4..+4%; Q4_K even and Q5_K 1-6% slower,
// so those two keep the 4 x 4 x 4 form.  At G = 8 (17-32 rows) the form was 3-36% slower than the
// 32 x 128 GEMM for most types and shards.
template <int G, int T>
constexpr bool w16() {
  return G == 4 && (T == GQK_Q4_0 || T == GQK_Q5_0 || T == GQK_Q8_0 || T == GQK_IQ4_NL || T == GQK_IQ3_S ||
                    T == GQK_IQ4_XS);
}

// A operand of one 32-weight group for lane (token, chunk c): 8 bf16 of x in the decoder's slot
// order for slots 2c, 2c + 1 (FAM_NAT: k 8c..8c+7; FAM_SWAP: pairs (4m, 4m+2), (4m+1, 4m+3);
// FAM_IQ4: (2m, 2m+16), (2m+1, 2m+17)).
template <int FAM>
__device__ __forceinline__ v4u_t w16_a(const uint16_t* xr, int c) {
  if constexpr (FAM == FAM_IQ4) {   // slots (2m, 2m+16, 2m+1, 2m+17): k 4c..4c+3 interleaved with 16+4c..
    const uint2 lo = *(const uint2*)(xr + 4 * c), hi = *(const uint2*)(xr + 16 + 4 * c);
    return v4u_t{__builtin_amdgcn_perm(hi.x, lo.x, 0x05040100u), __builtin_amdgcn_perm(hi.x, lo.x, 0x07060302u),
                 __builtin_amdgcn_perm(hi.y, lo.y, 0x05040100u), __builtin_amdgcn_perm(hi.y, lo.y, 0x07060302u)};
  } else {
    const uint4 a = *(const uint4*)(xr + 8 * c);
    if constexpr (FAM == FAM_SWAP)   // (4m, 4m+2, 4m+1, 4m+3)
      return v4u_t{__builtin_amdgcn_perm(a.y, a.x, 0x05040100u), __builtin_amdgcn_perm(a.y, a.x, 0x07060302u),
                   __builtin_amdgcn_perm(a.w, a.z, 0x05040100u), __builtin_amdgcn_perm(a.w, a.z, 0x07060302u)};
    else
      return v4u_t{a.x, a.y, a.z, a.w};
  }
}

// The 16 x 16 x 32 form of a wave (32-weight scale groups, 16 tokens per half): one
// v_mfma_f32_16x16x32_bf16 per row block of 16 rows, token half and group.  x is the A operand,
// loaded straight from global memory (lane 16 c + t: token t, the 8 weights of slots 2c, 2c + 1 in
// the decoder's order; no LDS staging); the weights, decoded one row per lane as in the 4 x 4 x 4
// form, reach the B operand (lane 16 c + r: row 16 b + r) through a 4 x 4 transpose of 16-lane
// groups, and the scales likewise, so the output lane holds its own row r of block b for tokens
// 16 h + 4 c .. + 3.  The group sums of x for the bias term come from one more MFMA against ones.
// acc is returned in the lane-per-row layout of the 4 x 4 x 4 form (a last transpose).
template <int G, int T>
__device__ __forceinline__ void gemv_wave_w16(const uint8_t* __restrict__ tbase, const uint16_t* __restrict__ x,
                                              int64_t ldx, int M, int kw0, int kw1, const Tabs& tb, const Masks& mk,
                                              v4f (&acc)[G]) {
  typedef Dec<T> D;
  constexpr int H = G / 4;
  constexpr bool BIAS = !(T == GQK_IQ4_NL || T == GQK_IQ4_XS || T == GQK_IQ3_S);
  const int lane = threadIdx.x & 63, lr = lane & 15, lc = lane >> 4;
  if (kw0 >= kw1) return;
  const uint16_t* xrow[H];
#pragma unroll
  for (int h = 0; h < H; ++h) xrow[h] = x + (int64_t)min(16 * h + lr, M - 1) * ldx;
  const v8bf_t ones = __builtin_bit_cast(v8bf_t, v4u_t{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
  const int last = kw1 - 1;
  auto recp = [&](int kb) { return tbase + (int64_t)min(kb, last) * (64 * D::REC); };
  auto process = [&](const D& rec, int kb) {
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      v4u_t av[H];
#pragma unroll
      for (int h = 0; h < H; ++h) av[h] = w16_a<D::FAM>(xrow[h] + (int64_t)kb * 256 + 32 * s, lc);
      float sc[4], bi[4];
      rec.scales(s, sc[0], bi[0]);
      sc[1] = sc[2] = sc[3] = sc[0];
      xpose4f(sc[0], sc[1], sc[2], sc[3]);
      if constexpr (BIAS) {
        bi[1] = bi[2] = bi[3] = bi[0];
        xpose4f(bi[0], bi[1], bi[2], bi[3]);
      }
      uint32_t P[4][4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        rec.pair(s, 2 * c, P[c][0], P[c][1], tb, mk);
        rec.pair(s, 2 * c + 1, P[c][2], P[c][3], tb, mk);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) xpose4(P[0][j], P[1][j], P[2][j], P[3][j]);
#pragma unroll
      for (int h = 0; h < H; ++h) {
        const v8bf_t A = __builtin_bit_cast(v8bf_t, av[h]);
        v4f xq = {0.f, 0.f, 0.f, 0.f};
        if constexpr (BIAS) xq = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, ones, xq, 0, 0, 0);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const v8bf_t B = __builtin_bit_cast(v8bf_t, v4u_t{P[b][0], P[b][1], P[b][2], P[b][3]});
          const v4f Dm = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, B, v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float a = __builtin_fmaf(sc[b], Dm[i], acc[4 * h + b][i]);
            if constexpr (BIAS) a = __builtin_fmaf(-bi[b], xq[i], a);
            acc[4 * h + b][i] = a;
          }
        }
      }
    }
  };
  D r0, r1;
  r0.load(recp(kw0), lane);
  r1.load(recp(kw0 + 1), lane);
  for (int kb = kw0;; kb += 2) {
    process(r0, kb);
    r0.load(recp(kb + 2), lane);
    if (kb + 1 > last) break;
    process(r1, kb + 1);
    r1.load(recp(kb + 3), lane);
    if (kb + 2 > last) break;
  }
#pragma unroll
  for (int h = 0; h < H; ++h)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float a0 = acc[4 * h][i], a1 = acc[4 * h + 1][i], a2 = acc[4 * h + 2][i], a3 = acc[4 * h + 3][i];
      xpose4f(a0, a1, a2, a3);
      acc[4 * h][i] = a0; acc[4 * h + 1][i] = a1; acc[4 * h + 2][i] = a2; acc[4 * h + 3][i] = a3;
    }
}

// Minimum waves per SIMD the register allocator must keep (1: no bound).  Q6_K at G = 2 runs
// faster at three waves than at two; it now needs 136 VGPRs, so the bound only keeps a later
// change from trading the third wave for registers.  (Q6_K at G = 4 takes 168 VGPRs, three waves,
// on its own.)
template <int G, int ONLY>
constexpr int gemv_waves() {
  return (G == 2 && ONLY == GQK_Q6_K) ? 3 : 1;
}

template <int G, int ONLY, bool ONE>
__global__ __launch_bounds__(64 * GQK_GEMV_MAX_WAVES) __attribute__((amdgpu_waves_per_eu(ONE ? 1 : gemv_waves<G, ONLY>())))
void gemv_kernel(const uint8_t* __restrict__ packed, const int32_t* __restrict__ desc, const uint16_t* __restrict__ x,
                 int64_t ldx, int M, uint16_t* __restrict__ y, int64_t ldy, const uint16_t* __restrict__ bias,
                 float* __restrict__ part, int* __restrict__ ctr) {
  constexpr int MPAD = 4 * G;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int32_t* dsc = desc + (int64_t)blockIdx.x * GQK_DESC_WORDS;
  const int type = dsc[D_TYPE];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  uint8_t* lds_tab = lds + nw * WaveX<MPAD>::BYTES;
  const bool iq = type == GQK_IQ4_NL || type == GQK_IQ4_XS || type == GQK_IQ3_S;
  Tabs tb{(const uint32_t*)lds_tab, (const uint2*)lds_tab, (const uint4*)(lds_tab + 4096)};
  if (iq) {
    build_tables(lds_tab, type);
    __syncthreads();
  }
  const Masks mk = make_masks();
  const int64_t off = (int64_t)(uint32_t)dsc[D_OFF_LO] | ((int64_t)dsc[D_OFF_HI] << 32);
  const int64_t tile = dsc[D_TILE0];
  const int nb = dsc[D_NB], kb0 = dsc[D_KB0], nk = dsc[D_KB1] - kb0;
  const int kw0 = kb0 + (wave * nk) / nw, kw1 = kb0 + ((wave + 1) * nk) / nw;
  uint8_t* wl = lds + wave * WaveX<MPAD>::BYTES;
  v4f acc[G];
#pragma unroll
  for (int g = 0; g < G; ++g) acc[g] = v4f{0.f, 0.f, 0.f, 0.f};

#define RUN(T)                                                                                           \
  if ((ONLY == 0 || ONLY == T) && type == T) {                                                           \
    if constexpr (w16<G, T>())                                                                           \
      gemv_wave_w16<G, T>(packed + off + tile * nb * (int64_t)(64 * Dec<T>::REC), x, ldx, M, kw0, kw1, tb, mk, acc); \
    else                                                                                                 \
      gemv_wave<G, T, ONE>(packed + off + tile * nb * (int64_t)(64 * Dec<T>::REC), x, ldx, M, kw0, kw1, wl, tb, mk, acc); \
  }
  RUN(GQK_Q4_0) RUN(GQK_Q5_0) RUN(GQK_Q8_0) RUN(GQK_Q2_K) RUN(GQK_Q3_K) RUN(GQK_Q4_K) RUN(GQK_Q5_K) RUN(GQK_Q6_K)
  RUN(GQK_IQ4_NL) RUN(GQK_IQ3_S) RUN(GQK_IQ4_XS)
#undef RUN

  // combine the waves (fixed order) in wave 0
  __syncthreads();                                  // every wave is done with its x region
  v4f* red = (v4f*)lds;                             // [wave][g][lane]
  if (wave > 0)
#pragma unroll
    for (int g = 0; g < G; ++g) red[(wave * G + g) * 64 + lane] = acc[g];
  __syncthreads();
  if (wave > 0) return;
  for (int w = 1; w < nw; ++w)
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g] += red[(w * G + g) * 64 + lane];

  const bool row_ok = lane < dsc[D_NVALID];
  const int64_t col = (int64_t)dsc[D_COL0] + lane;
  // the layer bias (bf16 per output column) joins before the one rounding to bf16
  const float bv = bias != nullptr && row_ok ? __builtin_bit_cast(float, (uint32_t)bias[col] << 16) : 0.f;
  const int nc = dsc[D_NC];   // workgroups sharing this tile
  if (nc == 1) {
    if (row_ok)
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = 4 * g + i;
          if (t < M) y[t * ldy + col] = __builtin_bit_cast(uint16_t, (__bf16)(acc[g][i] + bv));
        }
    return;
  }
  // Split-K exchange.  The nc partials of a tile sit in its slots D_SLOT0 .. D_SLOT0 + nc - 1 as
  // [slot][lane][MPAD] (1 KiB x G per workgroup, written as 16-byte stores).  They move through
  // device-coherent (sc1) buffer accesses only, which write through / bypass the per-XCD L2's
  // non-coherent lines, and the stores complete before the arrival count: no L2-wide writeback
  // or invalidate is needed.
  const int s = dsc[D_SPLIT];
  const int ctr_i = dsc[D_CTR];
  const int split = nc;
  float* tp = part + (int64_t)dsc[D_SLOT0] * 64 * MPAD;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(tp, 0, split * 64 * MPAD * 4, GQK_BUF_WORD3);
#pragma unroll
  for (int g = 0; g < G; ++g)
    __builtin_amdgcn_raw_buffer_store_b128(acc[g], rs, ((s * 64 + lane) * MPAD + 4 * g) * 4, 0, GQK_CPOL_SC1);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the partial stores are complete
  int arrived = 0;
  if (lane == 0) arrived = __hip_atomic_fetch_add(&ctr[ctr_i], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  arrived = __shfl(arrived, 0);
  if (arrived != split - 1) return;
  asm volatile("" ::: "memory");
  // the last workgroup: every partial of the tile, QC splits per round trip, summed in split order
  constexpr int QC = G <= 2 ? 8 : 4;
  v4f a[G];
#pragma unroll
  for (int g = 0; g < G; ++g) a[g] = v4f{0.f, 0.f, 0.f, 0.f};
  for (int q0 = 0; q0 < split; q0 += QC) {
    v4f v[QC][G];
#pragma unroll
    for (int j = 0; j < QC; ++j)
#pragma unroll
      for (int g = 0; g < G; ++g)
        v[j][g] = __builtin_amdgcn_raw_buffer_load_b128(rs, ((min(q0 + j, split - 1) * 64 + lane) * MPAD + 4 * g) * 4,
                                                        0, GQK_CPOL_SC1);
#pragma unroll
    for (int j = 0; j < QC; ++j)
#pragma unroll
      for (int g = 0; g < G; ++g)
        if (q0 + j < split) a[g] += v[j][g];
  }
  if (row_ok)
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 4 * g + i;
        if (t < M) y[t * ldy + col] = __builtin_bit_cast(uint16_t, (__bf16)(a[g][i] + bv));
      }
  if (lane == 0) __hip_atomic_store(&ctr[ctr_i], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // next launch
}

// x of super-block kb through whole 128-byte lines (MPAD = 8): load j (0..3) of lane l reads
// token t = l / 8's 16-byte piece u = 8 j + ((l % 8) ^ ((t >> 1) & 3)), so each load covers 8
// full lines (the item order of stage_load touches 32 lines per load, 32 bytes of each).  The
// pieces go to LDS in lane order (region + 1 KiB j + 16 l), come back in stage_load's item order
// (lane it: token it % 8, 32 weights it / 8; the swizzle puts every quarter-wave's 16 reads in
// distinct banks) and then take the usual stage_store, all within the super-block's own x
// region (the raw pieces are read before any slot is written: a wave's LDS accesses run in
// order).
__device__ __forceinline__ void stage_load_lines(const uint16_t* __restrict__ x, int64_t ldx, int M, int kb, int lane,
                                                 uint4 (&v)[4]) {
  const int t = lane >> 3, c = (lane & 7) ^ ((t >> 1) & 3);
  const uint16_t* p = x + (int64_t)min(t, M - 1) * ldx + (int64_t)kb * 256 + 8 * c;
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = *(const uint4*)(p + 64 * j);
}
__device__ __forceinline__ void stage_lines_to_items(uint8_t* wl, int lane, const uint4 (&v)[4], uint4 (&o)[1][4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) *(uint4*)(wl + 1024 * j + 16 * lane) = v[j];
  const int t = lane & 7, s32 = lane >> 3, f = (t >> 1) & 3;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    o[0][q] = *(const uint4*)(wl + 1024 * (s32 >> 1) + 16 * (8 * t + ((4 * (s32 & 1) + q) ^ f)));
}

// ---- the slab form (M <= 8, shards of at most one 32-row slab per CU): one workgroup per 32-row
// half (D_SPLIT) of a 64-row tile over the whole k-range, one wave per pair of super-blocks (lanes
// 0-31: rows of the slab in super-block 2 w, lanes 32-63: the same rows in 2 w + 1).  The waves'
// sums (two halves per lane row) combine in LDS in a fixed order: no split-K exchange through
// memory.  The x operands and group sums broadcast from
// registers within each half of the wave (the two halves multiply different super-blocks).
// Each wave stages the x of its own two super-blocks (no barrier before the products: a wave
// decodes as soon as its own loads land), and the combine's barriers wait for LDS only
// (s_waitcnt lgkmcnt(0); s_barrier).
static_assert(WaveX<4>::BYTES == GQK_SLAB_SB_BYTES(4) && WaveX<8>::BYTES == GQK_SLAB_SB_BYTES(8) &&
              GEMV_TAB_BYTES == GQK_GEMV_TAB_BYTES, "slab LDS sizes of the planner");
template <int G>
__host__ __device__ constexpr int slab_lds_bytes(int nb, bool tables) {
  return nb * WaveX<4 * G>::BYTES + (tables ? GEMV_TAB_BYTES : 0);
}

__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// One lane's record (row r of the tile in super-block record `c`) against its x region wl.
template <int G, int T>
__device__ __forceinline__ void slab_record(const Dec<T>& rec, const uint8_t* wl, const Tabs& tb, const Masks& mk,
                                            v4f (&acc)[G]) {
  typedef Dec<T> D;
  constexpr int MPAD = 4 * G, MPS = D::SUB / 4, NSUB = 256 / D::SUB;
  constexpr bool BIAS = !(T == GQK_IQ4_NL || T == GQK_IQ4_XS || T == GQK_IQ3_S);
  constexpr bool XG = x_groups_adjacent<T>();
  constexpr int NXQ = (NSUB + 7) / 8;
  const int li = threadIdx.x & 3, bl8 = (threadIdx.x >> 2) & 7;   // the lane's block within its half
  const uint2* xs = (const uint2*)wl;
  const float* xsm = (const float*)(wl + WaveX<MPAD>::X) + (D::SUB == 16 ? 0 : 16 * MPAD);
  // operands broadcast within each half: lane 4 b + i holds token 4 g + i's x at slot 8 j + b % 8
  // and its sum of group 8 k + b % 8
  float xq[G][NXQ];
  if constexpr (BIAS)
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int k = 0; k < NXQ; ++k) xq[g][k] = xsm[(8 * k + bl8) * MPAD + 4 * g + li];
  uint2 xa[G];
#pragma unroll
  for (int s = 0; s < NSUB; ++s) {
    float scale, bias;
    rec.scales(s, scale, bias);
    v4f C[G];
#pragma unroll
    for (int g = 0; g < G; ++g) C[g] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < MPS; ++m) {
      uint32_t b0, b1;
      rec.pair(s, m, b0, b1, tb, mk);
      const v4s B = __builtin_bit_cast(v4s, make_uint2(b0, b1));
      const int slot = s * MPS + m;
      if (slot % 8 == 0)
#pragma unroll
        for (int g = 0; g < G; ++g) xa[g] = xs[x_slot<MPAD, XG>(slot + bl8, 4 * g + li)];
#pragma unroll
      for (int g = 0; g < G; ++g) C[g] = mfma4_bcast8(slot % 8, __builtin_bit_cast(v4s, xa[g]), B, C[g]);
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if constexpr (BIAS) acc[g] = mfma1_bcast8(s % 8, xq[g][s / 8], -bias, acc[g]);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[g][i] = __builtin_fmaf(scale, C[g][i], acc[g][i]);
    }
  }
}

template <int G, int ONLY>
__global__ __launch_bounds__(64 * GQK_SLAB_MAX_WAVES) void gemv_slab_kernel(
    const uint8_t* __restrict__ packed, const int32_t* __restrict__ desc, const uint16_t* __restrict__ x,
    int64_t ldx, int M, uint16_t* __restrict__ y, int64_t ldy, const uint16_t* __restrict__ bias) {
  constexpr int MPAD = 4 * G, NI = (8 * MPAD + 63) / 64;
  __shared__ __attribute__((aligned(16))) uint8_t lds[GQK_SLAB_MAX_LDS];   // x of every super-block, IQ tables
  const int32_t* dsc = desc + (int64_t)blockIdx.x * GQK_DESC_WORDS;
  const int type = dsc[D_TYPE];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int nb = dsc[D_NB];
  uint8_t* lds_tab = lds + nb * WaveX<MPAD>::BYTES;
  const bool iq = type == GQK_IQ4_NL || type == GQK_IQ4_XS || type == GQK_IQ3_S;
  Tabs tb{(const uint32_t*)lds_tab, (const uint2*)lds_tab, (const uint4*)(lds_tab + 4096)};
  if (iq) {
    build_tables(lds_tab, type);
    lds_barrier();
  }
  const Masks mk = make_masks();
  const int64_t off = (int64_t)(uint32_t)dsc[D_OFF_LO] | ((int64_t)dsc[D_OFF_HI] << 32);
  const int64_t tile = dsc[D_TILE0];
  const int h = dsc[D_SPLIT];                        // the slab: rows 32 h .. 32 h + 31 of the tile
  const int q = lane >> 5, r = 32 * h + (lane & 31);
  const int kr = 2 * wave + q;                       // the lane's super-block (nb odd: the last wave's
  const bool dummy = kr >= nb;                       // upper half has none and drops its sums)
  const int kl = dummy ? nb - 1 : kr;
  v4f acc[G];
#pragma unroll
  for (int g = 0; g < G; ++g) acc[g] = v4f{0.f, 0.f, 0.f, 0.f};

#define RUN(T)                                                                                           \
  if ((ONLY == 0 || ONLY == T) && type == T) {                                                           \
    typedef Dec<T> D;                                                                                    \
    const uint8_t* tb0 = packed + off + tile * nb * (int64_t)(64 * D::REC);                            \
    uint4 xv0[NI][4], xv1[NI][4];                                                                        \
    const int s0 = 2 * wave, s1 = min(2 * wave + 1, nb - 1);                                             \
    uint8_t* w0 = lds + s0 * WaveX<MPAD>::BYTES;                                                         \
    uint8_t* w1 = lds + s1 * WaveX<MPAD>::BYTES;                                                         \
    D rec;                                                                                               \
    if constexpr (MPAD == 8) {                                                                           \
      uint4 l0[4], l1[4];                                                                                \
      stage_load_lines(x, ldx, M, s0, lane, l0);                                                         \
      stage_load_lines(x, ldx, M, s1, lane, l1);                                                         \
      rec.load(tb0 + (int64_t)kl * (64 * D::REC), r);                                                    \
      stage_lines_to_items(w0, lane, l0, xv0);                                                           \
      stage_store<MPAD, D::FAM, x_groups_adjacent<T>()>(w0, lane, xv0);                                  \
      if (s1 != s0) {                                                                                    \
        stage_lines_to_items(w1, lane, l1, xv1);                                                         \
        stage_store<MPAD, D::FAM, x_groups_adjacent<T>()>(w1, lane, xv1);                                \
      }                                                                                                  \
    } else {                                                                                             \
      stage_load<MPAD>(x, ldx, M, s0, lane, xv0);                                                        \
      stage_load<MPAD>(x, ldx, M, s1, lane, xv1);                                                        \
      rec.load(tb0 + (int64_t)kl * (64 * D::REC), r);                                                    \
      stage_store<MPAD, D::FAM, x_groups_adjacent<T>()>(w0, lane, xv0);                                  \
      stage_store<MPAD, D::FAM, x_groups_adjacent<T>()>(w1, lane, xv1);                                  \
    }                                                                                                    \
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");                                                   \
    slab_record<G, T>(rec, lds + kl * WaveX<MPAD>::BYTES, tb, mk, acc);                                  \
  }
  RUN(GQK_Q4_0) RUN(GQK_Q5_0) RUN(GQK_Q8_0) RUN(GQK_Q2_K) RUN(GQK_Q3_K) RUN(GQK_Q4_K) RUN(GQK_Q5_K) RUN(GQK_Q6_K)
  RUN(GQK_IQ4_NL) RUN(GQK_IQ3_S) RUN(GQK_IQ4_XS)
#undef RUN
  if (dummy)
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g] = v4f{0.f, 0.f, 0.f, 0.f};

  // combine: each wave's 64 lanes into its own x region (free once its products are done), one
  // barrier, then thread o sums output (token o / 32, row o % 32) over the waves in order, each
  // wave's two halves in order
  v4f* red = (v4f*)(lds + 2 * wave * WaveX<MPAD>::BYTES);   // [g][lane]
#pragma unroll
  for (int g = 0; g < G; ++g) red[g * 64 + lane] = acc[g];
  lds_barrier();
  for (int o = threadIdx.x; o < 32 * MPAD; o += blockDim.x) {
    const int t = o >> 5, rho = o & 31, g = t >> 2, i = t & 3;
    float sum = 0.f;
    for (int w = 0; w < nw; ++w) {
      const float* rw = (const float*)(lds + 2 * w * WaveX<MPAD>::BYTES);
      sum += rw[(g * 64 + rho) * 4 + i];
      sum += rw[(g * 64 + 32 + rho) * 4 + i];
    }
    const int rr = 32 * h + rho;
    if (t < M && rr < dsc[D_NVALID]) {
      const int64_t col = (int64_t)dsc[D_COL0] + rr;
      const float bv = bias != nullptr ? __builtin_bit_cast(float, (uint32_t)bias[col] << 16) : 0.f;
      y[t * ldy + col] = __builtin_bit_cast(uint16_t, (__bf16)(sum + bv));
    }
  }
}

template <int G>
static void launch_slab(int only, dim3 grid, int nw, hipStream_t st, const uint8_t* packed, const int32_t* desc,
                        const uint16_t* x, int64_t ldx, int M, uint16_t* y, int64_t ldy, const uint16_t* bias) {
  const size_t lds = 0;   // static: GQK_SLAB_MAX_LDS (one workgroup per CU)
  const dim3 block(64 * nw);
  switch (only) {
#define C(T) case T: hipLaunchKernelGGL((gemv_slab_kernel<G, T>), grid, block, lds, st, packed, desc, x, ldx, M, y, ldy, bias); return;
    C(GQK_Q4_0) C(GQK_Q5_0) C(GQK_Q8_0) C(GQK_Q2_K) C(GQK_Q3_K) C(GQK_Q4_K) C(GQK_Q5_K) C(GQK_Q6_K)
    C(GQK_IQ4_NL) C(GQK_IQ3_S) C(GQK_IQ4_XS)
#undef C
    default:
      hipLaunchKernelGGL((gemv_slab_kernel<G, 0>), grid, block, lds, st, packed, desc, x, ldx, M, y, ldy, bias);
  }
}

template <int G, bool ONE>
static void launch_g(int only, dim3 grid, int nw, hipStream_t st, const uint8_t* packed, const int32_t* desc,
                     const uint16_t* x, int64_t ldx, int M, uint16_t* y, int64_t ldy, const uint16_t* bias,
                     float* part, int* ctr) {
  const bool iq = only == 0 || only == GQK_IQ4_NL || only == GQK_IQ4_XS || only == GQK_IQ3_S;
  const size_t lds = (size_t)gemv_lds_bytes<G>(nw, iq);
  const dim3 block(64 * nw);
  switch (only) {
#define C(T) case T: hipLaunchKernelGGL((gemv_kernel<G, T, ONE>), grid, block, lds, st, packed, desc, x, ldx, M, y, ldy, bias, part, ctr); return;
    C(GQK_Q4_0) C(GQK_Q5_0) C(GQK_Q8_0) C(GQK_Q2_K) C(GQK_Q3_K) C(GQK_Q4_K) C(GQK_Q5_K) C(GQK_Q6_K)
    C(GQK_IQ4_NL) C(GQK_IQ3_S) C(GQK_IQ4_XS)
#undef C
    default:
      hipLaunchKernelGGL((gemv_kernel<G, 0, ONE>), grid, block, lds, st, packed, desc, x, ldx, M, y, ldy, bias, part, ctr);
  }
}

// types_mask: the single type of every row (> 0) or 0 for a mixed launch
int launch_gemv(const uint8_t* packed, const int32_t* desc, int n_desc, int types_mask, const void* x, int64_t ldx,
                int M, int G, int nw, int bm, int nb, void* y, int64_t ldy, const void* bias, float* partials,
                int* counters, hipStream_t st) {
  dim3 grid(n_desc);
  float* part = partials;
  const uint16_t* xx = (const uint16_t*)x;
  uint16_t* yy = (uint16_t*)y;
  const uint16_t* bb = (const uint16_t*)bias;
  if (bm == GQK_GEMV_SLAB && G == 8) {   // the mid form's slab: its x steps fit a static LDS block
    if (nw != (nb + 1) / 2) return GQK_ERR_FORM;
    return launch_gemv_mid(packed, desc, n_desc, types_mask, x, ldx, M, nw, true, y, ldy, bias, partials, counters, st);
  }
  if (bm == GQK_GEMV_SLAB) {
    // one wave per pair of super-blocks, each staging its own x in LDS
    if (nw != (nb + 1) / 2 || nw > GQK_SLAB_MAX_WAVES || (G != 1 && G != 2) ||
        (G == 1 ? slab_lds_bytes<1>(nb, true) : slab_lds_bytes<2>(nb, true)) > GQK_SLAB_MAX_LDS)
      return GQK_ERR_FORM;
    if (G == 1) launch_slab<1>(types_mask, grid, nw, st, packed, desc, xx, ldx, M, yy, ldy, bb);
    else launch_slab<2>(types_mask, grid, nw, st, packed, desc, xx, ldx, M, yy, ldy, bb);
    return GQK_OK;
  }
  if (nw < 1 || nw > GQK_GEMV_MAX_WAVES) return GQK_ERR_FORM;
  const bool one = bm == 1;
  if (G == 8) return launch_gemv_mid(packed, desc, n_desc, types_mask, x, ldx, M, nw, false, y, ldy, bias, partials, counters, st);
  switch (G) {
#define L(GG)                                                                                              \
    if (one) launch_g<GG, true>(types_mask, grid, nw, st, packed, desc, xx, ldx, M, yy, ldy, bb, part, counters); \
    else launch_g<GG, false>(types_mask, grid, nw, st, packed, desc, xx, ldx, M, yy, ldy, bb, part, counters);
    case 1: L(1) break;
    case 2: L(2) break;
    case 4: L(4) break;
#undef L
    default: return GQK_ERR_FORM;
  }
  return GQK_OK;
}

}  // namespace gqk
