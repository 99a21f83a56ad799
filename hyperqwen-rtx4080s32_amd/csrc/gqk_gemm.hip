// gqk_gemm.hip - the grouped dequant-GEMM (batch rows M > 32, the prefill regime) and the mid
// form (17..32 rows) that shares its decoders.
//
// Replaces the reference's prefill paths: the wide int8 forms of the grouped kernel and, for
// Q4_K / Q5_K, dequantize_tiles + cuBLAS bf16 (gguf-plugin/gluon/interface.py:159-188,
// gguf-plugin/gluon/tiles.py:141-149).  Here one persistent kernel does both: each workgroup
// takes BM x BN output tiles (BM tokens, BN weight rows of one shard) in turn, walks K in steps
// of 64, decodes the step's weights to bf16 in LDS (bf16 = round-to-nearest-even of the exact
// fp32 gguf-py value), stages the activations beside them, and runs v_mfma_f32_32x32x16_bf16
// with fp32 accumulation.  Tiles left over after whole rounds over the workgroups are split
// along K (stream-K) and their partial sums combined in a fixed order.
#include <hip/hip_runtime.h>
#include <algorithm>
#include <numeric>
#include <type_traits>
#include "gqk_common.h"
#include "gqk_internal.h"

namespace gqk {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

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

// ---- tile forms ------------------------------------------------------------------------------
// A workgroup owns BM tokens x BN weight rows (BN / 64 tiles of one shard) and walks K in steps of
// 64.  Forms: 256 x 256 with 8 waves (two per SIMD, one workgroup per CU: M > 128), 128 x 128 /
// 64 x 128 with 4 waves (two workgroups per CU: M 65..128 / 33..64).  Each wave owns a block of
// 32 x 32 v_mfma_f32_32x32x16_bf16 outputs.  Per step each thread decodes 32 weights of one row
// (two runs of 16 at step-local offsets OFF0 / OFF1, per type) and, in the forms that stage x
// through registers, stores activations of one token (the others load x straight into LDS); the
// next steps' loads are in flight during the MFMAs.  LDS: x and weights double-buffered plus the
// IQ3_S tables.

#define GQK_GB_WORD3 0x00020000   // buffer resource word 3: raw untyped dword access
#define GQK_GB_SC1 16             // device-scope cache policy (write through / bypass the XCD L2)
#define GB_K 64
#define GB_LD 72   // LDS row stride in bf16: 144 bytes, so 16 consecutive rows hit 16 distinct bank groups

struct GTabs {
  uint32_t kv[4];          // IQ4 kvalues + 128, four per dword
  const uint32_t* grid;    // IQ3_S grid magnitudes (LDS, 512 words)
  const uint4* sign;       // IQ3_S sign masks of a sign byte: bits 15 / 31 of four bf16 pairs (LDS)
};

// Per-step constants of a decoder (scales and biases of the step's two scale groups, or one),
// computed once per step by prep() and used by each quarter of out().
struct GS {
  float dl0, b0, dl1, b1;
  uint32_t aux;
};

// fma(dl, u_i, bias) for the four unsigned bytes u_i of u -> two bf16 pairs (RNE).  The empty asm
// hides u's known zero bits, so each byte converts with one v_cvt_f32_ubyteN instead of a
// bit-field extract plus a conversion.
__device__ __forceinline__ void cvt4(uint32_t u, float dl, float bias, uint32_t* o) {
  asm("" : "+v"(u));
  o[0] = g_bf16x2(__builtin_fmaf(dl, (float)(u & 0xFF), bias), __builtin_fmaf(dl, (float)((u >> 8) & 0xFF), bias));
  o[1] = g_bf16x2(__builtin_fmaf(dl, (float)((u >> 16) & 0xFF), bias), __builtin_fmaf(dl, (float)(u >> 24), bias));
}
// IQ4 lookup of four nibbles (bytes 0..15 of n): kvalues + 128 as four unsigned bytes
__device__ __forceinline__ uint32_t kv4(uint32_t n, const GTabs& tb) {
  const uint32_t s = n & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(tb.kv[1], tb.kv[0], s);
  const uint32_t hi = __builtin_amdgcn_perm(tb.kv[3], tb.kv[2], s);
  const uint32_t m = ((n >> 3) & 0x01010101u) * 0xFFu;
  return (hi & m) | (lo & ~m);
}
// Q4_K / Q5_K 6-bit scale and min of sub-block j (get_scale_min_k4) from the 12 scale bytes
__device__ __forceinline__ void k4_scale(const uint32_t* hdr, int j, int& sc, int& m) {
  const uint64_t s01 = (uint64_t)hdr[1] | ((uint64_t)hdr[2] << 32);
  if (j < 4) {
    sc = (int)((s01 >> (8 * j)) & 63);
    m = (int)((s01 >> (8 * j + 32)) & 63);
  } else {
    const uint32_t b = (hdr[3] >> (8 * (j - 4))) & 0xFF;   // byte j + 4
    sc = (int)((b & 0xF) | (((s01 >> (8 * (j - 4))) & 0xC0) >> 2));
    m = (int)((b >> 4) | (((s01 >> (8 * j)) & 0xC0) >> 2));
  }
}
// Q4_K / Q5_K constants of step kq: sub-blocks 2 kq (dl0, b0) and 2 kq + 1 (dl1, b1)
__device__ __forceinline__ GS k4_prep(const uint32_t* hdr, int kq) {
  int sc0, m0, sc1, m1;
  k4_scale(hdr, 2 * kq, sc0, m0);
  k4_scale(hdr, 2 * kq + 1, sc1, m1);
  const float d = g_h2f(hdr[0]), dm = g_h2f(hdr[0] >> 16);
  return GS{d * (float)sc0, -(dm * (float)m0), d * (float)sc1, -(dm * (float)m1), 0};
}
// Q3_K signed 6-bit scale i (0..15) from the 12 packed bytes
__device__ __forceinline__ int q3_scale(const uint32_t* sb, int i) {
  const uint64_t s01 = (uint64_t)sb[0] | ((uint64_t)sb[1] << 32);
  const int lo = (int)(((s01 >> (8 * (i & 7))) >> (4 * (i >> 3))) & 0xF);
  const int hi = (int)((sb[2] >> (8 * (i & 3) + 2 * (i >> 2))) & 3);
  return (lo | (hi << 4)) - 32;
}

template <int T> struct B2;
// out(i) of a decoder fills o[2 i], o[2 i + 1], o[8 + 2 i], o[9 + 2 i] unless its B2 sets SEQ
template <class B, class = void> struct b2_seq : std::false_type {};
template <class B> struct b2_seq<B, std::void_t<decltype(B::SEQ)>> : std::integral_constant<bool, B::SEQ> {};

template <> struct B2<GQK_Q4_0> {   // block b = 2 kq + h: low nibbles -> 16 weights, high -> next 16
  uint32_t q[4], d;
  static __device__ int off0(int h) { return 32 * h; }
  static __device__ int off1(int h) { return 32 * h + 16; }
  __device__ void load(const uint8_t* c, int r, int kq, int h) {
    gld<16>(q, col16(c, r, 2 * kq + h)); gld<2>(&d, c + 64 * 128 + r * 16 + 2 * (2 * kq + h));
  }
  __device__ GS prep(int, int) const {
    const float dd = g_h2f(d);
    return GS{dd, -8.f * dd, 0.f, 0.f, 0};
  }
  __device__ void out(const GS& st, int, int, uint32_t (&o)[16], const GTabs&, int i) const {
    cvt4(q[i] & 0x0F0F0F0Fu, st.dl0, st.b0, o + 2 * i);
    cvt4((q[i] >> 4) & 0x0F0F0F0Fu, st.dl0, st.b0, o + 8 + 2 * i);
  }
};

template <> struct B2<GQK_IQ4_NL> {
  uint32_t q[4], d;
  static __device__ int off0(int h) { return 32 * h; }
  static __device__ int off1(int h) { return 32 * h + 16; }
  __device__ void load(const uint8_t* c, int r, int kq, int h) {
    gld<16>(q, col16(c, r, 2 * kq + h)); gld<2>(&d, c + 64 * 128 + r * 16 + 2 * (2 * kq + h));
  }
  __device__ GS prep(int, int) const {
    const float dd = g_h2f(d);
    return GS{dd, -128.f * dd, 0.f, 0.f, 0};
  }
  __device__ void out(const GS& st, int, int, uint32_t (&o)[16], const GTabs& tb, int i) const {
    cvt4(kv4(q[i] & 0x0F0F0F0Fu, tb), st.dl0, st.b0, o + 2 * i);
    cvt4(kv4((q[i] >> 4) & 0x0F0F0F0Fu, tb), st.dl0, st.b0, o + 8 + 2 * i);
  }
};

template <> struct B2<GQK_Q5_0> {
  uint32_t q[4], qh, d;
  static __device__ int off0(int h) { return 32 * h; }
  static __device__ int off1(int h) { return 32 * h + 16; }
  __device__ void load(const uint8_t* c, int r, int kq, int h) {
    const int b = 2 * kq + h;
    gld<16>(q, col16(c, r, b)); gld<4>(&qh, col16(c + 64 * 128, r, b >> 2) + 4 * (b & 3));
    gld<2>(&d, c + 64 * 160 + r * 16 + 2 * b);
  }
  __device__ GS prep(int, int) const {
    const float dd = g_h2f(d);
    return GS{dd, -16.f * dd, 0.f, 0.f, 0};
  }
  __device__ void out(const GS& st, int, int, uint32_t (&o)[16], const GTabs&, int i) const {
    const uint32_t hl = ((((qh >> (4 * i)) & 0xFu) * 0x00204081u) & 0x01010101u) << 4;
    const uint32_t hh = ((((qh >> (16 + 4 * i)) & 0xFu) * 0x00204081u) & 0x01010101u) << 4;
    cvt4((q[i] & 0x0F0F0F0Fu) | hl, st.dl0, st.b0, o + 2 * i);
    cvt4(((q[i] >> 4) & 0x0F0F0F0Fu) | hh, st.dl0, st.b0, o + 8 + 2 * i);
  }
};

template <> struct B2<GQK_Q8_0> {   // block b = 2 kq + h, 32 int8 in two 16-byte columns
  static constexpr bool SEQ = true;   // out(i) fills o[4 i .. 4 i + 3]
  uint32_t q[8], d;
  static __device__ int off0(int h) { return 32 * h; }
  static __device__ int off1(int h) { return 32 * h + 16; }
  __device__ void load(const uint8_t* c, int r, int kq, int h) {
    const int b = 2 * kq + h;
    gld<16>(q, col16(c, r, 2 * b)); gld<16>(q + 4, col16(c, r, 2 * b + 1)); gld<2>(&d, c + 64 * 256 + r * 16 + 2 * b);
  }
  __device__ GS prep(int, int) const {
    const float dd = g_h2f(d);
    return GS{dd, -128.f * dd, 0.f, 0.f, 0};
  }
  __device__ void out(const GS& st, int, int, uint32_t (&o)[16], const GTabs&, int i) const {
    cvt4(q[2 * i] ^ 0x80808080u, st.dl0, st.b0, o + 4 * i);
    cvt4(q[2 * i + 1] ^ 0x80808080u, st.dl0, st.b0, o + 4 * i + 2);
  }
};

template <> struct B2<GQK_Q2_K> {   // groups 2 kq, 2 kq + 1 share the 16 bytes of the row's part h
  uint32_t q[4], scw, dd;
  static __device__ int off0(int h) { return 16 * h; }
  static __device__ int off1(int h) { return 32 + 16 * h; }
  __device__ void load(const uint8_t* c, int r, int kq, int h) {
    gld<16>(q, col16(c, r, 2 * (kq >> 1) + h)); gld<4>(&scw, c + 64 * 64 + r * 16 + 4 * kq); gld<4>(&dd, c + 64 * 80 + r * 4);
  }
  __device__ GS prep(int, int h) const {
    const float d = g_h2f(dd), dmin = g_h2f(dd >> 16);
    const uint32_t s0 = (scw >> (8 * h)) & 0xFF, s1 = (scw >> (8 * (2 + h))) & 0xFF;
    return GS{d * (float)(s0 & 0xF), -(dmin * (float)(s0 >> 4)), d * (float)(s1 & 0xF), -(dmin * (float)(s1 >> 4)), 0};
  }
  __device__ void out(const GS& st, int kq, int, uint32_t (&o)[16], const GTabs&, int i) const {
    const int j0 = 2 * (kq & 1);
    cvt4((q[i] >> (2 * j0)) & 0x03030303u, st.dl0, st.b0, o + 2 * i);
    cvt4((q[i] >> (2 * j0 + 2)) & 0x03030303u, st.dl1, st.b1, o + 8 + 2 * i);
  }
};

template <> struct B2<GQK_Q3_K> {
  uint32_t q[4], hm[4], sb[3], d;
  static __device__ int off0(int h) { return 16 * h; }
  static __device__ int off1(int h) { return 32 + 16 * h; }
  __device__ void load(const uint8_t* c, int r, int kq, int h) {
    gld<16>(q, col16(c, r, 2 * (kq >> 1) + h));
    gld<16>(hm, col16(c + 64 * 64, r, h));
    const uint32_t* p = (const uint32_t*)(c + 64 * 96);   // three 4-byte columns
    sb[0] = p[r]; sb[1] = p[64 + r]; sb[2] = p[128 + r];
    gld<2>(&d, c + 64 * 108 + r * 2);
  }
  __device__ GS prep(int kq, int h) const {
    const float dd = g_h2f(d);
    const float dl0 = dd * (float)q3_scale(sb, 4 * kq + h), dl1 = dd * (float)q3_scale(sb, 4 * kq + 2 + h);
    return GS{dl0, -4.f * dl0, dl1, -4.f * dl1, 0};
  }
  __device__ void out(const GS& st, int kq, int, uint32_t (&o)[16], const GTabs&, int i) const {
    const int j0 = 2 * (kq & 1), g0 = 2 * kq;
    const uint32_t u0 = ((q[i] >> (2 * j0)) & 0x03030303u) | (((hm[i] >> g0) & 0x01010101u) << 2);
    const uint32_t u1 = ((q[i] >> (2 * j0 + 2)) & 0x03030303u) | (((hm[i] >> (g0 + 1)) & 0x01010101u) << 2);
    cvt4(u0, st.dl0, st.b0, o + 2 * i);
    cvt4(u1, st.dl1, st.b1, o + 8 + 2 * i);
  }
};

template <> struct B2<GQK_Q4_K> {   // low nibbles: sub-block 2 kq, high: 2 kq + 1; part h = bytes 16h .. 16h + 15
  uint32_t q[4], hdr[4];
  static __device__ int off0(int h) { return 16 * h; }
  static __device__ int off1(int h) { return 32 + 16 * h; }
  __device__ void load(const uint8_t* c, int r, int kq, int h) {
    gld<16>(q, col16(c, r, 2 * kq + h)); gld<16>(hdr, c + 64 * 128 + r * 16);
  }
  __device__ GS prep(int kq, int) const { return k4_prep(hdr, kq); }
  __device__ void out(const GS& st, int, int, uint32_t (&o)[16], const GTabs&, int i) const {
    cvt4(q[i] & 0x0F0F0F0Fu, st.dl0, st.b0, o + 2 * i);
    cvt4((q[i] >> 4) & 0x0F0F0F0Fu, st.dl1, st.b1, o + 8 + 2 * i);
  }
};

template <> struct B2<GQK_Q5_K> {
  uint32_t q[4], qh[4], hdr[4];
  static __device__ int off0(int h) { return 16 * h; }
  static __device__ int off1(int h) { return 32 + 16 * h; }
  __device__ void load(const uint8_t* c, int r, int kq, int h) {
    gld<16>(q, col16(c, r, 2 * kq + h)); gld<16>(qh, col16(c + 64 * 128, r, h)); gld<16>(hdr, c + 64 * 160 + r * 16);
  }
  __device__ GS prep(int kq, int) const { return k4_prep(hdr, kq); }
  __device__ void out(const GS& st, int kq, int, uint32_t (&o)[16], const GTabs&, int i) const {
    cvt4((q[i] & 0x0F0F0F0Fu) | (((qh[i] >> (2 * kq)) & 0x01010101u) << 4), st.dl0, st.b0, o + 2 * i);
    cvt4(((q[i] >> 4) & 0x0F0F0F0Fu) | (((qh[i] >> (2 * kq + 1)) & 0x01010101u) << 4), st.dl1, st.b1, o + 8 + 2 * i);
  }
};

// Q6_K from the re-packed six-bit plane: step kq's 16-weight groups 4 kq .. 4 kq + 3 sit in columns
// 3 kq .. 3 kq + 2 (dword d of column 3 kq + m = P_m of group 4 kq + d); part h takes groups
// 4 kq + 2 h and 4 kq + 2 h + 1, dwords 2 h, 2 h + 1: 8 contiguous bytes of each column
template <> struct B2<GQK_Q6_K> {
  uint32_t P[3][2], scw, d;
  static __device__ int off0(int h) { return 32 * h; }
  static __device__ int off1(int h) { return 32 * h + 16; }
  __device__ void load(const uint8_t* c, int r, int kq, int h) {
#pragma unroll
    for (int m = 0; m < 3; ++m) gld<8>(P[m], col16(c, r, 3 * kq + m) + 8 * h);
    gld<4>(&scw, c + 64 * 192 + r * 16 + 4 * kq); gld<2>(&d, c + 64 * 208 + r * 2);
  }
  __device__ GS prep(int, int h) const {
    const float dd = g_h2f(d);
    const float dl0 = dd * (float)(int8_t)((scw >> (16 * h)) & 0xFF), dl1 = dd * (float)(int8_t)((scw >> (16 * h + 8)) & 0xFF);
    return GS{dl0, -32.f * dl0, dl1, -32.f * dl1, 0};
  }
  // weights 4 i .. 4 i + 3 of the part's group j (0, 1) as four bytes
  __device__ uint32_t q4(int j, int i) const {
    if (i < 3) return P[i][j] & 0x3F3F3F3Fu;
    return ((P[0][j] >> 6) & 0x03030303u) | ((P[1][j] >> 4) & 0x0C0C0C0Cu) | ((P[2][j] >> 2) & 0x30303030u);
  }
  __device__ void out(const GS& st, int, int, uint32_t (&o)[16], const GTabs&, int i) const {
    cvt4(q4(0, i), st.dl0, st.b0, o + 2 * i);
    cvt4(q4(1, i), st.dl1, st.b1, o + 8 + 2 * i);
  }
};

template <> struct B2<GQK_IQ4_XS> {
  uint32_t q[4], hdr[2];
  static __device__ int off0(int h) { return 32 * h; }
  static __device__ int off1(int h) { return 32 * h + 16; }
  __device__ void load(const uint8_t* c, int r, int kq, int h) {
    gld<16>(q, col16(c, r, 2 * kq + h)); gld<8>(hdr, c + 64 * 128 + r * 8);
  }
  __device__ GS prep(int kq, int h) const {
    const int g = 2 * kq + h;
    const int ls = (int)(((hdr[1] >> (4 * g)) & 0xF) | (((hdr[0] >> (16 + 2 * g)) & 3) << 4));
    const float dl = g_h2f(hdr[0]) * (float)(ls - 32);
    return GS{dl, -128.f * dl, 0.f, 0.f, 0};
  }
  __device__ void out(const GS& st, int, int, uint32_t (&o)[16], const GTabs& tb, int i) const {
    cvt4(kv4(q[i] & 0x0F0F0F0Fu, tb), st.dl0, st.b0, o + 2 * i);
    cvt4(kv4((q[i] >> 4) & 0x0F0F0F0Fu, tb), st.dl0, st.b0, o + 8 + 2 * i);
  }
};

template <> struct B2<GQK_IQ3_S> {   // group g = 2 kq + h: 32 weights, magnitudes from the grid, signs as bf16 masks
  static constexpr bool SEQ = true;   // out(i) fills o[4 i .. 4 i + 3]
  uint32_t qs[2], sg, qh[2], scb, d;
  static __device__ int off0(int h) { return 32 * h; }
  static __device__ int off1(int h) { return 32 * h + 16; }
  __device__ void load(const uint8_t* c, int r, int kq, int h) {
    const int g = 2 * kq + h;
    gld<8>(qs, col16(c, r, g >> 1) + 8 * (g & 1));
    gld<4>(&sg, col16(c + 64 * 64, r, g >> 2) + 4 * (g & 3));
    gld<8>(qh, c + 64 * 96 + r * 8);
    gld<4>(&scb, c + 64 * 104 + r * 4);
    gld<2>(&d, c + 64 * 108 + r * 2);
  }
  __device__ GS prep(int kq, int h) const {
    const int g = 2 * kq + h;
    const float dl = g_h2f(d) * (float)(1 + 2 * (int)((scb >> (4 * g)) & 0xF));
    const uint32_t qhb = (uint32_t)(((uint64_t)qh[0] | ((uint64_t)qh[1] << 32)) >> (8 * g)) & 0xFF;
    return GS{dl, 0.f, 0.f, 0.f, qhb};
  }
  __device__ void out(const GS& st, int, int, uint32_t (&o)[16], const GTabs& tb, int i) const {
    const float dl = st.dl0;
    const uint32_t qhb = st.aux;
    {
      const int l = i;
      const uint32_t qsw = qs[l >> 1] >> (16 * (l & 1));
      const uint32_t i1 = (qsw & 0xFF) | ((qhb << (8 - 2 * l)) & 256);
      const uint32_t i2 = ((qsw >> 8) & 0xFF) | ((qhb << (7 - 2 * l)) & 256);
      const uint4 sm = tb.sign[(sg >> (8 * l)) & 0xFF];
      uint32_t p[4];
      cvt4(tb.grid[i1], dl, 0.f, p);
      cvt4(tb.grid[i2], dl, 0.f, p + 2);
      o[4 * l] = p[0] ^ sm.x; o[4 * l + 1] = p[1] ^ sm.y; o[4 * l + 2] = p[2] ^ sm.z; o[4 * l + 3] = p[3] ^ sm.w;
    }
  }
};

// LDS bytes of the IQ3_S tables (after the tiles)
#define GB_TAB_BYTES (512 * 4 + 256 * 16)

// Where a tile's accumulators go: straight to y (part == nullptr), or - for a tile whose k-steps
// are shared by several workgroups (stream-K) - to this workgroup's fp32 partial slot, the last
// contributor to arrive summing every slot in k order (deterministic) and writing y.
struct GOut {
  float* part;   // partial slots, BM x BN fp32 each
  int* ctr;      // the tile's arrival counter (zero at rest, reset by the last contributor)
  int slot0;     // slot of the tile's first contributor
  int nc;        // contributors
  int self;      // this workgroup's index among them
};

// Tile geometry: BM tokens x BN weight rows per tile, a WGM x WGN grid of waves each owning
// (BM / WGM) x (BN / WGN) outputs in 32 x 32 MFMA blocks.  Thread t decodes part t & 1 of weight
// row t >> 1 each step.  x is staged one of two ways: through registers (AV 16-byte chunks per
// thread, loaded XD steps ahead, stored to padded LDS rows), or with XDMA by direct-to-LDS loads
// (global_load_lds_dwordx4: a wave's instruction writes 1 KiB of LDS, 16 bytes per lane in lane
// order) one step ahead into dense 128-byte token rows whose 16-byte chunks are XOR-swizzled.
template <int BM_, int BN_, int WGM_, int WGN_, int XD_, int WD_, bool XDMA_ = false>
struct Geo {
  static constexpr int BM = BM_, BN = BN_, WGM = WGM_, WGN = WGN_, NW = WGM * WGN, NT = 64 * NW;
  // pipeline depth: x loaded XD steps, weights WD steps before the step that multiplies them.
  // XD >= 2 also moves half of each step's LDS stores to mid-step (the buffer they fill was last
  // read before the previous barrier, and x two steps ahead is already in registers there).
  static constexpr int XD = XD_, WD = WD_, U = XD * WD / std::gcd(XD, WD);   // steps per unrolled trip
  static_assert(XD >= 1 && XD <= 3 && WD >= 2 && WD <= 3 && (U == 2 || U == 3 || U == 6), "pipeline depths");
  static constexpr bool XDMA = XDMA_;
  static constexpr int MB = BM / WGM / 32, NB = BN / WGN / 32;   // 32 x 32 blocks per wave
  static constexpr int AV = BM * 8 / NT;                          // x chunks per thread per step (registers)
  static constexpr int XI = BM * GB_K * 2 / 1024 / NW;            // 1 KiB x loads per wave per step (XDMA)
  static constexpr int XLD = XDMA ? GB_K : GB_LD;                 // LDS x row stride in bf16
  static constexpr int CH = MB * NB * 4;                          // 16-byte accumulator chunks per thread
  static constexpr int SLOT = BM * BN;                            // floats per partial slot
  static constexpr int LDS = 2 * (BM * XLD + BN * GB_LD) * 2;     // double-buffered x and weights
  static constexpr int WPE = 2;                                   // waves per SIMD kept resident
  static_assert(BN * 2 == NT, "one thread per (weight row, part)");
  static_assert(AV >= 1 && 8 % AV == 0, "x chunks per thread");
  static_assert(!XDMA || (XI >= 1 && XI * NW * 8 == BM), "whole 8-row x loads per wave");
};
// (x / weight prefetch depths of 2 / 2, 3 / 3 and 1 / 3 for the two smaller forms measured the
// same as 1 / 2 within noise.)
typedef Geo<256, 256, 4, 2, 2, 2> GeoBig;          // M > 128: 8 waves, one workgroup per CU
typedef Geo<128, 128, 2, 2, 1, 2, true> GeoMid;    // 65..128 tokens: 4 waves, two workgroups per CU
typedef Geo<64, 128, 2, 2, 1, 2> GeoSmall;         // 33..64 tokens
// x by direct-to-LDS loads (XDMA), measured against the register path on both 34816 x 5120 and
// 5120 x 17408 shards for all eleven types: the 128 x 128 form 1-13% faster at M = 100 (every
// type but Q5_0, even there); the 256 x 256 form 3-7% faster for Q3_K, Q4_K and IQ4_NL at
// M = 512 / 2048 and 1-6% slower for Q4_0, Q5_0, Q8_0, Q2_K and Q6_K; the 64 x 128 form even to
// 2-7% slower.  The direct loads go one step ahead (the register path's big form
// two), and the compiler completes them with a vmcnt(0) at the step's barrier, which also waits
// for the weight loads in flight; a variant that issued them from inline asm (no compiler wait)
// with weights three steps ahead measured no faster.
// The 256 x 256 tile with its 8 waves 2 x 4 (128 tokens x 64 rows each) instead of 4 x 2: the
// same fragment reads per step, another LDS access and register schedule.  Measured on both
// 34816 x 5120 and 5120 x 17408 shards at M = 512 / 2048 / 8192, it is 2-7% faster for Q5_0,
// Q5_K, Q6_K and IQ4_XS and 1-5% slower for Q4_0, Q8_0, Q3_K, Q4_K, IQ4_NL and IQ3_S (Q2_K
// even), so each type takes the faster grid.  A 8 x 1 grid was slower for every type tried.
typedef Geo<256, 256, 2, 4, 2, 2> GeoBigWide;
typedef Geo<256, 256, 4, 2, 2, 2, true> GeoBigDma;
template <class GE, int T> struct geo_of { typedef GE type; };
template <int T> struct geo_of<GeoBig, T> {
  typedef std::conditional_t<T == GQK_Q5_0 || T == GQK_Q5_K || T == GQK_Q6_K || T == GQK_IQ4_XS, GeoBigWide,
                             std::conditional_t<T == GQK_Q3_K || T == GQK_Q4_K || T == GQK_IQ4_NL, GeoBigDma, GeoBig>>
      type;
};

template <int S, class V>
__device__ __forceinline__ V& pick(V& a, V& b, V& c) {
  if constexpr (S == 0) return a;
  else if constexpr (S == 1) return b;
  else return c;
}

template <class GE, int T>
__device__ __forceinline__ void gemm_tile_sk(const uint8_t* __restrict__ packed, const int32_t* __restrict__ dsc,
                                             const uint16_t* __restrict__ x, int64_t ldx, int M, int m0, int k0,
                                             int k1, const GOut& go, uint16_t* __restrict__ y, int64_t ldy,
                                             const uint16_t* __restrict__ bias, uint16_t* As, uint16_t* Bs, int* flag,
                                             const GTabs& tb) {
  constexpr int REC = gqk_layout<T>::REC;
  constexpr int MB = GE::MB, NB = GE::NB, AV = GE::AV, NT = GE::NT;
  constexpr int WTM = GE::BM / GE::WGM, WTN = GE::BN / GE::WGN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % GE::WGM, wn = wave / GE::WGM;
  const int nb = dsc[D_NB], ntiles = dsc[D_NTILES];
  const int64_t off = (int64_t)(uint32_t)dsc[D_OFF_LO] | ((int64_t)dsc[D_OFF_HI] << 32);
  const int64_t tile0 = dsc[D_TILE0];

  // weight role: row br of the tile's BN rows, part h of the step's 64 weights
  const int br = tid >> 1, h = tid & 1;
  const int btile = br >> 6, brow = br & 63;
  const uint8_t* bbase = packed + off + (tile0 + (btile < ntiles ? btile : 0)) * nb * (int64_t)(64 * REC);
  // activation role (registers): AV consecutive 16-byte chunks (8 k each) of token ar
  const int ar = tid * AV / 8, ac = (tid * AV) % 8;
  const uint16_t* abase = x + (int64_t)min(m0 + ar, M - 1) * ldx + 8 * ac;
  // activation role (XDMA): load i of wave w fills token rows 8 (w XI + i) .. + 7 of the step's x
  // buffer; lane l writes row 8 (w XI + i) + l / 8, chunk slot l % 8, with the k-chunk
  // (l % 8) ^ swz(row), swz(row) = (row >> 1) & 7: the 16 rows a ds_read_b128 quarter-wave reads
  // at one k-chunk then fall in 16 distinct 16-byte bank groups of the 256-byte bank width.
  const uint16_t* xsrc[GE::XDMA ? GE::XI : 1];
  if constexpr (GE::XDMA) {
#pragma unroll
    for (int i = 0; i < GE::XI; ++i) {
      const int row = 8 * (wave * GE::XI + i) + (lane >> 3);
      xsrc[i] = x + (int64_t)min(m0 + row, M - 1) * ldx + 8 * ((lane & 7) ^ ((row >> 1) & 7));
    }
  }

  v16f acc[MB][NB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // Software pipeline over the k-steps [k0, k1): at step s the MFMAs read LDS buffer (s - k0) & 1
  // while the same wave decodes the weights of step s + 1 (loaded one step earlier) into the other
  // buffer, a quarter after each 16-k slice of MFMAs, and the loads of step s + 2's weights and
  // step s + 1's activations are in flight.  One barrier per step.  Loads are unconditional
  // (clamped to the last step).  Rows past M (x) and past the shard's rows (weights) hold clamped
  // copies of real data: they only reach accumulator entries that are never stored.
  const int last = k1 - 1;
  constexpr int XD = GE::XD, WD = GE::WD;
  // x of steps s + 1 .. s + XD and weights of steps s + 1 .. s + WD in flight (set j holds the
  // steps j mod XD, j mod WD); separate variables picked at compile time, so they stay in registers
  struct XS { v4u v[AV]; };   // clang vectors (not uint4's union), so the sets stay in registers
  XS x0, x1, x2;
  B2<T> w0, w1, w2;
  // register sets are picked by compile-time index (S: std::integral_constant)
  auto xload = [&](auto S, int s) __attribute__((always_inline)) {
    const v4u* ap = (const v4u*)(abase + (int64_t)s * GB_K);
#pragma unroll
    for (int i = 0; i < AV; ++i) pick<decltype(S)::value>(x0, x1, x2).v[i] = ap[i];
  };
  auto xstore = [&](auto S, int buf) __attribute__((always_inline)) {
    v4u* as = (v4u*)(As + (buf * GE::BM + ar) * GB_LD + 8 * ac);
#pragma unroll
    for (int i = 0; i < AV; ++i) as[i] = pick<decltype(S)::value>(x0, x1, x2).v[i];
  };
  // XDMA: step s's x into LDS buffer buf (the LDS address is wave-uniform; the hardware adds
  // 16 bytes per lane).  Complete at the s_waitcnt vmcnt(0) before the step's barrier.
  auto xdma = [&](int buf, int s) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < GE::XI; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(xsrc[i] + (int64_t)s * GB_K),
                                       (__attribute__((address_space(3))) void*)(As + (buf * GE::BM + 8 * (wave * GE::XI + i)) * GB_K),
                                       16, 0, 0);
  };
  auto wload = [&](auto S, int s) __attribute__((always_inline)) {
    pick<decltype(S)::value>(w0, w1, w2).load(bbase + (int64_t)(s >> 2) * (64 * REC), brow, s & 3, h);
  };
  auto wprep = [&](auto S, int s) __attribute__((always_inline)) { return pick<decltype(S)::value>(w0, w1, w2).prep(s & 3, h); };
  auto wdecode = [&](auto S, const GS& st, int s, uint32_t (&o)[16], int i) {
    pick<decltype(S)::value>(w0, w1, w2).out(st, s & 3, h, o, tb, i);
  };
  auto wstore = [&](const uint32_t (&o)[16], int buf) {
    uint16_t* bs = Bs + (buf * GE::BN + br) * GB_LD;
    uint4* d0 = (uint4*)(bs + B2<T>::off0(h));
    uint4* d1 = (uint4*)(bs + B2<T>::off1(h));
    d0[0] = make_uint4(o[0], o[1], o[2], o[3]);
    d0[1] = make_uint4(o[4], o[5], o[6], o[7]);
    d1[0] = make_uint4(o[8], o[9], o[10], o[11]);
    d1[1] = make_uint4(o[12], o[13], o[14], o[15]);
  };
  // half P of the decoded weights, complete after quarters 2P and 2P + 1 of out(): o[4P .. 4P+3]
  // and o[8+4P .. 8+4P+3], or o[8P .. 8P+7] for a decoder that fills o in order (SEQ)
  auto wstore_half = [&](const uint32_t (&o)[16], int buf, auto P) {
    constexpr int p = decltype(P)::value;
    uint16_t* bs = Bs + (buf * GE::BN + br) * GB_LD;
    if constexpr (b2_seq<B2<T>>::value) {
      uint4* d = (uint4*)(bs + (p == 0 ? B2<T>::off0(h) : B2<T>::off1(h)));
      d[0] = make_uint4(o[8 * p], o[8 * p + 1], o[8 * p + 2], o[8 * p + 3]);
      d[1] = make_uint4(o[8 * p + 4], o[8 * p + 5], o[8 * p + 6], o[8 * p + 7]);
    } else {
      ((uint4*)(bs + B2<T>::off0(h)))[p] = make_uint4(o[4 * p], o[4 * p + 1], o[4 * p + 2], o[4 * p + 3]);
      ((uint4*)(bs + B2<T>::off1(h)))[p] = make_uint4(o[8 + 4 * p], o[9 + 4 * p], o[10 + 4 * p], o[11 + 4 * p]);
    }
  };
  // step s = k0 + j (mod U): the sets that held step s (x stored, weights decoded during step
  // s - 1) take the loads of steps s + XD and s + WD.
  auto step = [&](auto J, int s) __attribute__((always_inline)) {
    constexpr int j = decltype(J)::value;
    const int buf = (s - k0) & 1;
    if constexpr (GE::XDMA) {
      if (s + 1 < k1) xdma(buf ^ 1, s + 1);
    } else {
      xload(std::integral_constant<int, j % XD>{}, min(s + XD, last));
    }
    wload(std::integral_constant<int, j % WD>{}, min(s + WD, last));
    const uint16_t* as = As + (buf * GE::BM + wm * WTM + (lane & 31)) * GE::XLD + (GE::XDMA ? 0 : 8 * (lane >> 5));
    const uint16_t* bs = Bs + (buf * GE::BN + wn * WTN + (lane & 31)) * GB_LD + 8 * (lane >> 5);
    const int swz = ((lane & 31) >> 1) & 7;   // XDMA row swizzle: the same for every 32-row block
    uint32_t o[16];
    GS st;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      v8bf af[MB], bf[NB];
#pragma unroll
      for (int i = 0; i < MB; ++i)
        af[i] = *(const v8bf*)(as + 32 * i * GE::XLD + (GE::XDMA ? 8 * ((2 * kk + (lane >> 5)) ^ swz) : 16 * kk));
#pragma unroll
      for (int j2 = 0; j2 < NB; ++j2) bf[j2] = *(const v8bf*)(bs + 32 * j2 * GB_LD + 16 * kk);
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j2 = 0; j2 < NB; ++j2)
          acc[i][j2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[j2], acc[i][j2], 0, 0, 0);
      if (kk == 0) st = wprep(std::integral_constant<int, (j + 1) % WD>{}, s + 1);   // after the first MFMAs
      wdecode(std::integral_constant<int, (j + 1) % WD>{}, st, s + 1, o, kk);
      // With x loaded two steps ahead (the 256 x 256 form), the other buffer's stores go out
      // mid-step: it was last read before the previous barrier.  Half the weights and x after
      // the second MFMA slice, the rest at the end (measured: +4-6% at M = 2048; the forms
      // with one-step x loads ran slower that way, their x may still be in flight here).
      if constexpr (XD >= 2) {
        if (kk == 1) {
          wstore_half(o, buf ^ 1, std::integral_constant<int, 0>{});
          if constexpr (!GE::XDMA) xstore(std::integral_constant<int, (j + 1) % XD>{}, buf ^ 1);
        }
      }
    }
    if constexpr (XD >= 2) {
      wstore_half(o, buf ^ 1, std::integral_constant<int, 1>{});
    } else {
      if constexpr (!GE::XDMA) xstore(std::integral_constant<int, (j + 1) % XD>{}, buf ^ 1);
      wstore(o, buf ^ 1);
    }
    if constexpr (GE::XDMA) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wave's x loads are in LDS
    __syncthreads();
  };

  if constexpr (GE::XDMA) {
    xdma(0, k0);
  } else {
    xload(std::integral_constant<int, 0>{}, k0);
    if constexpr (XD > 1) xload(std::integral_constant<int, 1>{}, min(k0 + 1, last));
    if constexpr (XD > 2) xload(std::integral_constant<int, 2>{}, min(k0 + 2, last));
  }
  wload(std::integral_constant<int, 0>{}, k0);
  wload(std::integral_constant<int, 1>{}, min(k0 + 1, last));
  if constexpr (WD > 2) wload(std::integral_constant<int, 2>{}, min(k0 + 2, last));
  {
    uint32_t o[16];
    if constexpr (!GE::XDMA) xstore(std::integral_constant<int, 0>{}, 0);
    const GS st = wprep(std::integral_constant<int, 0>{}, k0);
#pragma unroll
    for (int i = 0; i < 4; ++i) wdecode(std::integral_constant<int, 0>{}, st, k0, o, i);
    wstore(o, 0);
  }
  if constexpr (GE::XDMA) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  // U = lcm(XD, WD) steps per trip, so every set index is a constant; then the last k1 - s < U
  int s = k0;
  for (; s + GE::U <= k1; s += GE::U) {
    step(std::integral_constant<int, 0>{}, s);
    step(std::integral_constant<int, 1>{}, s + 1);
    if constexpr (GE::U > 2) step(std::integral_constant<int, 2>{}, s + 2);
    if constexpr (GE::U > 3) {
      step(std::integral_constant<int, 3>{}, s + 3);
      step(std::integral_constant<int, 4>{}, s + 4);
      step(std::integral_constant<int, 5>{}, s + 5);
    }
  }
  if (s < k1) {
    step(std::integral_constant<int, 0>{}, s);
    if constexpr (GE::U > 2)
      if (s + 1 < k1) step(std::integral_constant<int, 1>{}, s + 1);
    if constexpr (GE::U > 3) {
      if (s + 2 < k1) step(std::integral_constant<int, 2>{}, s + 2);
      if (s + 3 < k1) step(std::integral_constant<int, 3>{}, s + 3);
      if (s + 4 < k1) step(std::integral_constant<int, 4>{}, s + 4);
    }
  }

  // C block (i, j): lane -> weight row 32 j + (lane & 31), tokens 8 (v / 4) + 4 (lane / 32) + v % 4
  const int nvalid = dsc[D_NVALID];
  const int64_t col0 = dsc[D_COL0];
  auto store_y = [&](int i, int j, const v16f& a) {
    const int r = wn * WTN + 32 * j + (lane & 31);
    if (r >= nvalid) return;
    // the layer bias (bf16 per output column) joins before the one rounding to bf16
    const float bv = bias != nullptr ? __builtin_bit_cast(float, (uint32_t)bias[col0 + r] << 16) : 0.f;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int t = m0 + wm * WTM + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
      if (t < M) y[(int64_t)t * ldy + col0 + r] = __builtin_bit_cast(uint16_t, (__bf16)(a[v] + bv));
    }
  };
  if (go.part == nullptr) {
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j) store_y(i, j, acc[i][j]);
    return;
  }
  // Partial slot layout: chunk (i, j, e) = elements 4 e .. 4 e + 3 of acc[i][j] (four consecutive
  // tokens of one weight row) of thread tid at ((slot * CH + (i NB + j) 4 + e) * NT + tid) * 16, so
  // every store and load is coalesced.  Chunks of tokens >= M or rows >= nvalid are not written.
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      go.part + (int64_t)go.slot0 * GE::SLOT, 0, go.nc * GE::SLOT * 4, GQK_GB_WORD3);
  auto live = [&](int i, int j, int e) {
    return m0 + wm * WTM + 32 * i + 8 * e + 4 * (lane >> 5) < M && wn * WTN + 32 * j + (lane & 31) < nvalid;
  };   // chunks that reach y
  auto own = [&](int i, int j, int e) {
    const v16f& a = acc[i][j];
    return v4f{a[4 * e], a[4 * e + 1], a[4 * e + 2], a[4 * e + 3]};
  };
  auto slot_off = [&](int q, int i, int j, int e) { return ((q * GE::CH + (i * NB + j) * 4 + e) * NT + tid) * 16; };
  // Contributors count themselves on the tile's counter once their partial is complete; the last
  // one sums.  A contributor that finds the other nc - 1 already counted is the last for sure: it
  // skips writing its own partial and sums at once.
  if (tid == 0) *flag = __hip_atomic_load(go.ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  const bool last_now = *flag == go.nc - 1;
  __syncthreads();
  if (!last_now) {
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (live(i, j, e)) __builtin_amdgcn_raw_buffer_store_b128(own(i, j, e), rs, slot_off(go.self, i, j, e), 0, GQK_GB_SC1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this workgroup's partial is complete
    __syncthreads();
    if (tid == 0) *flag = __hip_atomic_fetch_add(go.ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (*flag != go.nc - 1) return;
  }
  asm volatile("" ::: "memory");
  // the last contributor: slot 0 + slot 1 + ... in k order (its own from registers), one 32 x 32
  // block at a time, the loads of QB slots in flight together.  Loads are unconditional (slot
  // clamped to the last): chunks never written only reach sums that are never stored.
  constexpr int QB = GE::CH >= 32 ? 2 : 4;
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      v4f sum[4];
      for (int q0 = 0; q0 < go.nc; q0 += QB) {
        v4f t[QB][4];
#pragma unroll
        for (int b = 0; b < QB; ++b)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            t[b][e] = __builtin_amdgcn_raw_buffer_load_b128(rs, slot_off(min(q0 + b, go.nc - 1), i, j, e), 0, GQK_GB_SC1);
#pragma unroll
        for (int b = 0; b < QB; ++b) {
          const int q = q0 + b;
          if (q < go.nc) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const v4f v = q == go.self ? own(i, j, e) : t[b][e];
              sum[e] = q == 0 ? v : sum[e] + v;
            }
          }
        }
      }
      const v16f a = {sum[0][0], sum[0][1], sum[0][2], sum[0][3], sum[1][0], sum[1][1], sum[1][2], sum[1][3],
                      sum[2][0], sum[2][1], sum[2][2], sum[2][3], sum[3][0], sum[3][1], sum[3][2], sum[3][3]};
      store_y(i, j, a);
    }
  if (tid == 0) __hip_atomic_store(go.ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // next launch
}

// Tile t -> (descriptor row, token block).  Groups of up to eight token blocks take consecutive
// tile ids, so with tiles dealt round robin to the workgroups and the dispatcher's round robin
// over the eight XCDs, each XCD keeps one token block of x hot in its L2 while the weight blocks
// stream by.
__device__ __forceinline__ void gb_map(int i, int n_desc, int nmb, int& d, int& mb) {
  const int full = (nmb / 8) * 8 * n_desc;
  if (i < full) {
    const int grp = i / (8 * n_desc), r = i % (8 * n_desc);
    mb = grp * 8 + (r & 7);
    d = r >> 3;
  } else {
    const int rem = nmb % 8, r = i - full;
    mb = (nmb / 8) * 8 + r % rem;
    d = r / rem;
  }
}

// Persistent schedule over G workgroups (all resident: two waves per SIMD, so at most 256 registers
// a lane; no workgroup ever waits for another, so residency is a matter of speed only): the first floor(T / G) * G tiles whole,
// dealt round robin; the remaining R tiles' k-steps split evenly over gsk workgroups (stream-K,
// gb_stream_k_workgroups), tiles shared by several workgroups combined through partial slots.
template <class GE, int ONLY>
__global__ __launch_bounds__(GE::NT) __attribute__((amdgpu_waves_per_eu(GE::WPE))) void gemm_sk_kernel(const uint8_t* __restrict__ packed,
                                                          const int32_t* __restrict__ desc, int n_desc,
                                                          const uint16_t* __restrict__ x, int64_t ldx, int M,
                                                          uint16_t* __restrict__ y, int64_t ldy,
                                                          const uint16_t* __restrict__ bias, float* part, int* ctr,
                                                          int G, int gsk) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[GE::LDS + GB_TAB_BYTES + 16];
  uint16_t* As = (uint16_t*)lds;
  uint16_t* Bs = As + 2 * GE::BM * GE::XLD;
  int* flag = (int*)(lds + GE::LDS + GB_TAB_BYTES);
  GTabs tb;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    tb.kv[i] = (uint32_t)(c_kvalues[4 * i] + 128) | ((uint32_t)(c_kvalues[4 * i + 1] + 128) << 8) |
               ((uint32_t)(c_kvalues[4 * i + 2] + 128) << 16) | ((uint32_t)(c_kvalues[4 * i + 3] + 128) << 24);
  uint32_t* grid = (uint32_t*)(lds + GE::LDS);
  uint4* sign = (uint4*)(lds + GE::LDS + 512 * 4);
  tb.grid = grid;
  tb.sign = sign;
  if (ONLY == 0 || ONLY == GQK_IQ3_S) {
    for (int t = threadIdx.x; t < 512; t += GE::NT) grid[t] = c_iq3s_grid[t];
    for (int t = threadIdx.x; t < 256; t += GE::NT) {
      uint32_t m[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) m[p] = (((t >> (2 * p)) & 1) << 15) | (((t >> (2 * p + 1)) & 1) << 31);
      sign[t] = make_uint4(m[0], m[1], m[2], m[3]);
    }
    __syncthreads();
  }
  const int nmb = (M + GE::BM - 1) / GE::BM;
  const int T = n_desc * nmb;
  const int nsteps = 4 * desc[D_NB];
  auto run = [&](int t, int k0, int k1, const GOut& go) {
    int d, mb;
    gb_map(t, n_desc, nmb, d, mb);
    const int32_t* dsc = desc + (int64_t)d * GQK_DESC_WORDS;
    const int type = dsc[D_TYPE];
#define RUN(TY)                                                                                          \
    if ((ONLY == 0 || ONLY == TY) && type == TY)                                                         \
      gemm_tile_sk<GE, TY>(packed, dsc, x, ldx, M, mb * GE::BM, k0, k1, go, y, ldy, bias, As, Bs, flag, tb);
    RUN(GQK_Q4_0) RUN(GQK_Q5_0) RUN(GQK_Q8_0) RUN(GQK_Q2_K) RUN(GQK_Q3_K) RUN(GQK_Q4_K) RUN(GQK_Q5_K) RUN(GQK_Q6_K)
    RUN(GQK_IQ4_NL) RUN(GQK_IQ3_S) RUN(GQK_IQ4_XS)
#undef RUN
  };
  const int tfull = (T / G) * G;
  const int R = T - tfull;
  const int64_t I = (int64_t)R * nsteps;
  const int w = blockIdx.x;
  auto owner = [&](int64_t i) { return (int)(((i + 1) * gsk + I - 1) / I - 1); };   // workgroup of step i
  int64_t it = 0, end = 0;
  if (R > 0 && w < gsk) {
    it = (int64_t)w * I / gsk;
    end = (int64_t)(w + 1) * I / gsk;
  }
  // one call site: whole tiles w, w + G, ... first, then this workgroup's stream-K steps
  for (int t_dp = w;;) {
    int t, k0, k1;
    GOut go{nullptr, nullptr, 0, 1, 0};
    if (t_dp < tfull) {
      t = t_dp;
      k0 = 0;
      k1 = nsteps;
      t_dp += G;
    } else if (it < end) {
      const int r = (int)(it / nsteps);
      k0 = (int)(it % nsteps);
      k1 = (int)min<int64_t>(nsteps, k0 + (end - it));
      t = tfull + r;
      if (k0 != 0 || k1 != nsteps) {
        const int wf = owner((int64_t)r * nsteps), wl = owner((int64_t)r * nsteps + nsteps - 1);
        go = GOut{part, ctr + r, r + wf, wl - wf + 1, w - wf};
      }
      it += k1 - k0;
    } else {
      break;
    }
    run(t, k0, k1, go);
  }
}

// ---- the mid form: 17..32 batch rows -----------------------------------------------------------
// The GEMV's work split (one workgroup per descriptor row: a 64-row tile and a k-range of
// super-blocks that its waves divide; tiles shared by several rows combine fp32 partials in
// split order, the last to arrive writing y) with the GEMM's arithmetic: each weight decoded
// once to bf16 (round-to-nearest-even of the exact fp32 value, the same B2 decoders) straight
// into registers, and v_mfma_f32_32x32x16_bf16 over all 32 tokens.  No LDS staging of weights and
// no barrier in the main loop: lane l acts as decoder thread (row l % 32 and 32 + l % 32, part
// l / 32) of each 64-weight step, which is exactly the MFMA's B-operand layout (column l % 32,
// k-chunk l / 32); its A operand is x of token l % 32 at the same eight k.  One step of weights
// and x is in flight while the previous one is decoded.  x goes through a 4 KiB LDS region of
// the wave: read straight in the A layout, every load touched 32 token rows (32 bytes of each
// 128-byte line), and loaded coalesced (8 whole rows per load) then re-read from LDS the launch
// is 14-20% faster on gate_up (Q4_K, Q6_K, Q8_0, IQ4_XS at M = 32), 20% on Q6_K down, 3-6% on
// qkv and the low-bit down shards, even on Q4_K down / o_proj.  Measured against the 32 x 128
// GEMM tile form it replaced (before the x staging; Q4_K gate_up / qkv / o_proj / down at
// M = 32: 0.87 / 0.86 / 0.84 / 0.76 of its time; Q2_K, Q8_0, Q6_K down 0.80 / 0.77 / 0.86,
// IQ4_XS gate_up 0.94; Q6_K and Q8_0 gate_up 1.04).  Tried: weights two steps ahead (more
// registers, fewer waves: 0-8% slower) and 64 tokens per wave (226-260 VGPRs: 23-45% slower than
// the 64 x 128 GEMM form, which keeps 33..64 rows).
template <int T, int NRB = 2>
__device__ __forceinline__ void mid_wave(const uint8_t* __restrict__ tbase, const uint16_t* __restrict__ x, int64_t ldx,
                                         int M, uint16_t* xl, int kw0, int kw1, int c, int r, const GTabs& tb,
                                         v16f (&acc)[NRB], int r0 = 0) {
  constexpr int REC = gqk_layout<T>::REC;
  if (kw0 >= kw1) return;
  // k offsets (within a 64-weight step) of the lane's four 8-weight chunks, in MFMA order
  const int koff[4] = {B2<T>::off0(c), B2<T>::off0(c) + 8, B2<T>::off1(c), B2<T>::off1(c) + 8};
  const int s0 = 4 * kw0, last = 4 * kw1 - 1;
  // x of a step (32 tokens x 64 k = 32 rows of 128 bytes) comes in with coalesced loads: load i
  // of lane j takes row 8 i + j / 8, 16-byte chunk (j % 8) ^ swz(row), and the wave writes the four
  // loads to its LDS region in lane order; the A operand (token l % 32, chunk koff / 8) is then read
  // at slot chunk ^ swz(token).  swz(t) = (t >> 1) & 7 puts the 16 rows a quarter-wave reads in 16
  // distinct 16-byte bank groups.
  const int lane = threadIdx.x & 63;
  const uint16_t* xsrc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = 8 * i + (lane >> 3);
    xsrc[i] = x + (int64_t)min(t, M - 1) * ldx + 8 * ((lane & 7) ^ ((t >> 1) & 7));
  }
  const int rs = (r >> 1) & 7;
  struct Step { B2<T> w[NRB]; v4u xg[4]; };
  Step p0, p1;
  auto load = [&](Step& p, int s) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) p.xg[i] = *(const v4u*)(xsrc[i] + (int64_t)s * 64);
    const uint8_t* rc = tbase + (int64_t)(s >> 2) * (64 * REC);
#pragma unroll
    for (int b = 0; b < NRB; ++b) p.w[b].load(rc, r0 + 32 * b + r, s & 3, c);
  };
  auto compute = [&](const Step& p, int s) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) ((v4u*)xl)[64 * i + lane] = p.xg[i];
    v8bf a[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) a[q] = *(const v8bf*)(xl + (r * 8 + ((koff[q] >> 3) ^ rs)) * 8);
#pragma unroll
    for (int b = 0; b < NRB; ++b) {
      const GS st = p.w[b].prep(s & 3, c);
      uint32_t o[16];
#pragma unroll
      for (int i = 0; i < 4; ++i) p.w[b].out(st, s & 3, c, o, tb, i);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            a[q], __builtin_bit_cast(v8bf, v4u{o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]}), acc[b], 0, 0, 0);
    }
  };
  // loads are unconditional (clamped to the wave's last step, re-read from L2 at the tail)
  load(p0, s0);
  load(p1, min(s0 + 1, last));
  for (int s = s0;; s += 2) {
    compute(p0, s);
    load(p0, min(s + 2, last));
    if (s + 1 > last) break;
    compute(p1, s + 1);
    load(p1, min(s + 3, last));
    if (s + 2 > last) break;
  }
}

#define MID_RED_BYTES (3 * 2 * 16 * 64 * 4 + 16)   // the waves' sums combined in LDS (nw <= 4), a flag

// Three waves per SIMD for the two instances that would otherwise take just over 168 VGPRs (Q3_K
// 170, the mixed-type build 176): Q3_K gate_up at M = 20 / 32 2.0-2.9 us faster; mixed layers
// (gate_up, qkv + o_proj) 0.5-2.4 us faster even with the mixed build's 20 bytes of scratch.
template <int ONLY>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(ONLY == GQK_Q3_K || ONLY == 0 ? 3 : 1))) void gemv_mid_kernel(const uint8_t* __restrict__ packed, const int32_t* __restrict__ desc,
                                                       const uint16_t* __restrict__ x, int64_t ldx, int M,
                                                       uint16_t* __restrict__ y, int64_t ldy,
                                                       const uint16_t* __restrict__ bias, float* __restrict__ part,
                                                       int* __restrict__ ctr) {
  constexpr int MP = 32;   // tokens of the plan (partial slots [slot][64 rows][MP])
  __shared__ __attribute__((aligned(16))) uint8_t lds[MID_RED_BYTES + GB_TAB_BYTES];
  __shared__ __attribute__((aligned(16))) uint16_t xlds[4 * 2048];   // a 4 KiB x step per wave
  const int32_t* dsc = desc + (int64_t)blockIdx.x * GQK_DESC_WORDS;
  const int type = dsc[D_TYPE];
  // the wave index is uniform: as an SGPR its k-range, addresses and branches stay scalar (Q6_K,
  // Q2_K 4-9% faster at M = 32)
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nw = blockDim.x >> 6;
  const int c = lane >> 5, r = lane & 31;
  GTabs tb;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    tb.kv[i] = (uint32_t)(c_kvalues[4 * i] + 128) | ((uint32_t)(c_kvalues[4 * i + 1] + 128) << 8) |
               ((uint32_t)(c_kvalues[4 * i + 2] + 128) << 16) | ((uint32_t)(c_kvalues[4 * i + 3] + 128) << 24);
  tb.grid = (uint32_t*)(lds + MID_RED_BYTES);
  tb.sign = (uint4*)(lds + MID_RED_BYTES + 512 * 4);
  if ((ONLY == 0 || ONLY == GQK_IQ3_S) && type == GQK_IQ3_S) {   // uniform over the workgroup
    uint32_t* grid = (uint32_t*)(lds + MID_RED_BYTES);
    uint4* sign = (uint4*)(lds + MID_RED_BYTES + 512 * 4);
    for (int t = threadIdx.x; t < 512; t += blockDim.x) grid[t] = c_iq3s_grid[t];
    for (int t = threadIdx.x; t < 256; t += blockDim.x) {
      uint32_t m[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) m[q] = (((t >> (2 * q)) & 1) << 15) | (((t >> (2 * q + 1)) & 1) << 31);
      sign[t] = make_uint4(m[0], m[1], m[2], m[3]);
    }
    __syncthreads();
  }
  const int64_t off = (int64_t)(uint32_t)dsc[D_OFF_LO] | ((int64_t)dsc[D_OFF_HI] << 32);
  const int64_t tile = dsc[D_TILE0];
  const int nb = dsc[D_NB], kb0 = dsc[D_KB0], nk = dsc[D_KB1] - kb0;
  const int kw0 = kb0 + (wave * nk) / nw, kw1 = kb0 + ((wave + 1) * nk) / nw;
  uint16_t* xl = xlds + wave * 2048;
  v16f acc[2];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[b][v] = 0.f;
#define RUN(T)                                                                                                 \
  if ((ONLY == 0 || ONLY == T) && type == T)                                                                   \
    mid_wave<T>(packed + off + tile * nb * (int64_t)(64 * gqk_layout<T>::REC), x, ldx, M, xl, kw0, kw1, c, r, tb, acc);
  RUN(GQK_Q4_0) RUN(GQK_Q5_0) RUN(GQK_Q8_0) RUN(GQK_Q2_K) RUN(GQK_Q3_K) RUN(GQK_Q4_K) RUN(GQK_Q5_K) RUN(GQK_Q6_K)
  RUN(GQK_IQ4_NL) RUN(GQK_IQ3_S) RUN(GQK_IQ4_XS)
#undef RUN

  // combine the waves (fixed order) in wave 0
  float* red = (float*)lds;   // [wave - 1][b][v][lane]
  int* flag = (int*)(lds + 3 * 2 * 16 * 64 * 4);
  if (wave > 0)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) red[(((wave - 1) * 2 + b) * 16 + v) * 64 + lane] = acc[b][v];
  __syncthreads();
  if (wave == 0)
    for (int w = 1; w < nw; ++w)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[b][v] += red[(((w - 1) * 2 + b) * 16 + v) * 64 + lane];

  // C block b: lane -> weight row 32 b + r, tokens 8 (v / 4) + 4 c + v % 4
  const int nvalid = dsc[D_NVALID];
  const int64_t col0 = dsc[D_COL0];
  const int nc = dsc[D_NC];   // workgroups sharing this tile
  // quarter qd of the outputs: block qd / 2, values 8 (qd % 2) .. + 7 of each lane
  auto store_q = [&](int qd, const float (&a)[8]) {
    const int b = qd >> 1, v0 = 8 * (qd & 1), row = 32 * b + r;
    if (row >= nvalid) return;
    // the layer bias (bf16 per output column) joins before the one rounding to bf16
    const float bv = bias != nullptr ? __builtin_bit_cast(float, (uint32_t)bias[col0 + row] << 16) : 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int v = v0 + e, t = 8 * (v >> 2) + 4 * c + (v & 3);
      if (t < M) y[(int64_t)t * ldy + col0 + row] = __builtin_bit_cast(uint16_t, (__bf16)(a[e] + bv));
    }
  };
  if (nc == 1) {
    if (wave > 0) return;
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      float a[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) a[e] = acc[qd >> 1][8 * (qd & 1) + e];
      store_q(qd, a);
    }
    return;
  }
  // Split-K exchange, as in the GEMV: the nc partials of a tile in slots D_SLOT0 .. + nc - 1 as
  // [slot][64 rows][32 tokens], moved by device-coherent (sc1) 16-byte buffer accesses only.  Wave
  // 0's sums go through LDS so that every wave stores quarters wave, wave + nw, .. of the partial;
  // all stores complete before the arrival count (one barrier), and in the last workgroup to
  // arrive every wave sums its quarters of the slots in split order and writes y; the counter is
  // reset for the next launch.
  __syncthreads();   // wave 0 has read the other waves' sums
  if (wave == 0)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) red[(b * 16 + v) * 64 + lane] = acc[b][v];
  __syncthreads();
  const int sp = dsc[D_SPLIT], ctr_i = dsc[D_CTR];
  float* tp = part + (int64_t)dsc[D_SLOT0] * 64 * MP;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(tp, 0, nc * 64 * MP * 4, GQK_GB_WORD3);
  auto soff = [&](int q, int b, int g) { return ((q * 64 + 32 * b + r) * MP + 8 * g + 4 * c) * 4; };
  for (int qd = wave; qd < 4; qd += nw) {
    const int b = qd >> 1, g0 = 2 * (qd & 1);
    float a[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) a[e] = red[(b * 16 + 8 * (qd & 1) + e) * 64 + lane];
    __builtin_amdgcn_raw_buffer_store_b128(v4f{a[0], a[1], a[2], a[3]}, rs, soff(sp, b, g0), 0, GQK_GB_SC1);
    __builtin_amdgcn_raw_buffer_store_b128(v4f{a[4], a[5], a[6], a[7]}, rs, soff(sp, b, g0 + 1), 0, GQK_GB_SC1);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wave's partial stores are complete
  __syncthreads();
  if (threadIdx.x == 0) *flag = __hip_atomic_fetch_add(&ctr[ctr_i], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (*flag != nc - 1) return;
  asm volatile("" ::: "memory");
  // split slots per round trip (loads clamped to the last slot): two measured 0.4-1.2 us faster
  // than four on `down` at M = 20 / 32 and eight 0.5-1.1 us slower; one is even with two
  constexpr int QB = 2;
  for (int qd = wave; qd < 4; qd += nw) {
    const int b = qd >> 1, g0 = 2 * (qd & 1);
    float a[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) a[e] = 0.f;
    for (int q0 = 0; q0 < nc; q0 += QB) {
      v4f t[QB][2];
#pragma unroll
      for (int j = 0; j < QB; ++j)
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2)
          t[j][h2] = __builtin_amdgcn_raw_buffer_load_b128(rs, soff(min(q0 + j, nc - 1), b, g0 + h2), 0, GQK_GB_SC1);
#pragma unroll
      for (int j = 0; j < QB; ++j)
        if (q0 + j < nc)
#pragma unroll
          for (int e = 0; e < 8; ++e) a[e] += t[j][e >> 2][e & 3];
    }
    store_q(qd, a);
  }
  if (threadIdx.x == 0) __hip_atomic_store(&ctr[ctr_i], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // next launch
}

// The mid form's slab variant (9..32 rows, x padded to 32 tokens; shards of at most one 32-row
// slab per CU): one
// workgroup per 32-row half (D_SPLIT) of a 64-row tile over the whole k-range, its waves splitting
// the k-range as in the mid form (two super-blocks each at K = 5120) with one 32 x 32 block of
// rows each; no split-K partials (whose 8 KiB per workgroup at 32 tokens made the exchange ~30% of
// the mid form's qkv / o_proj launches).  Each wave's sums go to its own 4 KiB x region once its
// products are done, and after one barrier every thread sums one output over the waves in order.
template <int ONLY>
__global__ __launch_bounds__(64 * GQK_SLAB_MAX_WAVES) void gemv_mid_slab_kernel(
    const uint8_t* __restrict__ packed, const int32_t* __restrict__ desc, const uint16_t* __restrict__ x,
    int64_t ldx, int M, uint16_t* __restrict__ y, int64_t ldy, const uint16_t* __restrict__ bias) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[GB_TAB_BYTES];
  __shared__ __attribute__((aligned(16))) uint16_t xlds[GQK_SLAB_MAX_WAVES * 2048];   // a 4 KiB x step per wave
  const int32_t* dsc = desc + (int64_t)blockIdx.x * GQK_DESC_WORDS;
  const int type = dsc[D_TYPE];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nw = blockDim.x >> 6;
  const int c = lane >> 5, r = lane & 31;
  GTabs tb;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    tb.kv[i] = (uint32_t)(c_kvalues[4 * i] + 128) | ((uint32_t)(c_kvalues[4 * i + 1] + 128) << 8) |
               ((uint32_t)(c_kvalues[4 * i + 2] + 128) << 16) | ((uint32_t)(c_kvalues[4 * i + 3] + 128) << 24);
  tb.grid = (uint32_t*)lds;
  tb.sign = (uint4*)(lds + 512 * 4);
  if ((ONLY == 0 || ONLY == GQK_IQ3_S) && type == GQK_IQ3_S) {   // uniform over the workgroup
    uint32_t* grid = (uint32_t*)lds;
    uint4* sign = (uint4*)(lds + 512 * 4);
    for (int t = threadIdx.x; t < 512; t += blockDim.x) grid[t] = c_iq3s_grid[t];
    for (int t = threadIdx.x; t < 256; t += blockDim.x) {
      uint32_t m[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) m[q] = (((t >> (2 * q)) & 1) << 15) | (((t >> (2 * q + 1)) & 1) << 31);
      sign[t] = make_uint4(m[0], m[1], m[2], m[3]);
    }
    __syncthreads();
  }
  const int64_t off = (int64_t)(uint32_t)dsc[D_OFF_LO] | ((int64_t)dsc[D_OFF_HI] << 32);
  const int64_t tile = dsc[D_TILE0];
  const int h = dsc[D_SPLIT];                        // the slab: rows 32 h .. 32 h + 31 of the tile
  const int nb = dsc[D_NB], kb0 = dsc[D_KB0], nk = dsc[D_KB1] - kb0;
  const int kw0 = kb0 + (wave * nk) / nw, kw1 = kb0 + ((wave + 1) * nk) / nw;
  uint16_t* xl = xlds + wave * 2048;
  v16f acc[1];
#pragma unroll
  for (int v = 0; v < 16; ++v) acc[0][v] = 0.f;
#define RUN(T)                                                                                                 \
  if ((ONLY == 0 || ONLY == T) && type == T)                                                                   \
    mid_wave<T, 1>(packed + off + tile * nb * (int64_t)(64 * gqk_layout<T>::REC), x, ldx, M, xl, kw0, kw1, c, r, tb, \
                   acc, 32 * h);
  RUN(GQK_Q4_0) RUN(GQK_Q5_0) RUN(GQK_Q8_0) RUN(GQK_Q2_K) RUN(GQK_Q3_K) RUN(GQK_Q4_K) RUN(GQK_Q5_K) RUN(GQK_Q6_K)
  RUN(GQK_IQ4_NL) RUN(GQK_IQ3_S) RUN(GQK_IQ4_XS)
#undef RUN

  // combine: C block lane -> row 32 h + r, tokens 8 (v / 4) + 4 c + v % 4; [v][lane] per wave
  float* red = (float*)xl;
#pragma unroll
  for (int v = 0; v < 16; ++v) red[v * 64 + lane] = acc[0][v];
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  const int nvalid = dsc[D_NVALID];
  const int64_t col0 = dsc[D_COL0];
  for (int o = threadIdx.x; o < 32 * 32; o += blockDim.x) {
    const int t = o >> 5, rho = o & 31;
    const int v = 4 * (t >> 3) + (t & 3), l = 32 * ((t >> 2) & 1) + rho;
    float sum = 0.f;
    for (int w = 0; w < nw; ++w) sum += ((const float*)(xlds + w * 2048))[v * 64 + l];
    const int row = 32 * h + rho;
    if (t < M && row < nvalid) {
      const float bv = bias != nullptr ? __builtin_bit_cast(float, (uint32_t)bias[col0 + row] << 16) : 0.f;
      y[(int64_t)t * ldy + col0 + row] = __builtin_bit_cast(uint16_t, (__bf16)(sum + bv));
    }
  }
}

int launch_gemv_mid(const uint8_t* packed, const int32_t* desc, int n_desc, int types_mask, const void* x, int64_t ldx,
                    int M, int nw, bool slab, void* y, int64_t ldy, const void* bias, float* part, int* ctr,
                    hipStream_t st) {
  const uint16_t* xx = (const uint16_t*)x;
  uint16_t* yy = (uint16_t*)y;
  const uint16_t* bb = (const uint16_t*)bias;
  if (slab) {
    if (nw < 1 || nw > GQK_SLAB_MAX_WAVES) return GQK_ERR_FORM;
    const dim3 grid(n_desc), block(64 * nw);
    switch (types_mask) {
#define C(T) case T: hipLaunchKernelGGL((gemv_mid_slab_kernel<T>), grid, block, 0, st, packed, desc, xx, ldx, M, yy, ldy, bb); return GQK_OK;
      C(GQK_Q4_0) C(GQK_Q5_0) C(GQK_Q8_0) C(GQK_Q2_K) C(GQK_Q3_K) C(GQK_Q4_K) C(GQK_Q5_K) C(GQK_Q6_K)
      C(GQK_IQ4_NL) C(GQK_IQ3_S) C(GQK_IQ4_XS)
#undef C
      default:
        hipLaunchKernelGGL((gemv_mid_slab_kernel<0>), grid, block, 0, st, packed, desc, xx, ldx, M, yy, ldy, bb);
    }
    return GQK_OK;
  }
  if (nw < 1 || nw > 4) return GQK_ERR_FORM;
  const dim3 grid(n_desc), block(64 * nw);
  switch (types_mask) {
#define C(T) case T: hipLaunchKernelGGL((gemv_mid_kernel<T>), grid, block, 0, st, packed, desc, xx, ldx, M, yy, ldy, bb, part, ctr); return GQK_OK;
    C(GQK_Q4_0) C(GQK_Q5_0) C(GQK_Q8_0) C(GQK_Q2_K) C(GQK_Q3_K) C(GQK_Q4_K) C(GQK_Q5_K) C(GQK_Q6_K)
    C(GQK_IQ4_NL) C(GQK_IQ3_S) C(GQK_IQ4_XS)
#undef C
    default:
      hipLaunchKernelGGL((gemv_mid_kernel<0>), grid, block, 0, st, packed, desc, xx, ldx, M, yy, ldy, bb, part, ctr);
  }
  return GQK_OK;
}

// CUs of the current device, cached per device
static int gb_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 0;
    cache[dev] = n;
  }
  return cache[dev];
}

// persistent workgroups of a form: every one resident (the 256 form takes a whole CU's LDS)
static int gb_workgroups(int bm) { return gb_cus() * (bm == 256 ? 1 : 2); }
static int gb_slot_floats(int bm) {
  return bm == 256 ? GeoBig::SLOT : bm == 128 ? GeoMid::SLOT : GeoSmall::SLOT;
}

// Stream-K workgroups for R remainder tiles of S = 4 nb steps: at most G, at least 16 steps per
// workgroup and at most 6 workgroups per tile.  The last contributor of a tile sums every other
// one's partial slot in dependent device-scope round trips, so contributors cost more than the
// steps they take over: measured on the 5120-row shards at M = 17..200, all G workgroups (13 per
// tile) took 33-110 us, 16 steps / <= 6 per tile 22-70 us; tile-rich shards keep all G.  (Up to
// 12 per tile measured 1-20% slower at M = 48-100.)
static int64_t gb_stream_k_workgroups(int G, int64_t R, int nb, int bm) {
  return std::max<int64_t>(1, std::min<int64_t>({(int64_t)G, R * 4 * nb / 16, 6 * R}));
}

// Workspace: ctr_bytes of counters (the plan's counter region: at least G ints), then the partial tiles.
int64_t gemm_workspace(int bm, int n_desc, int M, int nb, int64_t ctr_bytes) {
  const int G = gb_workgroups(bm);
  if (G <= 0) return -1;
  const int64_t T = (int64_t)n_desc * ((M + bm - 1) / bm);
  const int64_t R = T % G;
  if (R == 0) return 0;
  const int64_t gsk = gb_stream_k_workgroups(G, R, nb, bm);
  return ctr_bytes + (R + gsk - 1) * gb_slot_floats(bm) * 4;
}

// Any M: the remainder tiles R <= G - 1 and the stream-K workgroups gsk <= G, so R + gsk - 1 <=
// 2 G - 2 partial slots of the form's tile.
int64_t gemm_workspace_max() {
  int64_t m = 0;
  for (int bm : {64, 128, 256}) {
    const int G = gb_workgroups(bm);
    if (G <= 0) return -1;
    m = std::max<int64_t>(m, (int64_t)(2 * G - 2) * gb_slot_floats(bm) * 4);
  }
  return GQK_CTR_BYTES + m;
}

template <class GE>
static int launch_sk(int only, int n_desc, int M, int nb, hipStream_t st, const uint8_t* packed, const int32_t* desc,
                     const uint16_t* x, int64_t ldx, uint16_t* y, int64_t ldy, const uint16_t* bias,
                     int64_t ctr_bytes, void* ws, int64_t ws_bytes) {
  const int G = gb_workgroups(GE::BM);
  if (G <= 0) return GQK_ERR_HIP;
  if ((int64_t)G * 4 > ctr_bytes || (ctr_bytes & 255)) return GQK_ERR_FORM;
  const int64_t need = gemm_workspace(GE::BM, n_desc, M, nb, ctr_bytes);
  if (need > 0 && (ws == nullptr || ws_bytes < need || ((uintptr_t)ws & 255))) return GQK_ERR_SHAPE;
  int* ctr = (int*)ws;
  float* part = need > 0 ? (float*)((char*)ws + ctr_bytes) : nullptr;
  // G workgroups when there are at least G tiles; else the stream-K participants only
  const int64_t T = (int64_t)n_desc * ((M + GE::BM - 1) / GE::BM);
  const int gsk = (int)gb_stream_k_workgroups(G, T % G, nb, GE::BM);
  dim3 grid((unsigned)(T >= G ? G : gsk));
  switch (only) {
#define C(T) case T: hipLaunchKernelGGL((gemm_sk_kernel<typename geo_of<GE, T>::type, T>), grid, dim3(GE::NT), 0, st, packed, desc, n_desc, x, ldx, M, y, ldy, bias, part, ctr, G, gsk); return GQK_OK;
    C(GQK_Q4_0) C(GQK_Q5_0) C(GQK_Q8_0) C(GQK_Q2_K) C(GQK_Q3_K) C(GQK_Q4_K) C(GQK_Q5_K) C(GQK_Q6_K)
    C(GQK_IQ4_NL) C(GQK_IQ3_S) C(GQK_IQ4_XS)
#undef C
    default:
      hipLaunchKernelGGL((gemm_sk_kernel<GE, 0>), grid, dim3(GE::NT), 0, st, packed, desc, n_desc, x, ldx, M, y, ldy, bias, part, ctr, G, gsk);
  }
  return GQK_OK;
}

int launch_gemm(const uint8_t* packed, const int32_t* desc, int n_desc, int types_mask, const void* x, int64_t ldx,
                int M, int64_t K, void* y, int64_t ldy, const void* bias, int bm, int64_t ctr_bytes, void* ws,
                int64_t ws_bytes, hipStream_t st) {
  const int nb = (int)(K / 256);
  const uint16_t* xx = (const uint16_t*)x;
  uint16_t* yy = (uint16_t*)y;
  const uint16_t* bb = (const uint16_t*)bias;
  switch (bm) {
    case 256: return launch_sk<GeoBig>(types_mask, n_desc, M, nb, st, packed, desc, xx, ldx, yy, ldy, bb, ctr_bytes, ws, ws_bytes);
    case 128: return launch_sk<GeoMid>(types_mask, n_desc, M, nb, st, packed, desc, xx, ldx, yy, ldy, bb, ctr_bytes, ws, ws_bytes);
    case 64: return launch_sk<GeoSmall>(types_mask, n_desc, M, nb, st, packed, desc, xx, ldx, yy, ldy, bb, ctr_bytes, ws, ws_bytes);
    default: return GQK_ERR_FORM;
  }
}

}  // namespace gqk
