// Hand-written CDNA4 (gfx950) device templates instantiated by every fused
// kernel the HIP backend generates.
//
//  * 128-bit coalesced global loads/stores of fp16/bf16/fp32 packs
//    (load_pack / store_pack), converted to fp32 registers on load and back
//    with round-to-nearest-even on store;
//  * the pointwise driver: one thread per V-element pack over a flat space;
//  * wave64 cross-lane reductions for groups of 2..64 lanes using DPP
//    (quad_perm, row_half_mirror, row_mirror) and gfx950's v_permlane16_swap /
//    v_permlane32_swap (xor 16 and xor 32, VALU exchanges with no LDS round
//    trip), giving every lane of the group the bit-identical result; groups
//    wider than a wave combine per-wave partials through LDS in a fixed order;
//  * scalar math helpers with torch semantics (NaN-propagating max/min,
//    correctly rounded division, integer true division); transcendentals
//    are ROCm's device math library, except erf and a softmax's exp of a
//    non-positive argument, which are evaluated here;
//  * mixed-precision forms of add, sub and mul (an fma against an opaque
//    constant) that read fp16 operands without a separate conversion.
//
// No MFMA: every kernel generated here is HBM-bandwidth bound.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mlc {

typedef _Float16 f16;

// ---------------------------------------------------------------------------
// storage <-> register conversion
// ---------------------------------------------------------------------------
struct bf16 {
  uint16_t bits;
};

// The widened value passes through an empty inline-assembly statement (no
// instruction): ROCm 7.2's instruction selector, with packed fp32 off, folds
// a negation of such a value into the shift when two of them pair into a
// v2f32 operation, and then either aborts ("Cannot select: v2f32 = bitcast")
// or drops the sign of one lane (exp(x) for exp(-x) in a sigmoid). An opaque
// fp32 value is negated like any other.
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  float f = __builtin_bit_cast(float, static_cast<uint32_t>(b) << 16);
  asm("" : "+v"(f));
  return f;
}

// Round-to-nearest-even fp32 -> bf16 (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float ld(const float* p) { return *p; }
__device__ __forceinline__ float ld(const f16* p) { return static_cast<float>(*p); }
__device__ __forceinline__ float ld(const bf16* p) { return bf16_to_f32(p->bits); }
__device__ __forceinline__ double ld(const double* p) { return *p; }
__device__ __forceinline__ int64_t ld(const int64_t* p) { return *p; }
__device__ __forceinline__ int64_t ld(const int32_t* p) { return *p; }
__device__ __forceinline__ int64_t ld(const int16_t* p) { return *p; }
__device__ __forceinline__ int64_t ld(const int8_t* p) { return *p; }
__device__ __forceinline__ int64_t ld(const uint8_t* p) { return *p; }
__device__ __forceinline__ bool ld(const bool* p) { return *reinterpret_cast<const uint8_t*>(p) != 0; }

template <class S, class X> __device__ __forceinline__ S cvt(X x) { return static_cast<S>(x); }
template <> __device__ __forceinline__ f16 cvt<f16, float>(float x) { return static_cast<f16>(x); }
template <> __device__ __forceinline__ f16 cvt<f16, double>(double x) { return static_cast<f16>(static_cast<float>(x)); }
template <> __device__ __forceinline__ bf16 cvt<bf16, float>(float x) { return bf16{f32_to_bf16(x)}; }
template <> __device__ __forceinline__ bf16 cvt<bf16, double>(double x) { return bf16{f32_to_bf16(static_cast<float>(x))}; }
template <> __device__ __forceinline__ bf16 cvt<bf16, int64_t>(int64_t x) { return bf16{f32_to_bf16(static_cast<float>(x))}; }
template <> __device__ __forceinline__ bf16 cvt<bf16, bool>(bool x) { return bf16{f32_to_bf16(x ? 1.0f : 0.0f)}; }
template <> __device__ __forceinline__ bool cvt<bool, float>(float x) { return x != 0.0f; }
template <> __device__ __forceinline__ bool cvt<bool, double>(double x) { return x != 0.0; }
template <> __device__ __forceinline__ bool cvt<bool, int64_t>(int64_t x) { return x != 0; }

template <class S, class X> __device__ __forceinline__ void st(S* p, X x) { *p = cvt<S>(x); }

// value rounded through a narrow float type, as a cast inside a kernel body
// MFMA operand/accumulator fragments and a 16-byte bit copy of 8 halfs
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
struct alignas(16) f16x8 { f16 v[8]; };

// One 16x16x32 MFMA step, D = A B + C with fp32 accumulation, for either
// 16-bit operand type (the attention kernels are written once for both).
__device__ __forceinline__ float4v mfma_16x16x32(half8 a, half8 b, float4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float4v mfma_16x16x32(bf16x8 a, bf16x8 b, float4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// LDS row of key k in a staged K tile of the attention kernels. The score
// MFMA of 16-key tile t reads LDS rows 16t..16t+15, and row 16t + r holds key
// 32(t/2) + 8(r/4) + 4(t%2) + r%4: lane (q, g) then ends with keys
// 32m + 8g .. 32m + 8g + 7 of every 32-key chunk m, so a lane's mask words are
// 16 contiguous bytes and its probabilities are the P.V MFMA's B operand in
// key order (V^T is staged unpermuted).
__device__ __forceinline__ int krow(int k) {
  return (k & ~31) | (((k >> 2) & 1) << 4) | (((k >> 3) & 3) << 2) | (k & 3);
}

__device__ __forceinline__ float round_f16(float x) { return static_cast<float>(static_cast<f16>(x)); }
__device__ __forceinline__ float round_bf16(float x) { return bf16_to_f32(f32_to_bf16(x)); }

// ---------------------------------------------------------------------------
// 128-bit packs
// ---------------------------------------------------------------------------
template <class S, int V> struct alignas(sizeof(S) * V) pack {
  S x[V];
};

// V contiguous elements starting at an address aligned to V*sizeof(S).
template <int V, class S, class R>
__device__ __forceinline__ void load_pack(R (&dst)[V], const S* __restrict__ p) {
  if constexpr (sizeof(S) * V > 16) {
    constexpr int H = 16 / sizeof(S);
    static_assert(V % H == 0, "pack split");
#pragma unroll
    for (int h = 0; h < V / H; ++h) {
      const pack<S, H> w = *reinterpret_cast<const pack<S, H>*>(p + h * H);
#pragma unroll
      for (int i = 0; i < H; ++i) dst[h * H + i] = ld(&w.x[i]);
    }
  } else {
    const pack<S, V> w = *reinterpret_cast<const pack<S, V>*>(p);
#pragma unroll
    for (int i = 0; i < V; ++i) dst[i] = ld(&w.x[i]);
  }
}

template <int V, class S, class R>
__device__ __forceinline__ void store_pack(S* __restrict__ p, const R (&src)[V]) {
  if constexpr (sizeof(S) * V > 16) {
    constexpr int H = 16 / sizeof(S);
#pragma unroll
    for (int h = 0; h < V / H; ++h) {
      pack<S, H> w;
#pragma unroll
      for (int i = 0; i < H; ++i) w.x[i] = cvt<S>(src[h * H + i]);
      *reinterpret_cast<pack<S, H>*>(p + h * H) = w;
    }
  } else {
    pack<S, V> w;
#pragma unroll
    for (int i = 0; i < V; ++i) w.x[i] = cvt<S>(src[i]);
    *reinterpret_cast<pack<S, V>*>(p) = w;
  }
}

// ---------------------------------------------------------------------------
// scalar math with torch semantics
// ---------------------------------------------------------------------------
__device__ __forceinline__ float exp_(float x) { return expf(x); }
// exp(x) = 2^(x log2 e) on the hardware v_exp_f32, for results that are rounded
// to fp16 before use (the fused attention kernel's softmax). The product's
// rounding costs ln2 * |x log2 e| * 2^-24 relative, about 1.2e-6 for |x| <= 20
// (where exp(x) > 2e-9), two hundred times below fp16's half ulp.
__device__ __forceinline__ float exp_fast(float x) {
  return __builtin_amdgcn_exp2f(x * 0x1.715476p+0f);
}
// exp(a - b) for the same use, with b a row's maximum: 2^(a log2 e - RN(b log2 e))
// in one fma. The rounding of b log2 e multiplies every exp of the row by the
// same factor, which cancels when the row is normalised by its sum; what is
// left is the fma's one rounding of the exponent, as in exp_fast. Infinities
// and NaN come out as for exp(a - b) (-inf - -inf is NaN, a - +inf is -inf).
__device__ __forceinline__ float exp_fast_shift(float a, float b) {
  return __builtin_amdgcn_exp2f(__builtin_fmaf(a, 0x1.715476p+0f, -(b * 0x1.715476p+0f)));
}
// exp(x) for x <= 0, -inf or NaN: a softmax's exp(x - rowmax(x)).
// h = RN(x log2 e) goes to v_exp_f32 whole, and the rounding of h is put back
// by one correction: with r = x - h ln2 (formed by two fmas against ln2 split
// into an fp32 head and tail, so r carries no rounding error that matters;
// |r| <= 8e-6 over the clamped range), exp(x) = 2^h e^r = 2^h (1 + r) up to
// r^2/2 < 4e-11 relative. Error: v_exp_f32's (0.8 ulp measured) plus the
// final fma's half ulp. v_exp_f32 flushes results below 2^-126 to zero, so
// exp(x) < 2^-126 (x < -87.34) comes out as 0, an absolute error below
// 1.2e-38. No overflow path: x is at most 0. The clamp at -104 (exp is 0 in
// fp32 below it) keeps r finite for x = -inf; the NaN-propagating maximum
// keeps NaN.
__device__ __forceinline__ float exp_nonpos(float x) {
  x = __builtin_elementwise_maximum(x, -104.0f);
  const float h = x * 0x1.715476p+0f;
  float r = __builtin_fmaf(-h, 0x1.62e430p-1f, x);
  r = __builtin_fmaf(-h, -0x1.05c610p-29f, r);
  const float e = __builtin_amdgcn_exp2f(h);
  return __builtin_fmaf(e, r, e);
}
__device__ __forceinline__ double exp_(double x) { return exp(x); }
// erf in fp32 from two polynomials fitted for this build (weighted least
// squares iterated to minimax, then checked in emulated fp32 arithmetic over
// every other float in [0.5, 2)):
//   |x| <= 1.125: erf(a) = a + a * Q(a^2), Q of degree 6 (Q(0) = 2/sqrt(pi) - 1),
//                 one rounding at the end, so the result never passes through
//                 the coarser binade of erf(a)/a;
//   |x| >  1.125: erf(a) = 1 - 2^(-a^2 log2 e) * S(min(a, 4)), S(a) ~ erfc(a) e^(a^2)
//                 of degree 9, fitted for absolute accuracy in erf; 2^y on the
//                 hardware v_exp_f32 (y -> -inf gives 0 past a = 4, where erf is 1).
// The second form is a branch: a wave evaluates it for an element only when
// one of its lanes needs it (for activations ~N(0, 0.4), one element in five).
// Error 1.48 ulp in emulation with an exact 2^y. NaN stays NaN (it takes the
// first form), +-inf -> +-1, -0 -> -0.
__device__ __forceinline__ float erf_(float x) {
  const float a = __builtin_fabsf(x);
  const float t = a * a;
  float q = 0x1.289392p-14f;
  q = __builtin_fmaf(q, t, -0x1.973b10p-11f);
  q = __builtin_fmaf(q, t, 0x1.522dd8p-8f);
  q = __builtin_fmaf(q, t, -0x1.b7ba86p-6f);
  q = __builtin_fmaf(q, t, 0x1.ce2942p-4f);
  q = __builtin_fmaf(q, t, -0x1.81272ap-2f);
  q = __builtin_fmaf(q, t, 0x1.06eba8p-3f);
  float r = __builtin_fmaf(a, q, a);
  if (a > 1.125f) {
    const float c = __builtin_fminf(a, 4.0f);
    float s = -0x1.5ad6b0p-16f;
    s = __builtin_fmaf(s, c, 0x1.cfa6ccp-12f);
    s = __builtin_fmaf(s, c, -0x1.180806p-8f);
    s = __builtin_fmaf(s, c, 0x1.95d9f8p-6f);
    s = __builtin_fmaf(s, c, -0x1.8b9b96p-4f);
    s = __builtin_fmaf(s, c, 0x1.1405e2p-2f);
    s = __builtin_fmaf(s, c, -0x1.1ee140p-1f);
    s = __builtin_fmaf(s, c, 0x1.c7d78ap-1f);
    s = __builtin_fmaf(s, c, -0x1.171bbep+0f);
    s = __builtin_fmaf(s, c, 0x1.fce7eep-1f);
    const float e = __builtin_amdgcn_exp2f(t * -0x1.715476p+0f);
    r = __builtin_fmaf(-e, s, 1.0f);
  }
  return __builtin_copysignf(r, x);
}
__device__ __forceinline__ float log_(float x) { return logf(x); }
__device__ __forceinline__ double log_(double x) { return log(x); }
__device__ __forceinline__ float sqrt_(float x) { return sqrtf(x); }
__device__ __forceinline__ double sqrt_(double x) { return sqrt(x); }
__device__ __forceinline__ float rsqrt_(float x) { return 1.0f / sqrtf(x); }
__device__ __forceinline__ double rsqrt_(double x) { return 1.0 / sqrt(x); }
__device__ __forceinline__ float sin_(float x) { return sinf(x); }
__device__ __forceinline__ double sin_(double x) { return sin(x); }
__device__ __forceinline__ float cos_(float x) { return cosf(x); }
__device__ __forceinline__ double cos_(double x) { return cos(x); }
__device__ __forceinline__ float tanh_(float x) { return tanhf(x); }
__device__ __forceinline__ double tanh_(double x) { return tanh(x); }
__device__ __forceinline__ double erf_(double x) { return erf(x); }
__device__ __forceinline__ float sigmoid_(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ double sigmoid_(double x) { return 1.0 / (1.0 + exp(-x)); }
__device__ __forceinline__ float floor_(float x) { return floorf(x); }
__device__ __forceinline__ double floor_(double x) { return floor(x); }
__device__ __forceinline__ int64_t floor_(int64_t x) { return x; }
__device__ __forceinline__ float abs_(float x) { return fabsf(x); }
__device__ __forceinline__ double abs_(double x) { return fabs(x); }
__device__ __forceinline__ int64_t abs_(int64_t x) { return x < 0 ? -x : x; }
// fp32 negation: the sign bit flipped by one v_xor_b32. Written as an
// instruction the compiler cannot see through because, with packed fp32 off,
// ROCm 7.2's instruction selector fails on the negation of a value read from
// bf16 storage when it pairs two such negations into a v2f32 operation
// ("Cannot select: v2f32 = bitcast"). NaN's sign flips too, as in torch.
__device__ __forceinline__ float neg_(float x) {
  float r;
  asm("v_xor_b32 %0, 0x80000000, %1" : "=v"(r) : "v"(x));
  return r;
}
__device__ __forceinline__ float pow_(float a, float b) { return powf(a, b); }
__device__ __forceinline__ double pow_(double a, double b) { return pow(a, b); }

// integer operands of a float-only function are promoted to fp32 first
__device__ __forceinline__ float exp_(int64_t x) { return expf(static_cast<float>(x)); }
__device__ __forceinline__ float log_(int64_t x) { return logf(static_cast<float>(x)); }
__device__ __forceinline__ float sqrt_(int64_t x) { return sqrtf(static_cast<float>(x)); }
__device__ __forceinline__ float rsqrt_(int64_t x) { return 1.0f / sqrtf(static_cast<float>(x)); }
__device__ __forceinline__ float tanh_(int64_t x) { return tanhf(static_cast<float>(x)); }
__device__ __forceinline__ float erf_(int64_t x) { return erf_(static_cast<float>(x)); }
__device__ __forceinline__ float sigmoid_(int64_t x) { return sigmoid_(static_cast<float>(x)); }

// NaN-propagating max/min (torch.maximum/amax semantics). fp32 maps to the
// single gfx950 instructions v_maximum3_f32 / v_minimum3_f32.
template <class T> __device__ __forceinline__ T max_(T a, T b) {
  if (a != a) return a;
  if (b != b) return b;
  return a > b ? a : b;
}
template <class T> __device__ __forceinline__ T min_(T a, T b) {
  if (a != a) return a;
  if (b != b) return b;
  return a < b ? a : b;
}
template <> __device__ __forceinline__ float max_<float>(float a, float b) {
  return __builtin_elementwise_maximum(a, b);
}
template <> __device__ __forceinline__ float min_<float>(float a, float b) {
  return __builtin_elementwise_minimum(a, b);
}

// x / d given y = RN(1/d): q = RN(x*y), r = x - q*d (exact through the fma),
// RN(q + r*y) is the correctly rounded quotient (Markstein's theorem, P.
// Markstein, IBM J. Res. Dev. 34(1), 1990) while d, 1/d and x/d stay in the
// normal range. An infinite q (x infinite) makes r NaN; q itself is then the
// quotient. A handful of instructions instead of the IEEE division sequence.
__device__ __forceinline__ float div_rcp(float x, float d, float y) {
  const float q = x * y;
  const float r = __builtin_fmaf(-q, d, x);
  const float q2 = __builtin_fmaf(r, y, q);
  return q2 == q2 ? q2 : q;
}
// div_rcp for an x that is never infinite (a softmax's exp(x - rowmax), at
// most 1): the same quotient without the guard for an infinite x.
__device__ __forceinline__ float div_rcp_finite(float x, float d, float y) {
  const float q = x * y;
  return __builtin_fmaf(__builtin_fmaf(-q, d, x), y, q);
}
// Constants hidden from the optimiser. fma(a, 1, b), fma(b, -1, a) and
// fma(a, b, -0) are bit for bit a + b, a - b and a * b (one rounding of an
// exact value, the same signed zeros), but the compiler folds them back into
// the plain operation when it can see the constant. Kept opaque, the fma of a
// value just converted from fp16 is selected as v_fma_mix_f32, which reads the
// fp16 half directly and saves the v_cvt_f32_f16.
__device__ __forceinline__ float opaque_(float v) {
  asm("" : "+s"(v));
  return v;
}
__device__ __forceinline__ float one_() { return opaque_(1.0f); }
__device__ __forceinline__ float neg_one_() { return opaque_(-1.0f); }
__device__ __forceinline__ float neg_zero_() { return opaque_(-0.0f); }
// whether div_rcp is exact for every x with this divisor
__device__ __forceinline__ bool rcp_ok(float d) {
  const float a = __builtin_fabsf(d);
  return a > 0x1p-120f && a < 0x1p+120f;
}

// ---------------------------------------------------------------------------
// reduction operators
// ---------------------------------------------------------------------------
struct OpSum {
  template <class T> __device__ __forceinline__ static T f(T a, T b) { return a + b; }
};
struct OpProd {
  template <class T> __device__ __forceinline__ static T f(T a, T b) { return a * b; }
};
struct OpMax {
  template <class T> __device__ __forceinline__ static T f(T a, T b) { return max_(a, b); }
};
struct OpMin {
  template <class T> __device__ __forceinline__ static T f(T a, T b) { return min_(a, b); }
};

// ---------------------------------------------------------------------------
// cross-lane movement (32-bit payloads through DPP and the permlane swaps;
// 64-bit payloads through ds_bpermute shuffles)
// ---------------------------------------------------------------------------
template <int CTRL> __device__ __forceinline__ float dpp(float x) {
  const int v = __builtin_bit_cast(int, x);
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(v, v, CTRL, 0xf, 0xf, false));
}
template <int CTRL> __device__ __forceinline__ int dpp(int x) {
  return __builtin_amdgcn_update_dpp(x, x, CTRL, 0xf, 0xf, false);
}

constexpr int kQuadSwap1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kQuadSwap2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kRowHalfMirror = 0x141;
constexpr int kRowMirror = 0x140;

// Reduce over aligned groups of G lanes (G a power of two <= 64); every lane
// of a group ends with the same value.
// x combined by Op with the value of lane (lane ^ 16) (xor16) or (lane ^ 32)
// (xor32) of the wave, on gfx950's v_permlane16_swap / v_permlane32_swap: a
// VALU lane exchange with no LDS round trip. Each lane receives its own value
// and its partner's, in one order or the other, so Op must be commutative
// (sum, product, max and min are, exactly, in IEEE arithmetic). A lane's
// partner must be active whenever the lane is: true when whole aligned groups
// of 32 (xor16) or 64 (xor32) lanes are active or inactive together.
template <class Op> __device__ __forceinline__ float xor16(float x) {
  const unsigned v = __builtin_bit_cast(unsigned, x);
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return Op::f(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
}
template <class Op> __device__ __forceinline__ float xor32(float x) {
  const unsigned v = __builtin_bit_cast(unsigned, x);
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return Op::f(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
}

template <int G, class Op>
__device__ __forceinline__ float group_reduce(float x) {
  if constexpr (G >= 2) x = Op::f(x, dpp<kQuadSwap1>(x));
  if constexpr (G >= 4) x = Op::f(x, dpp<kQuadSwap2>(x));
  if constexpr (G >= 8) x = Op::f(x, dpp<kRowHalfMirror>(x));
  if constexpr (G >= 16) x = Op::f(x, dpp<kRowMirror>(x));
  if constexpr (G >= 32) x = xor16<Op>(x);
  if constexpr (G >= 64) x = xor32<Op>(x);
  return x;
}

template <int G, class Op, class T>
__device__ __forceinline__ T group_reduce(T x) {
#pragma unroll
  for (int m = 1; m < G; m <<= 1) x = Op::f(x, __shfl_xor(x, m, 64));
  return x;
}

// Reduce over a row spread across W = G/64 whole waves of one workgroup.
// ``slot`` is this reduction's private LDS array of W entries.
template <int G, class Op, class T>
__device__ __forceinline__ T block_reduce(T x, T* slot) {
  static_assert(G % 64 == 0, "block_reduce spans whole waves");
  constexpr int W = G / 64;
  x = group_reduce<64, Op>(x);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) slot[wave] = x;
  __syncthreads();
  T r = slot[0];
#pragma unroll
  for (int w = 1; w < W; ++w) r = Op::f(r, slot[w]);
  return r;
}

template <int G, class Op, class T>
__device__ __forceinline__ T row_reduce(T x, T* slot) {
  if constexpr (G <= 64) {
    (void)slot;
    return group_reduce<G, Op>(x);
  } else {
    return block_reduce<G, Op>(x, slot);
  }
}

}  // namespace mlc
