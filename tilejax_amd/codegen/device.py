"""Device-side helpers every generated gfx950 source starts with (written into the source: hiprtc gets no
include paths, and the generated source is standalone, as the reference's generated modules are)."""

PRELUDE = r"""
// ---- tilejax_amd device prelude (gfx950) ----
#ifndef __HIPCC_RTC__
#include <hip/hip_runtime.h>  // hiprtc provides these itself; hipcc (offline inspection) needs them
#endif
typedef __bf16 ak_bf16x8 __attribute__((ext_vector_type(8)));
typedef float ak_f32x16 __attribute__((ext_vector_type(16)));
typedef float ak_f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int ak_u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int ak_u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned short ak_u16;
typedef short ak_i16x4 __attribute__((ext_vector_type(4)));

#define AK_INLINE __device__ __forceinline__

// s_waitcnt with only vmcnt (<= n vector memory ops outstanding) or only lgkmcnt (0) waited for; gfx9's
// encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8.
#define AK_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))
#define AK_WAIT_LGKM0() __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4))
#define AK_LDS(p) ((__attribute__((address_space(3))) void*)(p))
#define AK_LDS4(p) ((__attribute__((address_space(3))) ak_i16x4*)(p))

// Python's floor division and modulo on ints.
AK_INLINE int ak_floordiv(int a, int b) { int q = a / b; return (q * b != a && ((a < 0) != (b < 0))) ? q - 1 : q; }
AK_INLINE int ak_floormod(int a, int b) { int r = a % b; return (r != 0 && ((r < 0) != (b < 0))) ? r + b : r; }
AK_INLINE int ak_imin(int a, int b) { return a < b ? a : b; }
// A read of memory no kernel writes while this one runs (tables, index inputs) through the constant
// address space: where the address is uniform the compiler makes it a scalar load, which leaves the vector
// memory queue (and its in-order wait counts) to the data streams.
template <typename T> AK_INLINE T ak_ldc(const T* p, long long i) { return ((const __attribute__((address_space(4))) T*)p)[i]; }
AK_INLINE int ak_imax(int a, int b) { return a > b ? a : b; }
AK_INLINE int ak_clamp(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }
// An integer index into a dim of n as JAX takes it: a negative one counts from the end (ak_wrap); a read
// then clamps it into the dim (ak_index), where an update out of the dim is dropped.
AK_INLINE int ak_wrap(int v, int n) { return v < 0 ? v + n : v; }
AK_INLINE int ak_index(int v, int n) { return ak_clamp(ak_wrap(v, n), 0, n - 1); }

// bf16 <-> f32. Rounding is to nearest, ties to even (gfx950's v_cvt_pk_bf16_f32); NaN stays NaN.
typedef __bf16 ak_bf16x2 __attribute__((ext_vector_type(2)));
typedef float ak_f32x2 __attribute__((ext_vector_type(2)));
AK_INLINE unsigned ak_pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(unsigned, __builtin_convertvector((ak_f32x2){lo, hi}, ak_bf16x2));
}
AK_INLINE unsigned ak_bf16_bits(float x) { return ak_pack_bf16x2(x, 0.0f) & 0xffffu; }
AK_INLINE float ak_round_bf16(float x) { return __builtin_bit_cast(float, ak_bf16_bits(x) << 16); }
AK_INLINE float ak_bf16_to_f32(unsigned short b) { return __builtin_bit_cast(float, (unsigned)b << 16); }
AK_INLINE float ak_round_f16(float x) { return (float)(_Float16)x; }
// x as three bf16 parts, x = p1 + p2 + p3 to within about 2^-24 |x|: p1 = bf16(x), p2 = bf16(x - p1),
// p3 = bf16(x - p1 - p2) (the differences are exact in f32). Parts after one that isn't finite are 0.
AK_INLINE void ak_split3(float x, float& p1, float& p2, float& p3) {
  p1 = ak_round_bf16(x);
  const float r1 = __builtin_isfinite(p1) ? x - p1 : 0.0f;
  p2 = ak_round_bf16(r1);
  p3 = ak_round_bf16(r1 - p2);
}

// Elementwise functions with the tile code's meaning.
AK_INLINE float ak_exp(float x) { return __expf(x); }
AK_INLINE float ak_exp2(float x) { return exp2f(x); }
AK_INLINE float ak_rsqrt(float x) { return rsqrtf(x); }
AK_INLINE float ak_rcp(float x) { return 1.0f / x; }
AK_INLINE float ak_square(float x) { return x * x; }
AK_INLINE float ak_sign(float x) { return (float)((x > 0.0f) - (x < 0.0f)); }
AK_INLINE float ak_sigmoid(float x) { return 1.0f / (1.0f + __expf(-x)); }
// jnp.maximum/minimum propagate NaN.
AK_INLINE float ak_maximum(float a, float b) { return (a != a || b != b) ? (a + b) : (a > b ? a : b); }
AK_INLINE float ak_minimum(float a, float b) { return (a != a || b != b) ? (a + b) : (a < b ? a : b); }

// The value lane ^ 32 holds, through v_permlane32_swap (no LDS round trip). The swap exchanges the upper
// half of its first operand with the lower half of its second; the lower half's partner is read from the
// second result and the upper half's from the first, which is also right when the compiler gives both
// operands one register (the swap then rotates it by 32 lanes and both results hold the partners).
AK_INLINE float ak_xor32(float x) {
  const unsigned b = __builtin_bit_cast(unsigned, x);
  const auto r = __builtin_amdgcn_permlane32_swap(b, b, false, false);
  return __builtin_bit_cast(float, (__lane_id() < 32) ? r[1] : r[0]);
}
AK_INLINE float ak_xor32_max(float x) { return fmaxf(x, ak_xor32(x)); }
AK_INLINE float ak_xor32_sum(float x) { return x + ak_xor32(x); }
// The sum over the wave's 64 lanes, in every lane.
AK_INLINE float ak_wave_sum(float x) {
  x += ak_xor32(x);
#pragma unroll
  for (int d = 16; d >= 1; d >>= 1) x += __shfl_xor(x, d);
  return x;
}

// 8x8 transpose of 16-bit elements held as 8 rows of 4 dwords: out[c] holds column c (8 elements).
AK_INLINE void ak_transpose8x8_b16(const ak_u32x4 in[8], ak_u32x4 out[8]) {
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const unsigned sel = (c & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      out[c][d] = __builtin_amdgcn_perm(in[2 * d + 1][c >> 1], in[2 * d][c >> 1], sel);
    }
  }
}
// ---- end of prelude ----
"""
