// CDNA4 (gfx950) device templates used by the Enceladus HIP emitter.
//
// Every generated kernel includes this header. It provides:
//   - element conversions with the language's semantics (saturating float->int,
//     round-to-nearest-even bf16, C-style integer division that never traps);
//   - raw 1/2/4/8/16-byte vector moves for coalesced global and LDS access;
//   - wave64 cross-lane primitives (DPP row ops and ds_bpermute shuffles);
//   - MFMA wrappers for the gfx950 fp16/bf16/fp32 matrix instructions.
// The header is compiled by hiprtc; it uses only compiler builtins, no system headers.
#pragma once

typedef __INT8_TYPE__ int8_t;
typedef __UINT8_TYPE__ uint8_t;
typedef __INT16_TYPE__ int16_t;
typedef __UINT16_TYPE__ uint16_t;
typedef __INT32_TYPE__ int32_t;
typedef __UINT32_TYPE__ uint32_t;
typedef __INT64_TYPE__ int64_t;
typedef __UINT64_TYPE__ uint64_t;

#define EK_INLINE __device__ __attribute__((always_inline)) inline

// Device printf (tl.device_print); the HIP runtime services it through its hostcall buffer.
extern "C" __device__ int printf(const char*, ...);

namespace ek {

// ---------------------------------------------------------------------------
// bfloat16 storage type (bit pattern); arithmetic always goes through float.
// ---------------------------------------------------------------------------
struct bf16 {
  uint16_t x;
};

EK_INLINE float bits_f32(uint32_t u) { return __builtin_bit_cast(float, u); }
EK_INLINE uint32_t f32_bits(float f) { return __builtin_bit_cast(uint32_t, f); }

EK_INLINE float bf16_to_f32(bf16 h) { return bits_f32(((uint32_t)h.x) << 16); }
// fp32 -> bf16, round to nearest even (gfx950 converts in hardware: v_cvt_pk_bf16_f32).
EK_INLINE bf16 f32_to_bf16(float f) {
  return bf16{__builtin_bit_cast(uint16_t, (__bf16)f)};
}

// ---------------------------------------------------------------------------
// Conversions. `f32(x)` widens any element to the float compute type; `cvt<T>(x)`
// converts with the language's rules.
// ---------------------------------------------------------------------------
EK_INLINE float f32(float x) { return x; }
EK_INLINE float f32(_Float16 x) { return (float)x; }
EK_INLINE float f32(bf16 x) { return bf16_to_f32(x); }

template <typename T> struct int_limits;
template <> struct int_limits<int8_t> { static constexpr float lo = -128.f, hi = 127.f; };
template <> struct int_limits<uint8_t> { static constexpr float lo = 0.f, hi = 255.f; };
template <> struct int_limits<int16_t> { static constexpr float lo = -32768.f, hi = 32767.f; };
template <> struct int_limits<uint16_t> { static constexpr float lo = 0.f, hi = 65535.f; };

// float -> integer: truncate toward zero; NaN -> 0; out of range saturates (all widths
// except int64, which wraps modulo 2^64 and maps infinities to 0).
// v_cvt_i32_f32 / v_cvt_u32_f32 implement exactly that for 32 bits (the ISA: out-of-range
// values, infinities included, saturate and NaN converts to 0), so they are issued as is:
// one instruction instead of a NaN test and two clamps, which the compiler emits as nested
// branches. C++'s (int)x leaves out-of-range values undefined, hence the inline asm.
template <typename T> EK_INLINE T f2i(float x);
template <> EK_INLINE int32_t f2i<int32_t>(float x) {
  int32_t r;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(x));
  return r;
}
template <> EK_INLINE uint32_t f2i<uint32_t>(float x) {
  uint32_t r;
  asm("v_cvt_u32_f32 %0, %1" : "=v"(r) : "v"(x));
  return r;
}
template <> EK_INLINE uint64_t f2i<uint64_t>(float x) {
  if (x != x || x <= 0.0f) return 0ull;
  if (x >= 18446744073709551616.0f) return ~0ull;
  return (uint64_t)x;
}
template <> EK_INLINE int64_t f2i<int64_t>(float x) {
  if (x != x || x == __builtin_inff() || x == -__builtin_inff()) return 0;
  float t = __builtin_truncf(x);
  float a = t < 0.f ? -t : t;
  if (a < 9223372036854775808.0f) return (int64_t)t;
  // |t| >= 2^63: t is a multiple of 2^40 at least; reduce modulo 2^64 exactly.
  double d = (double)t;
  double r = __builtin_fmod(d, 18446744073709551616.0);
  if (r >= 9223372036854775808.0) r -= 18446744073709551616.0;
  if (r < -9223372036854775808.0) r += 18446744073709551616.0;
  return (int64_t)r;
}
// 8/16-bit: the saturating 32-bit conversion, then a clamp (truncation commutes with it).
#define EK_SMALL_F2I(T)                                                       \
  template <> EK_INLINE T f2i<T>(float x) {                                   \
    const int32_t i = f2i<int32_t>(x);                                        \
    const int32_t lo = (int32_t)int_limits<T>::lo, hi = (int32_t)int_limits<T>::hi; \
    return (T)(i < lo ? lo : (i > hi ? hi : i));                              \
  }
EK_SMALL_F2I(int8_t)
EK_SMALL_F2I(uint8_t)
EK_SMALL_F2I(int16_t)
EK_SMALL_F2I(uint16_t)
#undef EK_SMALL_F2I
template <> EK_INLINE bool f2i<bool>(float x) { return x != 0.0f; }

template <typename To> struct Cvt {
  template <typename From> static EK_INLINE To from(From x) {
    if constexpr (__is_same(From, float) || __is_same(From, _Float16) || __is_same(From, bf16)) {
      return f2i<To>(f32(x));
    } else {
      return (To)x;
    }
  }
};
template <> struct Cvt<bool> {
  template <typename From> static EK_INLINE bool from(From x) {
    if constexpr (__is_same(From, bf16)) return (x.x & 0x7fffu) != 0;
    else return x != (From)0;
  }
};
template <> struct Cvt<float> {
  template <typename From> static EK_INLINE float from(From x) {
    if constexpr (__is_same(From, bf16) || __is_same(From, _Float16)) return f32(x);
    else return (float)x;
  }
};
template <> struct Cvt<_Float16> {
  template <typename From> static EK_INLINE _Float16 from(From x) {
    if constexpr (__is_same(From, bf16)) return (_Float16)f32(x);
    else if constexpr (__is_same(From, int64_t) || __is_same(From, uint64_t)) return (_Float16)(float)x;
    else return (_Float16)x;
  }
};
template <> struct Cvt<bf16> {
  template <typename From> static EK_INLINE bf16 from(From x) {
    if constexpr (__is_same(From, bf16)) return x;
    else if constexpr (__is_same(From, float)) return f32_to_bf16(x);
    else if constexpr (__is_same(From, _Float16)) return f32_to_bf16((float)x);
    else return f32_to_bf16((float)x);
  }
};
template <typename To, typename From> EK_INLINE To cvt(From x) { return Cvt<To>::from(x); }

// Round a float result to the storage type T (identity for non-half types).
template <typename T> EK_INLINE T rnd(float x) { return cvt<T>(x); }

// ---------------------------------------------------------------------------
// Integer arithmetic that never traps: x / 0 gives x, x % 0 gives 0 (matching the
// language's interpreter), and shifts by >= the width give 0 (or the sign fill).
// ---------------------------------------------------------------------------
template <typename T> EK_INLINE T idiv(T a, T b) { return b == (T)0 ? a : (T)(a / b); }
template <typename T> EK_INLINE T imod(T a, T b) { return b == (T)0 ? (T)0 : (T)(a % b); }
template <int N> struct uint_of;
template <> struct uint_of<1> { typedef uint8_t type; };
template <> struct uint_of<2> { typedef uint16_t type; };
template <> struct uint_of<4> { typedef uint32_t type; };
template <> struct uint_of<8> { typedef uint64_t type; };
// The left shift runs on the unsigned type of the same width, so bits shifted into or
// past the sign bit wrap instead of being undefined behaviour; a negative count (huge as
// an unsigned number) or one >= the width gives 0, as NumPy's left_shift does.
template <typename T> EK_INLINE T ishl(T a, T b) {
  typedef typename uint_of<sizeof(T)>::type U;
  return ((uint64_t)b >= sizeof(T) * 8) ? (T)0 : (T)(U)((U)a << b);
}
template <typename T> EK_INLINE T ishr(T a, T b) {
  if ((uint64_t)b >= sizeof(T) * 8) return (T)((T)-1 > (T)0 ? 0 : (a < (T)0 ? (T)-1 : (T)0));
  return (T)(a >> b);
}
EK_INLINE float fmodf_(float a, float b) { return __builtin_fmodf(a, b); }

// erf(x) by Abramowitz & Stegun, Handbook of Mathematical Functions, formula 7.1.26:
// erf(x) = 1 - (a1 t + a2 t^2 + a3 t^3 + a4 t^4 + a5 t^5) exp(-x^2), t = 1 / (1 + p x),
// x >= 0, extended as an odd function; |error| <= 1.5e-7. Branch-free, so it unrolls well
// in register-resident epilogues.
EK_INLINE float erf_as(float x) {
  const float ax = __builtin_fabsf(x);
  // v_rcp_f32 (1 ulp) instead of an IEEE division: t's rounding changes erf by < 1e-7
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.3275911f, ax, 1.0f));
  float poly = __builtin_fmaf(1.061405429f, t, -1.453152027f);
  poly = __builtin_fmaf(poly, t, 1.421413741f);
  poly = __builtin_fmaf(poly, t, -0.284496736f);
  poly = __builtin_fmaf(poly, t, 0.254829592f);
  poly *= t;
  const float y = 1.0f - poly * __builtin_amdgcn_exp2f(-ax * ax * 1.4426950408889634f);
  return __builtin_copysignf(y, x);
}

// 2^x with the hardware v_exp_f32 (1 ulp; results below 2^-126 flush to zero).
EK_INLINE float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------------------
// Raw vector moves. N is the byte count (1, 2, 4, 8 or 16).
// ---------------------------------------------------------------------------
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
template <int N> struct raw_t;
template <> struct raw_t<1> { typedef uint8_t type; };
template <> struct raw_t<2> { typedef uint16_t type; };
template <> struct raw_t<4> { typedef uint32_t type; };
template <> struct raw_t<8> { typedef u32x2 type; };
template <> struct raw_t<16> { typedef u32x4 type; };

template <typename T, int V> EK_INLINE void vload(T* dst, const T* src) {
  typedef typename raw_t<sizeof(T) * V>::type R;
  R v = *reinterpret_cast<const R*>(src);
  __builtin_memcpy(dst, &v, sizeof(R));
}
// Streaming variants: non-temporal hint (data touched once; don't keep it in the caches).
template <typename T, int V> EK_INLINE void vload_nt(T* dst, const T* src) {
  typedef typename raw_t<sizeof(T) * V>::type R;
  R v = __builtin_nontemporal_load(reinterpret_cast<const R*>(src));
  __builtin_memcpy(dst, &v, sizeof(R));
}
template <typename T, int V> EK_INLINE void vstore_nt(T* dst, const T* src) {
  typedef typename raw_t<sizeof(T) * V>::type R;
  R v;
  __builtin_memcpy(&v, src, sizeof(R));
  __builtin_nontemporal_store(v, reinterpret_cast<R*>(dst));
}
template <typename T, int V> EK_INLINE void vstore(T* dst, const T* src) {
  typedef typename raw_t<sizeof(T) * V>::type R;
  R v;
  __builtin_memcpy(&v, src, sizeof(R));
  *reinterpret_cast<R*>(dst) = v;
}

// ---------------------------------------------------------------------------
// Wave64 cross-lane moves.
// ---------------------------------------------------------------------------
EK_INLINE int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

// Reads `v` from lane `src` (any lane of the wave); ds_bpermute.
EK_INLINE uint32_t shfl_u32(uint32_t v, int src) {
  return (uint32_t)__builtin_amdgcn_ds_bpermute(src << 2, (int)v);
}
template <typename T> EK_INLINE T shfl(T v, int src) {
  if constexpr (sizeof(T) == 8) {
    uint64_t u;
    __builtin_memcpy(&u, &v, 8);
    uint32_t lo = shfl_u32((uint32_t)u, src), hi = shfl_u32((uint32_t)(u >> 32), src);
    u = ((uint64_t)hi << 32) | lo;
    T r;
    __builtin_memcpy(&r, &u, 8);
    return r;
  } else {
    uint32_t u = 0;
    __builtin_memcpy(&u, &v, sizeof(T));
    u = shfl_u32(u, src);
    T r;
    __builtin_memcpy(&r, &u, sizeof(T));
    return r;
  }
}

// A 32-bit exchange with lane ^ MASK that stays in the VALU for every power of two
// (ds_bpermute, the general path, is an LDS round trip that the reductions would wait on):
// - 1, 2: one DPP quad permute ([1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E);
// - 4: row_half_mirror (lane ^ 7), then quad_perm [3,2,1,0] = 0x1B (lane ^ 3);
// - 8: row_mirror (lane ^ 15), then row_half_mirror (lane ^ 7);
// - 16: v_permlane16_swap of the value with itself leaves rows (0,0,2,2) in the first
//   result and rows (1,1,3,3) in the second; a lane takes the other row of its pair;
// - 32: v_permlane32_swap likewise leaves halves (lo,lo) and (hi,hi).
template <int MASK> EK_INLINE uint32_t xor_lanes_u32(uint32_t u) {
  const int x = (int)u;
  if constexpr (MASK == 1 || MASK == 2) {
    return (uint32_t)__builtin_amdgcn_mov_dpp(x, MASK == 1 ? 0xB1 : 0x4E, 0xF, 0xF, false);
  } else if constexpr (MASK == 4) {
    const int t = __builtin_amdgcn_mov_dpp(x, 0x141, 0xF, 0xF, false);
    return (uint32_t)__builtin_amdgcn_mov_dpp(t, 0x1B, 0xF, 0xF, false);
  } else if constexpr (MASK == 8) {
    const int t = __builtin_amdgcn_mov_dpp(x, 0x140, 0xF, 0xF, false);
    return (uint32_t)__builtin_amdgcn_mov_dpp(t, 0x141, 0xF, 0xF, false);
  } else if constexpr (MASK == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return (lane_id() & 16) ? (uint32_t)r[0] : (uint32_t)r[1];
  } else if constexpr (MASK == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return (lane_id() & 32) ? (uint32_t)r[0] : (uint32_t)r[1];
  } else {
    return shfl_u32(u, lane_id() ^ MASK);
  }
}

// Exchange with lane ^ MASK, for values of up to 8 bytes (all lanes active).
template <int MASK, typename T> EK_INLINE T shfl_xor(T v) {
  if constexpr (sizeof(T) == 8) {
    uint64_t u;
    __builtin_memcpy(&u, &v, 8);
    const uint32_t lo = xor_lanes_u32<MASK>((uint32_t)u), hi = xor_lanes_u32<MASK>((uint32_t)(u >> 32));
    u = ((uint64_t)hi << 32) | lo;
    T r;
    __builtin_memcpy(&r, &u, 8);
    return r;
  } else {
    uint32_t u = 0;
    __builtin_memcpy(&u, &v, sizeof(T));
    u = xor_lanes_u32<MASK>(u);
    T r;
    __builtin_memcpy(&r, &u, sizeof(T));
    return r;
  }
}

// Inclusive prefix sum over lanes 0..63 of a 32-bit value with DPP moves: Kogge-Stone
// inside each 16-lane row (row_shr 1, 2, 4, 8), then row_bcast:15 carries row 0 into
// row 1 and row 2 into row 3, and row_bcast:31 carries lane 31 into rows 2 and 3. Lanes
// whose DPP source is out of range (or outside the row mask) add 0.
template <typename T> EK_INLINE T wave_prefix_sum(T v) {
  static_assert(sizeof(T) == 4, "32-bit values");
  int x = __builtin_bit_cast(int, v);
#define EK_SCAN_STEP(ctrl, rmask)                                                        \
  {                                                                                     \
    const int y = __builtin_amdgcn_update_dpp(0, x, ctrl, rmask, 0xF, false);           \
    x = __builtin_bit_cast(int, __builtin_bit_cast(T, x) + __builtin_bit_cast(T, y));  \
  }
  EK_SCAN_STEP(0x111, 0xF)   // row_shr:1
  EK_SCAN_STEP(0x112, 0xF)   // row_shr:2
  EK_SCAN_STEP(0x114, 0xF)   // row_shr:4
  EK_SCAN_STEP(0x118, 0xF)   // row_shr:8
  EK_SCAN_STEP(0x142, 0xA)   // row_bcast:15 into rows 1 and 3
  EK_SCAN_STEP(0x143, 0xC)   // row_bcast:31 into rows 2 and 3
#undef EK_SCAN_STEP
  return __builtin_bit_cast(T, x);
}

// ---------------------------------------------------------------------------
// Combine functions for reductions and scans.
// ---------------------------------------------------------------------------
struct Sum {
  template <typename T> static EK_INLINE T op(T a, T b) { return a + b; }
};
// Keeps the first operand: the element of a size-1 axis (split of a (2,) tile).
struct First {
  template <typename T> static EK_INLINE T op(T a, T) { return a; }
};
struct Max {
  template <typename T> static EK_INLINE T op(T a, T b) {
    if constexpr (__is_same(T, float)) return __builtin_fmaxf(a, b);
    else return a > b ? a : b;
  }
};
struct Min {
  template <typename T> static EK_INLINE T op(T a, T b) {
    if constexpr (__is_same(T, float)) return __builtin_fminf(a, b);
    else return a < b ? a : b;
  }
};

// ---------------------------------------------------------------------------
// MFMA wrappers (gfx950). Operand registers are passed as arrays of 2-byte elements;
// the accumulator as an array of floats. The array element order is the order of the
// instruction's per-lane operand registers.
// ---------------------------------------------------------------------------
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename V, typename T> EK_INLINE V pack(const T* p) {
  V v;
  __builtin_memcpy(&v, p, sizeof(V));
  return v;
}
template <typename V, typename T> EK_INLINE void unpack(T* p, V v) {
  __builtin_memcpy(p, &v, sizeof(V));
}
typedef int i32x16m __attribute__((ext_vector_type(16)));
typedef int i32x4m __attribute__((ext_vector_type(4)));

// D[32x32] += A[32x16] * B[16x32], fp16/bf16 inputs, 8 elements per lane.
EK_INLINE void mfma_32x32x16(float* acc, const _Float16* a, const _Float16* b) {
  f32x16 c = pack<f32x16>(acc);
  c = __builtin_amdgcn_mfma_f32_32x32x16_f16(pack<f16x8>(a), pack<f16x8>(b), c, 0, 0, 0);
  unpack(acc, c);
}
EK_INLINE void mfma_32x32x16(float* acc, const bf16* a, const bf16* b) {
  f32x16 c = pack<f32x16>(acc);
  c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pack<bf16x8>(a), pack<bf16x8>(b), c, 0, 0, 0);
  unpack(acc, c);
}
// D[16x16] += A[16x32] * B[32x16], 8 elements per lane.
EK_INLINE void mfma_16x16x32(float* acc, const _Float16* a, const _Float16* b) {
  f32x4 c = pack<f32x4>(acc);
  c = __builtin_amdgcn_mfma_f32_16x16x32_f16(pack<f16x8>(a), pack<f16x8>(b), c, 0, 0, 0);
  unpack(acc, c);
}
EK_INLINE void mfma_16x16x32(float* acc, const bf16* a, const bf16* b) {
  f32x4 c = pack<f32x4>(acc);
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pack<bf16x8>(a), pack<bf16x8>(b), c, 0, 0, 0);
  unpack(acc, c);
}
// D[32x32] += A[32x8] * B[8x32], 4 elements per lane.
EK_INLINE void mfma_32x32x8(float* acc, const _Float16* a, const _Float16* b) {
  f32x16 c = pack<f32x16>(acc);
  c = __builtin_amdgcn_mfma_f32_32x32x8f16(pack<f16x4>(a), pack<f16x4>(b), c, 0, 0, 0);
  unpack(acc, c);
}
EK_INLINE void mfma_32x32x8(float* acc, const bf16* a, const bf16* b) {
  f32x16 c = pack<f32x16>(acc);
  c = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(pack<s16x4>(a), pack<s16x4>(b), c, 0, 0, 0);
  unpack(acc, c);
}
// D[16x16] += A[16x16] * B[16x16], 4 elements per lane.
EK_INLINE void mfma_16x16x16(float* acc, const _Float16* a, const _Float16* b) {
  f32x4 c = pack<f32x4>(acc);
  c = __builtin_amdgcn_mfma_f32_16x16x16f16(pack<f16x4>(a), pack<f16x4>(b), c, 0, 0, 0);
  unpack(acc, c);
}
EK_INLINE void mfma_16x16x16(float* acc, const bf16* a, const bf16* b) {
  f32x4 c = pack<f32x4>(acc);
  c = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pack<s16x4>(a), pack<s16x4>(b), c, 0, 0, 0);
  unpack(acc, c);
}
// fp32 inputs: D[16x16] += A[16x4] * B[4x16], one element per lane.
EK_INLINE void mfma_16x16x4(float* acc, const float* a, const float* b) {
  f32x4 c = pack<f32x4>(acc);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[0], b[0], c, 0, 0, 0);
  unpack(acc, c);
}
// fp32 inputs: D[32x32] += A[32x2] * B[2x32], one element per lane.
EK_INLINE void mfma_32x32x2(float* acc, const float* a, const float* b) {
  f32x16 c = pack<f32x16>(acc);
  c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[0], b[0], c, 0, 0, 0);
  unpack(acc, c);
}
// int8 inputs, int32 accumulator; integer sums wrap modulo 2^32.
// D[32x32] += A[32x32] * B[32x32], 16 elements per lane (gfx950).
EK_INLINE void mfma_32x32x32(int32_t* acc, const int8_t* a, const int8_t* b) {
  i32x16m c = pack<i32x16m>(acc);
  c = __builtin_amdgcn_mfma_i32_32x32x32_i8(pack<i32x4m>(a), pack<i32x4m>(b), c, 0, 0, 0);
  unpack(acc, c);
}
// D[16x16] += A[16x64] * B[64x16], 16 elements per lane (gfx950).
EK_INLINE void mfma_16x16x64(int32_t* acc, const int8_t* a, const int8_t* b) {
  i32x4m c = pack<i32x4m>(acc);
  c = __builtin_amdgcn_mfma_i32_16x16x64_i8(pack<i32x4m>(a), pack<i32x4m>(b), c, 0, 0, 0);
  unpack(acc, c);
}
// D[32x32] += A[32x16] * B[16x32], 8 elements per lane.
EK_INLINE void mfma_32x32x16(int32_t* acc, const int8_t* a, const int8_t* b) {
  i32x16m c = pack<i32x16m>(acc);
  c = __builtin_amdgcn_mfma_i32_32x32x16_i8(pack<long>(a), pack<long>(b), c, 0, 0, 0);
  unpack(acc, c);
}
// D[16x16] += A[16x32] * B[32x16], 8 elements per lane.
EK_INLINE void mfma_16x16x32(int32_t* acc, const int8_t* a, const int8_t* b) {
  i32x4m c = pack<i32x4m>(acc);
  c = __builtin_amdgcn_mfma_i32_16x16x32_i8(pack<long>(a), pack<long>(b), c, 0, 0, 0);
  unpack(acc, c);
}


// ---------------------------------------------------------------------------
// Block GEMM main loop for `for k in range(lo, hi, BK): acc = dot(A.load([m0, k]),
// B.load([k, n0]), acc)` with row-major 16-bit A [M, K] (lda) and B [K, N] (ldb).
//
// NT threads = WM x WN waves; each wave owns a (BM/WM) x (BN/WN) block of 32x32 MFMA tiles
// (v_mfma_f32_32x32x16_{f16,bf16}). The accumulator is held in the emitter's MFMA layout:
// acc[(tm * TN + tn) * 16 + j]. With TR the instruction computes each tile's transpose
// (B^T A^T, the same fragments in swapped slots), so a lane holds one row of C and 4
// consecutive columns per 4 registers instead of one column and 4 rows.
//
// Per iteration each thread prefetches its share of the next A and B tiles from global
// memory into registers (16-byte loads), computes the current tile from LDS, then writes
// the prefetched registers into the other LDS stage: one barrier per iteration.
// LDS holds A as [BM][BK] and B transposed as [BN][BK], both with k contiguous and the
// 16-byte chunk index XOR-swizzled by the row, so every MFMA operand is one 128-bit LDS
// read. B is transposed in registers: each thread loads an 8x8 block (8 k rows x 8 n
// columns) and permutes it with v_perm_b32 before writing 8 rows of B^T.
// ---------------------------------------------------------------------------
EK_INLINE uint32_t perm_lo(uint32_t lo_src, uint32_t hi_src) {
  return __builtin_amdgcn_perm(hi_src, lo_src, 0x05040100u);  // (lo16(lo_src), lo16(hi_src))
}
EK_INLINE uint32_t perm_hi(uint32_t lo_src, uint32_t hi_src) {
  return __builtin_amdgcn_perm(hi_src, lo_src, 0x07060302u);  // (hi16(lo_src), hi16(hi_src))
}

// r[j] holds 8 halves of row j (columns 0..7); o[i] receives column i (rows 0..7).
EK_INLINE void transpose8x8(const u32x4* r, u32x4* o) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int w = i >> 1;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t a = r[2 * q][w], b = r[2 * q + 1][w];
      o[i][q] = (i & 1) ? perm_hi(a, b) : perm_lo(a, b);
    }
  }
}

EK_INLINE void transpose8x8(const u32x4* r, u32x4* o, int) { transpose8x8(r, o); }

// r[j] holds 4 halves of row j (columns 0..3); o[i] receives column i (rows 0..7).
EK_INLINE void transpose8x4(const u32x2* r, u32x4* o) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int w = i >> 1;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t a = r[2 * q][w], b = r[2 * q + 1][w];
      o[i][q] = (i & 1) ? perm_hi(a, b) : perm_lo(a, b);
    }
  }
}

// Element offset in a staged LDS tile. Lines of 2^LENSH elements are packed 2^LSH to a row of
// PITCH elements; inside its row, a position's group of 2^CSH 8-element chunks is XOR-swizzled
// by ((row >> SA) ^ (row >> SB)) & MASK.
template <int PITCH, int MASK, int SA, int SB, int LSH, int LENSH, int CSH = 0>
EK_INLINE int swz(int line, int sp) {
  const int row = line >> LSH;
  const int vp = ((line & ((1 << LSH) - 1)) << LENSH) | sp;
  if constexpr (MASK == 0) {
    return row * PITCH + vp;
  } else {
    return row * PITCH + (vp ^ ((((row >> SA) ^ (row >> SB)) & MASK) << (3 + CSH)));
  }
}

// Raw buffer loads: the hardware range-checks each access against the resource size and
// returns zeros out of range, so edge tiles need no per-element predicates. Offsets are in
// bytes (< 2^31); a negative or too-large offset reads zeros.
EK_INLINE __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t nbytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)nbytes,
                                           0x00020000);
}
EK_INLINE u32x4 buffer_load16(__amdgpu_buffer_rsrc_t r, int byte_off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}
EK_INLINE u32x2 buffer_load8(__amdgpu_buffer_rsrc_t r, int byte_off) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, 0));
}
constexpr int kOOB = 0x7ffffff0;  // an offset past any resource: loads read zeros

// ds_read_b64_tr_b16: in each group of 16 lanes, output lane L receives element L % 4 of the
// 8-byte LDS reads made by lanes 4t + L / 4, t = 0..3 (a 4x4 transpose of 16-bit elements).
template <typename T>
EK_INLINE void tr_read4(T* dst, const T* src) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  const v4s v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4s*)(src));
  __builtin_memcpy(dst, &v, 8);
}

// tl.device_assert: the first failure claims word 0 and records the assert index and the
// program id (words 1..4); later failures leave the record alone.
EK_INLINE void assert_fail(uint32_t* buf, int index, int px, int py, int pz) {
  uint32_t expected = 0;
  if (__hip_atomic_compare_exchange_strong(buf, &expected, 1u, __ATOMIC_RELAXED,
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
    __hip_atomic_store(buf + 1, (uint32_t)index, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(buf + 2, (uint32_t)px, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(buf + 3, (uint32_t)py, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(buf + 4, (uint32_t)pz, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}
// Two's-complement wrapping add/sub/mul/neg for the language's signed 32/64-bit integers
// (signed overflow is undefined in C++).
EK_INLINE int32_t wadd(int32_t a, int32_t b) { return (int32_t)((uint32_t)a + (uint32_t)b); }
EK_INLINE int32_t wsub(int32_t a, int32_t b) { return (int32_t)((uint32_t)a - (uint32_t)b); }
EK_INLINE int32_t wmul(int32_t a, int32_t b) { return (int32_t)((uint32_t)a * (uint32_t)b); }
EK_INLINE int32_t wneg(int32_t a) { return (int32_t)(0u - (uint32_t)a); }
EK_INLINE int64_t wadd(int64_t a, int64_t b) { return (int64_t)((uint64_t)a + (uint64_t)b); }
EK_INLINE int64_t wsub(int64_t a, int64_t b) { return (int64_t)((uint64_t)a - (uint64_t)b); }
EK_INLINE int64_t wmul(int64_t a, int64_t b) { return (int64_t)((uint64_t)a * (uint64_t)b); }
EK_INLINE int64_t wneg(int64_t a) { return (int64_t)(0ull - (uint64_t)a); }

// Atomic read-modify-write as a compare-and-swap loop: `f(old)` gives the new value. Used for
// the updates without a native instruction: float max/min, value-compare CAS on floats, and
// every 8- and 16-bit element, which is updated inside its aligned 32-bit word (the CAS
// retries when a neighbour in the same word changed). Returns the old value.
template <int N> struct UBits;
template <> struct UBits<1> { typedef uint8_t type; };
template <> struct UBits<2> { typedef uint16_t type; };
template <> struct UBits<4> { typedef uint32_t type; };
template <typename T, typename F> EK_INLINE T atomic_update(T* p, F f) {
  static_assert(sizeof(T) == 1 || sizeof(T) == 2 || sizeof(T) == 4, "8/16/32-bit elements");
  if constexpr (sizeof(T) == 4) {
    uint32_t* w = reinterpret_cast<uint32_t*>(p);
    uint32_t o = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    while (true) {
      const T ov = __builtin_bit_cast(T, o);
      const uint32_t n = __builtin_bit_cast(uint32_t, (T)f(ov));
      if (n == o || __hip_atomic_compare_exchange_strong(w, &o, n, __ATOMIC_RELAXED,
                                                        __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT))
        return ov;
    }
  } else {
    typedef typename UBits<sizeof(T)>::type Bits;
    const uint64_t a = reinterpret_cast<uint64_t>(p);
    uint32_t* w = reinterpret_cast<uint32_t*>(a & ~(uint64_t)3);
    const int sh = (int)(a & 3) * 8;
    const uint32_t m = (uint32_t)(Bits)~(Bits)0 << sh;
    uint32_t o = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    while (true) {
      const T ov = __builtin_bit_cast(T, (Bits)(o >> sh));
      const uint32_t n = (o & ~m) | ((uint32_t)__builtin_bit_cast(Bits, (T)f(ov)) << sh);
      if (n == o || __hip_atomic_compare_exchange_strong(w, &o, n, __ATOMIC_RELAXED,
                                                        __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT))
        return ov;
    }
  }
}

// tl.device_print: 16-bit floats print through float; everything else as itself.
template <typename T> EK_INLINE T f32_or_self(T x) { return x; }
EK_INLINE float f32_or_self(_Float16 x) { return (float)x; }
EK_INLINE float f32_or_self(bf16 x) { return bf16_to_f32(x); }

// Buffer resource as four SGPR words, for the inline-asm copy below.
typedef int i32x4 __attribute__((ext_vector_type(4)));
EK_INLINE i32x4 rsrc_words(const void* base, uint32_t nbytes) {
  const uint64_t b = (uint64_t)base;
  return i32x4{(int)(uint32_t)b, (int)((b >> 32) & 0xffff), (int)nbytes, 0x00020000};
}
// LDS byte address of a pointer into __shared__ memory.
EK_INLINE uint32_t lds_addr(const void* p) {
  return (uint32_t)(uint64_t)(const __attribute__((address_space(3))) void*)p;
}
// One 16-byte-per-lane global -> LDS copy (buffer_load_dwordx4 ... lds): lane l's chunk lands
// at LDS byte `lds + 16 * l` (`lds` is wave-uniform). Issued from inline asm so the compiler
// does not order later LDS reads behind it: the caller waits with an explicit vmcnt.
EK_INLINE void dma16(i32x4 rsrc, uint32_t lds, int voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               ::"s"(lds), "v"(voff), "s"(rsrc) : "memory", "m0");
}

template <typename T, int BM, int BN, int BK, int WM, int WN, int NT, bool BUF = false,
          bool TR = false>
struct Gemm {
  static constexpr int TM = BM / WM / 32, TN = BN / WN / 32, TK = BK / 16;
  static constexpr int KC = BK / 8;                    // 16-byte chunks per k row
  static constexpr int A_CH = BM * KC / NT;            // A chunks per thread
  static constexpr int B_TOTAL = KC * (BN / 8);        // B 8x8 blocks per tile
  static constexpr int B_BL = (B_TOTAL + NT - 1) / NT; // B 8x8 blocks per thread
  static constexpr int STAGE = (BM + BN) * BK;         // elements per LDS stage
  static constexpr int LDS_BYTES = 2 * STAGE * 2;
  static_assert(TM >= 1 && TN >= 1 && TK >= 1, "tile too small for 32x32x16 MFMA");
  static_assert((BM * KC) % NT == 0 && (B_TOTAL % NT == 0 || B_TOTAL < NT),
                "tile/thread mismatch");
  static_assert(WM * WN * 64 == NT, "warps must tile the block");

  u32x4 ra[A_CH];
  u32x4 rb[B_BL][8];

  EK_INLINE void load(const uint16_t* A, int lda, const uint16_t* B, int ldb, int M, int N,
                      int K, int m0, int n0, int k, int tid) {
    if constexpr (BUF) {
      // Rows past M (A) or K (B) fall outside the resources; chunks past the last column
      // are sent out of range explicitly.
      const __amdgpu_buffer_rsrc_t ra_r = buffer_rsrc(A, (uint32_t)M * lda * 2);
      const __amdgpu_buffer_rsrc_t rb_r = buffer_rsrc(B, (uint32_t)K * ldb * 2);
#pragma unroll
      for (int i = 0; i < A_CH; ++i) {
        const int c = tid + i * NT, row = c / KC, kc = c % KC;
        const int gk = k + kc * 8;
        const int off = (gk + 8 <= K) ? ((m0 + row) * lda + gk) * 2 : kOOB;
        ra[i] = buffer_load16(ra_r, off);
      }
#pragma unroll
      for (int i = 0; i < B_BL; ++i) {
        const int b = tid + i * NT, nb = b % (BN / 8), kb = b / (BN / 8);
        if (B_TOTAL < NT && b >= B_TOTAL) break;
        const int gn = n0 + nb * 8;
        const int base = (gn + 8 <= N) ? ((k + kb * 8) * ldb + gn) * 2 : kOOB;
#pragma unroll
        for (int j = 0; j < 8; ++j)
          rb[i][j] = buffer_load16(rb_r, base == kOOB ? kOOB : base + j * ldb * 2);
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int c = tid + i * NT, row = c / KC, kc = c % KC;
      const int gr = m0 + row, gk = k + kc * 8;
      if ((unsigned)gr < (unsigned)M && gk >= 0 && gk + 8 <= K) {
        ra[i] = *reinterpret_cast<const u32x4*>(A + (int64_t)gr * lda + gk);
      } else {
        uint16_t h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          h[e] = ((unsigned)gr < (unsigned)M && (unsigned)(gk + e) < (unsigned)K)
                     ? A[(int64_t)gr * lda + gk + e] : 0;
        __builtin_memcpy(&ra[i], h, 16);
      }
    }
#pragma unroll
    for (int i = 0; i < B_BL; ++i) {
      const int b = tid + i * NT, nb = b % (BN / 8), kb = b / (BN / 8);
      if (B_TOTAL < NT && b >= B_TOTAL) break;
      const int gn = n0 + nb * 8;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int gk = k + kb * 8 + j;
        if ((unsigned)gk < (unsigned)K && gn >= 0 && gn + 8 <= N) {
          rb[i][j] = *reinterpret_cast<const u32x4*>(B + (int64_t)gk * ldb + gn);
        } else {
          uint16_t h[8];
#pragma unroll
          for (int e = 0; e < 8; ++e)
            h[e] = ((unsigned)gk < (unsigned)K && (unsigned)(gn + e) < (unsigned)N)
                       ? B[(int64_t)gk * ldb + gn + e] : 0;
          __builtin_memcpy(&rb[i][j], h, 16);
        }
      }
    }
  }

  // LDS addressing (in 16-byte chunks). gfx950 serves LDS reads 256 bytes per pass (16
  // lanes of 16 bytes) and writes 128 bytes per pass (8 lanes). A: row-major [BM][KC]
  // chunks, chunk index xor'ed with (row >> ASH) & AMASK, so the 16 rows a read pass
  // touches land on 16 distinct chunk slots and a write pass (8 chunks of one row) stays
  // contiguous. B^T: k-chunk-major [KC][BN] chunks with the column permuted as
  // n ^ ((n >> 3) & 7), so reads of 16 consecutive columns and writes of the 8 columns
  // n = 8 nb + q (one per 8x8 block) are both conflict-free.
  static constexpr int ASH = KC >= 16 ? 0 : (KC == 8 ? 1 : (KC == 4 ? 2 : 3));
  static constexpr int AMASK = (KC < 16 ? KC : 16) - 1;
  static EK_INLINE int a_chunk(int row, int kc) { return row * KC + (kc ^ ((row >> ASH) & AMASK)); }
  static EK_INLINE int b_chunk(int n, int kc) { return kc * BN + (n ^ ((n >> 3) & 7)); }

  EK_INLINE void store(uint16_t* st, int tid) {
    u32x4* sA = reinterpret_cast<u32x4*>(st);
    u32x4* sB = reinterpret_cast<u32x4*>(st + BM * BK);
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int c = tid + i * NT, row = c / KC, kc = c % KC;
      sA[a_chunk(row, kc)] = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_BL; ++i) {
      const int b = tid + i * NT, nb = b % (BN / 8), kb = b / (BN / 8);
      if (B_TOTAL < NT && b >= B_TOTAL) break;
      u32x4 o[8];
      transpose8x8(rb[i], o);
#pragma unroll
      for (int q = 0; q < 8; ++q) sB[b_chunk(nb * 8 + q, kb)] = o[q];
    }
  }

  EK_INLINE void compute(float* acc, const uint16_t* st, int lane, int wm, int wn) {
    const u32x4* sA = reinterpret_cast<const u32x4*>(st);
    const u32x4* sB = reinterpret_cast<const u32x4*>(st + BM * BK);
    const int r32 = lane & 31, h = lane >> 5;
#pragma unroll
    for (int kk = 0; kk < TK; ++kk) {
      T a[TM][8], b[TN][8];
      const int kc = kk * 2 + h;
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) {
        const u32x4 v = sA[a_chunk(wm * (BM / WM) + tm * 32 + r32, kc)];
        __builtin_memcpy(a[tm], &v, 16);
      }
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const u32x4 v = sB[b_chunk(wn * (BN / WN) + tn * 32 + r32, kc)];
        __builtin_memcpy(b[tn], &v, 16);
      }
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
          if constexpr (TR) mfma_32x32x16(&acc[(tm * TN + tn) * 16], b[tn], a[tm]);
          else mfma_32x32x16(&acc[(tm * TN + tn) * 16], a[tm], b[tn]);
        }
    }
  }

  // Runs the whole k loop: k = lo, lo + BK, ... < hi.
  EK_INLINE void run(float* acc, const T* A, int lda, const T* B, int ldb, int M, int N, int K,
                     int m0, int n0, int lo, int hi, char* smem, int tid) {
    if (hi <= lo) return;
    const int niter = (hi - lo + BK - 1) / BK;
    const int lane = tid & 63, warp = tid >> 6;
    const int wm = warp % WM, wn = warp / WM;
    const uint16_t* A16 = reinterpret_cast<const uint16_t*>(A);
    const uint16_t* B16 = reinterpret_cast<const uint16_t*>(B);
    uint16_t* s16 = reinterpret_cast<uint16_t*>(smem);
    __syncthreads();
    load(A16, lda, B16, ldb, M, N, K, m0, n0, lo, tid);
    store(s16, tid);
    __syncthreads();
    // s_waitcnt vmcnt(0): nothing loaded before the loop (the accumulator's initial value
    // included) is outstanding at its head, so the first MFMA does not wait for the prefetch.
    __builtin_amdgcn_s_waitcnt(0x0F70);
    for (int it = 0; it < niter; ++it) {
      const bool more = it + 1 < niter;
      if (more) load(A16, lda, B16, ldb, M, N, K, m0, n0, lo + (it + 1) * BK, tid);
      compute(acc, s16 + (it & 1) * STAGE, lane, wm, wn);
      if (more) store(s16 + ((it + 1) & 1) * STAGE, tid);
      __syncthreads();
    }
  }
};

// ---------------------------------------------------------------------------
// GEMM main loop fed by LDS DMA: C[BM x BN] += A[BM x K] * B[K x BN], 16-bit row-major
// operands, fp32 accumulators in the 32x32x16 MFMA layout (same as Gemm).
//
//  - Tiles move global -> LDS with buffer_load ... lds (16 bytes per lane, no VGPRs): the 64
//    lanes of one instruction fill 64 consecutive 16-byte LDS chunks, so each lane fetches
//    the global chunk that belongs at its LDS position under the swizzle below. Rows past
//    M (A) or K (B) fall outside the buffer resource and arrive as zeros; chunks past the
//    last column are sent out of range explicitly (K and N are multiples of 8).
//  - S stages in LDS; S - 1 tiles are in flight while one is computed. A stage is waited
//    for with an explicit vmcnt (this wave's copies) and a barrier (everyone's), which also
//    frees the stage consumed one step earlier for the next copy.
//  - A fragments are 16-byte LDS reads; B stays row-major in LDS and its k-major fragments
//    come from ds_read_b64_tr_b16: in each group of 16 lanes, lane 4i + q reads 4 columns of
//    k row i, and output lane L receives column L of the 4 rows.
//  - LDS swizzles (reads are served 256 bytes per pass): A chunk (row, kc) sits at
//    row * KC + (kc ^ ((row >> ASH) & AMASK)); B chunk (k, nc) at
//    k * NCB + (nc ^ (((k >> RSH) & RMASK) << 2)), which spreads the 4 rows a transpose
//    read touches over the 4 64-byte quarters of a pass.
// ---------------------------------------------------------------------------
template <typename T, int BM, int BN, int BK, int WM, int WN, int NT, int S, int SPLIT = 1,
          bool TR = false>
struct GemmDma {
  static constexpr int TM = BM / WM / 32, TN = BN / WN / 32, TK = BK / 16;
  static constexpr int KC = BK / 8;                       // A chunks per row
  static constexpr int NCB = BN / 8;                      // B chunks per row
  static constexpr int A_DMA = BM * KC / NT;              // copies per thread per stage
  static constexpr int B_DMA = BK * NCB / NT;
  static constexpr int D = A_DMA + B_DMA;
  static constexpr int A_ELEMS = BM * BK, STAGE = BM * BK + BK * BN;
  static constexpr int LDS_BYTES = S * STAGE * 2;
  static constexpr int ASH = KC >= 16 ? 0 : (KC == 8 ? 1 : (KC == 4 ? 2 : 3));
  static constexpr int AMASK = (KC < 16 ? KC : 16) - 1;
  static constexpr int RP = BN >= 128 ? 1 : 128 / BN;     // B rows per 256 bytes
  static constexpr int RSH = RP == 1 ? 0 : (RP == 2 ? 1 : 2);
  static constexpr int RMASK = 4 / RP - 1;
  static_assert(TM >= 1 && TN >= 1 && TK >= 1, "tile too small for 32x32x16 MFMA");
  static_assert((BM * KC) % NT == 0 && (BK * NCB) % NT == 0, "tile/thread mismatch");
  static_assert(WM * WN * 64 == NT, "warps must tile the block");
  static_assert(S >= 2 && (S - 2) * D <= 63, "vmcnt range");
  static_assert(NCB >= 4 * (RMASK + 1), "B swizzle needs the row's chunks");
  static_assert(SPLIT >= 0 && SPLIT <= TK, "copies issue after SPLIT of the TK k slices");

  static EK_INLINE int a_chunk(int row, int kc) { return row * KC + (kc ^ ((row >> ASH) & AMASK)); }
  static EK_INLINE int b_chunk(int k, int nc) { return k * NCB + (nc ^ (((k >> RSH) & RMASK) << 2)); }

  // Per-thread copy plan, fixed for the whole loop: the global element offset of each chunk
  // relative to the k origin, or -1 when the chunk's column lies outside the operand.
  int a_off[A_DMA], b_off[B_DMA], a_kc[A_DMA];

  EK_INLINE void plan(int lda, int ldb, int N, int m0, int n0, int tid) {
#pragma unroll
    for (int i = 0; i < A_DMA; ++i) {
      const int p = i * NT + tid, row = p / KC;
      const int kc = (p % KC) ^ ((row >> ASH) & AMASK);
      a_kc[i] = kc * 8;
      a_off[i] = (m0 + row) * lda + kc * 8;
    }
#pragma unroll
    for (int i = 0; i < B_DMA; ++i) {
      const int p = i * NT + tid, k = p / NCB;
      const int nc = (p % NCB) ^ (((k >> RSH) & RMASK) << 2);
      const int gn = n0 + nc * 8;
      b_off[i] = (gn + 8 <= N) ? k * ldb + gn : -1;
    }
  }

  // Copies the k-th tile (k = first column of A / row of B) into the stage at LDS byte `st`.
  EK_INLINE void copy(i32x4 ra, i32x4 rb, int ldb, int K, int k, uint32_t st, int wave) {
    if (k + BK <= K) {
      // the whole k slice lies inside A: no per-chunk column test
#pragma unroll
      for (int i = 0; i < A_DMA; ++i) dma16(ra, st + (i * NT + wave * 64) * 16, (a_off[i] + k) * 2);
    } else {
#pragma unroll
      for (int i = 0; i < A_DMA; ++i) {
        const int off = (k + a_kc[i] + 8 <= K) ? (a_off[i] + k) * 2 : kOOB;
        dma16(ra, st + (i * NT + wave * 64) * 16, off);
      }
    }
#pragma unroll
    for (int i = 0; i < B_DMA; ++i) {
      const int off = b_off[i] >= 0 ? (b_off[i] + k * ldb) * 2 : kOOB;
      dma16(rb, st + A_ELEMS * 2 + (i * NT + wave * 64) * 16, off);
    }
  }

  // The j-th of this thread's D copies of the k-th tile (j < A_DMA: A, else B).
  EK_INLINE void copy_one(int j, i32x4 ra, i32x4 rb, int ldb, int K, int k, uint32_t st,
                          int wave) {
    if (j < A_DMA) {
      const int off = (k + BK <= K || k + a_kc[j] + 8 <= K) ? (a_off[j] + k) * 2 : kOOB;
      dma16(ra, st + (j * NT + wave * 64) * 16, off);
    } else {
      const int i = j - A_DMA;
      const int off = b_off[i] >= 0 ? (b_off[i] + k * ldb) * 2 : kOOB;
      dma16(rb, st + A_ELEMS * 2 + (i * NT + wave * 64) * 16, off);
    }
  }

  // One k slice: every A and B fragment read, then the TM x TN MFMAs.
  EK_INLINE void compute_kk(int kk, float* acc, const uint16_t* st, int lane, int wm, int wn) {
    typedef short v4s __attribute__((ext_vector_type(4)));
    const u32x4* sA = reinterpret_cast<const u32x4*>(st);
    const uint16_t* sB = st + A_ELEMS;
    const int r32 = lane & 31, h = lane >> 5;
    const int g = lane >> 4, ti = (lane >> 2) & 3, tq = lane & 3;
    T a[TM][8], b[TN][8];
    const int kc = kk * 2 + h;
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      const u32x4 v = sA[a_chunk(wm * (BM / WM) + tm * 32 + r32, kc)];
      __builtin_memcpy(a[tm], &v, 16);
    }
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const int n = wn * (BN / WN) + tn * 32 + 16 * (g & 1) + 4 * tq;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int k = kk * 16 + 8 * (g >> 1) + 4 * half + ti;
        const uint16_t* src = sB + b_chunk(k, n >> 3) * 8 + (n & 7);
        const v4s v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4s*)(src));
        __builtin_memcpy(&b[tn][4 * half], &v, 8);
      }
    }
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        if constexpr (TR) mfma_32x32x16(&acc[(tm * TN + tn) * 16], b[tn], a[tm]);
        else mfma_32x32x16(&acc[(tm * TN + tn) * 16], a[tm], b[tn]);
      }
  }

  template <int KK0, int KK1>
  EK_INLINE void compute(float* acc, const uint16_t* st, int lane, int wm, int wn) {
#pragma unroll
    for (int kk = KK0; kk < KK1; ++kk) compute_kk(kk, acc, st, lane, wm, wn);
  }

  // Runs the whole k loop: k = lo, lo + BK, ... < hi.
  EK_INLINE void run(float* acc, const T* A, int lda, const T* B, int ldb, int M, int N, int K,
                     int m0, int n0, int lo, int hi, char* smem, int tid) {
    if (hi <= lo) return;
    const int niter = (hi - lo + BK - 1) / BK;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % WM, wn = wave / WM;
    const i32x4 ra = rsrc_words(A, (uint32_t)M * lda * 2);
    const i32x4 rb = rsrc_words(B, (uint32_t)K * ldb * 2);
    const uint16_t* s16 = reinterpret_cast<const uint16_t*>(smem);
    const uint32_t l0 = lds_addr(smem);
    plan(lda, ldb, N, m0, n0, tid);
    __syncthreads();  // earlier users of the LDS are done with it
    // nothing loaded before the loop is outstanding, so the explicit vmcnt below counts
    // this loop's copies only
    __builtin_amdgcn_s_waitcnt(0x0F70);
#pragma unroll
    for (int s = 0; s < S - 1; ++s) copy(ra, rb, ldb, K, lo + s * BK, l0 + s * STAGE * 2, wave);
    for (int it = 0; it < niter; ++it) {
      // this wave's copies of stage `it` have landed (S - 2 younger stages may still fly),
      // its reads of the previous stage are complete; then everyone's are.
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((S - 2) * D) : "memory");
      // The first SPLIT k slices' fragment reads go out before any copy, so their latency
      // hides behind the copy issue instead of stalling the first MFMA; the copies of the
      // stage S - 1 ahead are then spread over the remaining slices, a share before each
      // slice's reads, so each share's issue overlaps the MFMAs already queued (as one block
      // the copies kept the wave from issuing for 500-800 cycles per k step).
      const uint16_t* cur = s16 + (it % S) * STAGE;
      compute<0, SPLIT>(acc, cur, lane, wm, wn);
      if constexpr (SPLIT < TK) {
        constexpr int SL = TK - SPLIT, PER = (D + SL - 1) / SL;
        const int kn = lo + (it + S - 1) * BK;
        const uint32_t stn = l0 + ((it + S - 1) % S) * STAGE * 2;
#pragma unroll
        for (int q = 0; q < SL; ++q) {
#pragma unroll
          for (int j = q * PER; j < (q + 1) * PER && j < D; ++j)
            copy_one(j, ra, rb, ldb, K, kn, stn, wave);
          compute_kk(SPLIT + q, acc, cur, lane, wm, wn);
        }
      } else {
        copy(ra, rb, ldb, K, lo + (it + S - 1) * BK, l0 + ((it + S - 1) % S) * STAGE * 2, wave);
      }
    }
    // drain the copies issued past the end before anyone reuses the LDS
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  }
};

}  // namespace ek
