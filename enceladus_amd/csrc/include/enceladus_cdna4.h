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

typedef signed char int8_t;
typedef unsigned char uint8_t;
typedef short int16_t;
typedef unsigned short uint16_t;
typedef int int32_t;
typedef unsigned int uint32_t;
typedef long long int64_t;
typedef unsigned long long uint64_t;

#define EK_INLINE __device__ __attribute__((always_inline)) inline

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
EK_INLINE bf16 f32_to_bf16(float f) {
  uint32_t u = f32_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return bf16{(uint16_t)((u >> 16) | 0x40u)};  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest, ties to even
  return bf16{(uint16_t)(u >> 16)};
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
template <typename T> EK_INLINE T f2i(float x);
template <> EK_INLINE int32_t f2i<int32_t>(float x) {
  if (x != x) return 0;
  if (x >= 2147483648.0f) return 2147483647;
  if (x <= -2147483648.0f) return (int32_t)0x80000000u;
  return (int32_t)x;
}
template <> EK_INLINE uint32_t f2i<uint32_t>(float x) {
  if (x != x || x <= 0.0f) return 0u;
  if (x >= 4294967296.0f) return 0xffffffffu;
  return (uint32_t)x;
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
#define EK_SMALL_F2I(T)                                          \
  template <> EK_INLINE T f2i<T>(float x) {                      \
    if (x != x) return 0;                                        \
    if (x <= int_limits<T>::lo) return (T)int_limits<T>::lo;     \
    if (x >= int_limits<T>::hi) return (T)int_limits<T>::hi;     \
    return (T)(int32_t)x;                                        \
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
template <typename T> EK_INLINE T ishl(T a, T b) {
  return ((uint64_t)b >= sizeof(T) * 8) ? (T)0 : (T)(a << b);
}
template <typename T> EK_INLINE T ishr(T a, T b) {
  if ((uint64_t)b >= sizeof(T) * 8) return (T)((T)-1 > (T)0 ? 0 : (a < (T)0 ? (T)-1 : (T)0));
  return (T)(a >> b);
}
EK_INLINE float fmodf_(float a, float b) { return __builtin_fmodf(a, b); }

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

// Exchange with lane ^ mask. Masks 1 and 2 use DPP quad permutes, which need no LDS
// hardware; other masks use ds_bpermute.
template <int MASK, typename T> EK_INLINE T shfl_xor(T v) {
  if constexpr (sizeof(T) == 4 && (MASK == 1 || MASK == 2)) {
    int u = __builtin_bit_cast(int, v);
    // quad_perm selectors: [1,0,3,2] = 0xB1 for xor 1; [2,3,0,1] = 0x4E for xor 2.
    constexpr int ctrl = MASK == 1 ? 0xB1 : 0x4E;
    int r = __builtin_amdgcn_mov_dpp(u, ctrl, 0xF, 0xF, false);
    return __builtin_bit_cast(T, r);
  } else {
    return shfl(v, lane_id() ^ MASK);
  }
}

// ---------------------------------------------------------------------------
// Combine functions for reductions and scans.
// ---------------------------------------------------------------------------
struct Sum {
  template <typename T> static EK_INLINE T op(T a, T b) { return a + b; }
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
template <typename V> EK_INLINE void unpack(float* p, V v) { __builtin_memcpy(p, &v, sizeof(V)); }

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

}  // namespace ek
