// Shared helpers of libeinshard_hip: error state, element conversions,
// division by run-time invariant divisors, launch bookkeeping.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "einshard_hip.h"

namespace es {

// ---------------------------------------------------------------------------
// error / diagnostics state (per calling thread)
void set_error(const std::string& message);
void set_kernel(const char* name);
int fail(int status, const std::string& message);
int check_launch(const char* what);

// ---------------------------------------------------------------------------
// Division by an invariant 32-bit divisor with one multiply-high, following
// Granlund & Montgomery, "Division by Invariant Integers using Multiplication"
// (PLDI 1994), Fig. 4.1: for d >= 1 let l = ceil(log2 d) and
//     m = floor(2^32 * (2^l - d) / d) + 1   (fits in 32 bits),
// then for every 0 <= n < 2^32:  n / d = (mulhi(m, n) + n) >> l,
// with the addition carried out in 64 bits.
struct FastDiv {
  uint32_t d;
  uint32_t m;
  uint32_t l;

  __host__ __device__ FastDiv() : d(1), m(1), l(0) {}
  __host__ explicit FastDiv(uint32_t divisor) { init(divisor); }

  __host__ void init(uint32_t divisor) {
    d = divisor < 1 ? 1 : divisor;
    l = 0;
    while ((uint64_t(1) << l) < d) ++l;
    m = uint32_t(((uint64_t(1) << 32) * ((uint64_t(1) << l) - d)) / d + 1);
  }

  __host__ __device__ __forceinline__ uint32_t div(uint32_t n) const {
#if defined(__HIP_DEVICE_COMPILE__)
    uint32_t hi = __umulhi(m, n);
#else
    uint32_t hi = uint32_t((uint64_t(m) * n) >> 32);
#endif
    return uint32_t((uint64_t(hi) + n) >> l);
  }

  // quotient of n < 2^31: mulhi + n cannot carry out of 32 bits
  __host__ __device__ __forceinline__ uint32_t div31(uint32_t n) const {
#if defined(__HIP_DEVICE_COMPILE__)
    return (__umulhi(m, n) + n) >> l;
#else
    return (uint32_t((uint64_t(m) * n) >> 32) + n) >> l;
#endif
  }

  // quotient, remainder in `rem`
  __host__ __device__ __forceinline__ uint32_t divmod(uint32_t n, uint32_t& rem) const {
    uint32_t q = div(n);
    rem = n - q * d;
    return q;
  }
};

// ---------------------------------------------------------------------------
// element conversions
//
// fp32 -> bf16 rounds to nearest-even and maps every NaN to 0x7FC0: the same
// bit pattern torch produces for a bfloat16 result on the CPU.
__host__ __device__ __forceinline__ float bits_to_f32(uint32_t u) {
  union {
    uint32_t u;
    float f;
  } v;
  v.u = u;
  return v.f;
}

__host__ __device__ __forceinline__ uint32_t f32_to_bits(float f) {
  union {
    float f;
    uint32_t u;
  } v;
  v.f = f;
  return v.u;
}

__host__ __device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return bits_to_f32(uint32_t(h) << 16);
}

__host__ __device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = f32_to_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

template <typename T>
struct Elem;

template <>
struct Elem<float> {
  using storage = float;
  static __device__ __forceinline__ float load(float v) { return v; }
  static __device__ __forceinline__ float store(float v) { return v; }
};

struct bf16_t {
  uint16_t bits;
};
struct f16_t {
  uint16_t bits;
};

template <>
struct Elem<bf16_t> {
  using storage = uint16_t;
  static __device__ __forceinline__ float load(uint16_t v) { return bf16_to_f32(v); }
  static __device__ __forceinline__ uint16_t store(float v) { return f32_to_bf16(v); }
};

template <>
struct Elem<f16_t> {
  using storage = uint16_t;
  static __device__ __forceinline__ float load(uint16_t v) {
    union {
      uint16_t u;
      _Float16 h;
    } c;
    c.u = v;
    return float(c.h);
  }
  static __device__ __forceinline__ uint16_t store(float v) {
    union {
      _Float16 h;
      uint16_t u;
    } c;
    c.h = _Float16(v);  // round to nearest even
    return c.u;
  }
};

// ---------------------------------------------------------------------------
// Streaming (nontemporal) access for data a kernel touches exactly once: the
// load or store carries the nontemporal hint, so streamed lines do not displace
// reused data in the caches.  On MI355X this lifts a pure read stream from about
// 78 % to about 87 % of HBM bandwidth.  V is any trivially copyable 1, 2, 4, 8 or
// 16-byte value.
template <int N>
struct NtWord;
template <>
struct NtWord<1> { using type = uint8_t; };
template <>
struct NtWord<2> { using type = uint16_t; };
template <>
struct NtWord<4> { using type = uint32_t; };
template <>
struct NtWord<8> { using type = unsigned int __attribute__((ext_vector_type(2))); };
template <>
struct NtWord<16> { using type = unsigned int __attribute__((ext_vector_type(4))); };

template <typename V>
__device__ __forceinline__ V load_nt(const V* p) {
  using W = typename NtWord<sizeof(V)>::type;
  return __builtin_bit_cast(V, __builtin_nontemporal_load(reinterpret_cast<const W*>(p)));
}

template <typename V>
__device__ __forceinline__ void store_nt(V* p, const V& v) {
  using W = typename NtWord<sizeof(V)>::type;
  __builtin_nontemporal_store(__builtin_bit_cast(W, v), reinterpret_cast<W*>(p));
}

inline int dtype_size(int dtype) {
  switch (dtype) {
    case ES_F32: return 4;
    case ES_BF16: return 2;
    case ES_F16: return 2;
    default: return 0;
  }
}

inline const char* dtype_name(int dtype) {
  switch (dtype) {
    case ES_F32: return "f32";
    case ES_BF16: return "bf16";
    case ES_F16: return "f16";
    default: return "?";
  }
}

inline bool aligned(const void* p, int bytes) {
  return (reinterpret_cast<uintptr_t>(p) % uintptr_t(bytes)) == 0;
}

constexpr uint64_t kU32Max = 0xffffffffull;

// Number of work-groups that keeps every CU of an MI355X (256 CUs, 8 XCDs)
// busy with several resident groups; fixed so that sizing decisions are a
// pure function of the descriptor.
constexpr int kTargetGroups = 256 * 8;
// Compute units of an MI355X: tile-count decisions assume them, so they too are a
// pure function of the descriptor.
constexpr int kCUs = 256;

}  // namespace es
