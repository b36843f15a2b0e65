// Kernel template behind es_contract (see es_contract.h for the design).
// Included by one translation unit per element type.
#pragma once

#include "es_contract.h"

#include <type_traits>

namespace es {
namespace contract {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

// offset of linear index `i` of a group in the operand selected by WHICH
// (0 = A, 1 = B, 2 = C)
template <int WHICH>
__device__ __forceinline__ int64_t group_offset(const GroupArgs& g, uint32_t i) {
  int64_t off = 0;
#pragma unroll
  for (int d = ES_MAX_AXES - 1; d >= 0; --d) {
    if (d < g.n) {
      uint32_t r;
      i = g.div[d].divmod(i, r);
      const int64_t s = WHICH == 0 ? g.sa[d] : (WHICH == 1 ? g.sb[d] : g.sc[d]);
      off += int64_t(r) * s;
    }
  }
  return off;
}

// ---- element-type traits ----------------------------------------------------
template <typename T>
struct Traits;

template <>
struct Traits<float> {
  using S = float;
  static constexpr int VEC = 4;  // elements per 16 bytes
  static __device__ __forceinline__ void mma(f32x16& acc, const uint4& nfrag, const uint4& mfrag) {
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(nfrag.x), __uint_as_float(mfrag.x), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(nfrag.y), __uint_as_float(mfrag.y), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(nfrag.z), __uint_as_float(mfrag.z), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(nfrag.w), __uint_as_float(mfrag.w), acc, 0, 0, 0);
  }
  static __device__ __forceinline__ S from_float(float v) { return v; }
};

template <>
struct Traits<bf16_t> {
  using S = uint16_t;
  static constexpr int VEC = 8;
  static __device__ __forceinline__ void mma(f32x16& acc, const uint4& nfrag, const uint4& mfrag) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, nfrag), __builtin_bit_cast(bf16x8, mfrag),
                                                  acc, 0, 0, 0);
  }
  static __device__ __forceinline__ S from_float(float v) { return f32_to_bf16(v); }
  // two values rounded to nearest even and packed (v_cvt_pk_bf16_f32); a NaN stays a
  // quiet NaN (its bit pattern is not specified: torch itself rounds NaN to 0x7FC0 in
  // scalar code and to 0xFFFF in vectorised code)
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
  }
};

template <>
struct Traits<f16_t> {
  using S = uint16_t;
  static constexpr int VEC = 8;
  static __device__ __forceinline__ void mma(f32x16& acc, const uint4& nfrag, const uint4& mfrag) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, nfrag), __builtin_bit_cast(f16x8, mfrag),
                                                 acc, 0, 0, 0);
  }
  static __device__ __forceinline__ S from_float(float v) { return Elem<f16_t>::store(v); }
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    return uint32_t(from_float(a)) | (uint32_t(from_float(b)) << 16);
  }
};

// ---- LDS tile geometry -----------------------------------------------------------
// A tile is ROWS rows of BK elements (128 bytes for every element type: BK = 64 for
// 16-bit types, 32 for fp32), K-contiguous, no padding.  The 16-byte chunk c of row r
// lives at chunk position c ^ ((r / 2) % 8): sixteen consecutive rows then cover all
// sixteen 16-byte slots of a 256-byte LDS line, so the fragment reads (32 consecutive
// rows, one chunk) and the global->LDS writes are free of bank conflicts.
constexpr int kRowBytes = 128;
constexpr int kChunks = kRowBytes / 16;  // 8
constexpr int kLdsBytes = 160 * 1024;    // LDS of one work-group on gfx950

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row >> 1) & (kChunks - 1)); }

// ---- register transposes for MN-contiguous tiles -----------------------------
// in[r] holds VEC consecutive mn-elements of k-row r; out[j] holds the VEC
// k-elements of mn-column j.
__device__ __forceinline__ void transpose_block(const uint4 (&in)[8], uint4 (&out)[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int p = j / 2;
    const bool hi = j & 1;
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t a = (&in[2 * q].x)[p];
      const uint32_t b = (&in[2 * q + 1].x)[p];
      w[q] = hi ? __builtin_amdgcn_perm(b, a, 0x07060302u) : __builtin_amdgcn_perm(b, a, 0x05040100u);
    }
    out[j] = uint4{w[0], w[1], w[2], w[3]};
  }
}

__device__ __forceinline__ void transpose_block(const uint4 (&in)[4], uint4 (&out)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) out[j] = uint4{(&in[0].x)[j], (&in[1].x)[j], (&in[2].x)[j], (&in[3].x)[j]};
}

// ---- incremental K walk ----------------------------------------------------------
// Fast paths have at most kKLevels K sub-axes and the innermost one is a multiple of
// BK, so the offset of K tile t+1 follows from tile t by one addition: the delta of the
// lowest level that does not wrap (see ContractArgs::kcnt).  L is the number of levels
// the walk keeps (1, 2 or kKLevels; levels beyond the descriptor's never wrap).  The
// limits and deltas are read from the kernel arguments once, at start, and kept in
// (scalar) registers: an advance is a handful of compares and selects, with no memory
// access that could make the wave wait behind its LDS reads.
template <int L>
struct KWalk {
  static constexpr int W = L > 1 ? L - 1 : 1;  // levels that can wrap (all but the outermost)
  uint32_t cnt[W];  // position at each wrapping level
  uint32_t lim[W];  // its extent
  int64_t da[L], db[L];
  int64_t off_a;  // element offset of the tile in A
  int64_t off_b;  // ... in B
  __device__ __forceinline__ void start(const ContractArgs& p) {
#pragma unroll
    for (int l = 0; l < W; ++l) {
      cnt[l] = 0;
      lim[l] = p.kcnt[l];
    }
#pragma unroll
    for (int l = 0; l < L; ++l) {
      da[l] = p.kda[l];
      db[l] = p.kdb[l];
    }
    off_a = 0;
    off_b = 0;
  }
  // the step from K tile t to t + 1
  __device__ __forceinline__ void next(int64_t& sa, int64_t& sb, uint32_t (&c)[W]) const {
    sa = da[L - 1];
    sb = db[L - 1];
#pragma unroll
    for (int l = 0; l < W; ++l) c[l] = cnt[l];
    if constexpr (L > 1) {
      // the lowest level that does not wrap takes the increment (and its delta); the
      // levels below it wrap to 0; if every wrapping level wraps, the outermost level
      // takes it and sa / sb keep its delta
      bool done = false;
#pragma unroll
      for (int l = 0; l < L - 1; ++l) {
        const bool wrap = cnt[l] + 1 == lim[l];
        const bool inc = !done && !wrap;
        sa = inc ? da[l] : sa;
        sb = inc ? db[l] : sb;
        c[l] = done ? cnt[l] : (wrap ? 0u : cnt[l] + 1);
        done = done || !wrap;
      }
    }
  }
  __device__ __forceinline__ void advance() {
    int64_t sa, sb;
    uint32_t c[W];
    next(sa, sb, c);
    off_a += sa;
    off_b += sb;
#pragma unroll
    for (int l = 0; l < W; ++l) cnt[l] = c[l];
  }
};

// ---- work-group -> tile ------------------------------------------------------------
// The hardware deals work-groups to the 8 XCDs round robin.  Work-group b is given
// logical tile (b % 8) * (tiles / 8) + b / 8, so each XCD owns a contiguous run of
// logical tiles; logical tiles walk groups of group_n N-tiles, M fastest inside a
// group, so that run is a compact rectangle of group_n N-tiles by run / group_n
// M-tiles and the XCD's L2 sees few distinct A and B panels.
// The three divisions use divisors prepared on the host (a multiply-high and a shift
// each instead of an integer division sequence).
__device__ __forceinline__ void tile_of(const ContractArgs& p, uint32_t b, uint32_t& bidx, uint32_t& tm, uint32_t& tn) {
  if (p.total_tiles % 8 == 0) b = (b % 8) * (p.total_tiles / 8) + b / 8;
  bidx = p.tdiv_batch.div31(b);
  const uint32_t rem = b - bidx * p.tdiv_batch.d;
  const uint32_t g = p.tdiv_group.div31(rem);
  const uint32_t r = rem - g * p.tdiv_group.d;
  tm = p.tdiv_gn.div31(r);
  tn = g * p.group_n + (r - tm * p.group_n);
}

// Offset of index i of a group in the operand selected by WHICH: the generic walk over
// the sub-axes (G = 0), or (G > 0: the group has at most G sub-axes; the unused ones have
// extent 1 and stride 0) G - 1 divisions, unrolled, with the outermost sub-axis taking
// the quotient left (i is below the group's extent).
template <int WHICH, int G>
__device__ __forceinline__ int64_t group_offset_d(const GroupArgs& g, uint32_t i) {
  if constexpr (G == 0) {
    return group_offset<WHICH>(g, i);
  } else {
    int64_t off = 0;
#pragma unroll
    for (int d = G - 1; d > 0; --d) {
      uint32_t r;
      i = g.div[d].divmod(i, r);
      off += int64_t(r) * (WHICH == 0 ? g.sa[d] : (WHICH == 1 ? g.sb[d] : g.sc[d]));
    }
    return off + int64_t(i) * (WHICH == 0 ? g.sa[0] : (WHICH == 1 ? g.sb[0] : g.sc[0]));
  }
}

// The same in 32 bits (a row's offset within an operand whose every offset fits 32 bits;
// `scale` the element size): the low 32 bits of group_offset_d's result times scale.
template <int WHICH, int G>
__device__ __forceinline__ uint32_t group_offset_d32(const GroupArgs& g, uint32_t i, uint32_t scale) {
  static_assert(G > 0, "bounded groups only");
  uint32_t off = 0;
#pragma unroll
  for (int d = G - 1; d > 0; --d) {
    uint32_t r;
    i = g.div[d].divmod(i, r);
    off += r * uint32_t((WHICH == 0 ? g.sa[d] : (WHICH == 1 ? g.sb[d] : g.sc[d])) * scale);
  }
  return off + i * uint32_t((WHICH == 0 ? g.sa[0] : (WHICH == 1 ? g.sb[0] : g.sc[0])) * scale);
}

// ---- tile loaders -------------------------------------------------------------
__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return uint32_t(uintptr_t((const lds_void*)p));
}

// One 1 KB global -> LDS copy from per-lane 64-bit addresses (global_load_lds_dwordx4,
// vector-address form): lane l moves 16 bytes from src into LDS byte address
// lds + 16 * l.  Inline assembly: a copy the compiler can see makes it wait for every
// copy in flight, the prefetched ones included, before the next LDS read.  The
// kernels order LDS reads behind the copies with explicit s_waitcnt vmcnt and
// barriers; loads the compiler cannot see only make its own waits longer.  lds is the
// same in every lane.
__device__ __forceinline__ void copy_to_lds_v(const void* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src),
               "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}

// A 4-byte load per lane into a 256-byte LDS sink (global_load_lds_dword): brings the
// line at src into L2 ahead of its copy.  Inline assembly for the same reason.
__device__ __forceinline__ void touch_to_lds(const void* src, uint32_t sink) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(src),
               "s"(__builtin_amdgcn_readfirstlane(sink))
               : "memory");
}

// Bias of output column n (0 past the last column), loaded without a branch: the index
// is clamped to the last column and the value dropped afterwards.  A run of these is
// issued back to back; a load behind `n < N` got a branch and a wait of its own each.
template <typename T>
__device__ __forceinline__ float bias_at(const ContractArgs& p, uint32_t n) {
  using S = typename Traits<T>::S;
  const float v = Elem<T>::load(static_cast<const S*>(p.bias)[n < p.N ? n : p.N - 1]);
  return n < p.N ? v : 0.f;
}

// SIDE 0 loads the M-side tile from A, SIDE 1 the N-side tile from B.
template <typename T, int ROWS, int BK, int NT, int LAYOUT, int SIDE>
struct Loader;

// K-contiguous: direct global -> LDS copies (global_load_lds_dwordx4).  One wave
// instruction fills one 1 KB region (8 rows x 128 bytes); lane l writes slot l, i.e.
// row l / 8 and chunk position l % 8, so it fetches the logical chunk stored there.
template <typename T, int ROWS, int BK, int NT, int SIDE>
struct Loader<T, ROWS, BK, NT, kKContig, SIDE> {
  using S = typename Traits<T>::S;
  static constexpr int VEC = Traits<T>::VEC;
  static constexpr int NW = NT / 64;
  static constexpr int RPI = 64 / kChunks;  // rows per wave instruction
  static constexpr int NI = ROWS / RPI / NW;
  static_assert(NI >= 1 && ROWS % (RPI * NW) == 0, "tile shape");
  static constexpr bool kDirect = true;

  const S* src[NI];
  int region0;  // first 1 KB region of this wave

  __device__ __forceinline__ void init(const ContractArgs& p, int tid, uint32_t row0, int64_t boff) {
    const int lane = tid % 64;
    const int wave = tid / 64;
    region0 = wave * NI;
    const GroupArgs& g = SIDE == 0 ? p.gm : p.gn;
    const uint32_t lim = (SIDE == 0 ? p.M : p.N) - 1;
    const S* base = static_cast<const S*>(SIDE == 0 ? p.a : p.b);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int row = (region0 + i) * RPI + lane / kChunks;
      const int chunk = swz(row, lane % kChunks);
      uint32_t r = row0 + row;
      r = r > lim ? lim : r;  // rows past the edge re-read the last row; never stored
      src[i] = base + boff + group_offset<SIDE>(g, r) + chunk * VEC;
    }
  }

  // enqueue the copies of the K tile at element offset `koff` into LDS tile `dst`.
  // ASM: as inline assembly, when both operands are copied this way (then the compiler
  // would otherwise wait for the next tile's copies before this tile's LDS reads).
  // Beside an operand staged through registers the builtin measured faster: the
  // compiler then interleaved waits with that operand's loads.
  template <bool ASM>
  __device__ __forceinline__ void issue(S* dst, int64_t koff) const {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      if constexpr (ASM)
        copy_to_lds_v(src[i] + koff, lds_address(dst + (region0 + i) * 512 * 2 / sizeof(S)));
      else
        __builtin_amdgcn_global_load_lds((const void*)(src[i] + koff),
                                         (lds_void*)(dst + (region0 + i) * 512 * 2 / sizeof(S)), 16, 0, 0);
    }
  }
  __device__ __forceinline__ void load(const ContractArgs&, uint32_t, int64_t) {}
  __device__ __forceinline__ void store(S*) const {}
};

// MN-contiguous: VEC x VEC blocks loaded along mn, transposed in registers
template <typename T, int ROWS, int BK, int NT, int SIDE>
struct Loader<T, ROWS, BK, NT, kMNContig, SIDE> {
  using S = typename Traits<T>::S;
  static constexpr int VEC = Traits<T>::VEC;
  static constexpr int MG = ROWS / VEC;
  static constexpr int KG = BK / VEC;
  static constexpr int NB = (MG * KG + NT - 1) / NT;
  static constexpr bool kDirect = false;

  const S* src[NB];
  uint4 reg[NB][VEC];
  int mg[NB], kg[NB];
  int64_t kstride;

  __device__ __forceinline__ void init(const ContractArgs& p, int tid, uint32_t row0, int64_t boff) {
    const GroupArgs& g = SIDE == 0 ? p.gm : p.gn;
    const uint32_t lim = (SIDE == 0 ? p.M : p.N) - VEC;  // last full group (extent % VEC == 0)
    const S* base = static_cast<const S*>(SIDE == 0 ? p.a : p.b);
    kstride = SIDE == 0 ? p.ka_inner : p.kb_inner;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int b = tid + j * NT;
      mg[j] = b % MG;
      kg[j] = b / MG;
      uint32_t r = row0 + mg[j] * VEC;
      r = r > lim ? lim : r;
      src[j] = base + boff + group_offset<SIDE>(g, r) + int64_t(kg[j] * VEC) * kstride;
    }
  }
  template <bool ASM>
  __device__ __forceinline__ void issue(S*, int64_t) const {}

  __device__ __forceinline__ void load(const ContractArgs&, uint32_t, int64_t koff) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      if ((MG * KG) % NT == 0 || kg[j] < KG) {
#pragma unroll
        for (int kk = 0; kk < VEC; ++kk) reg[j][kk] = *reinterpret_cast<const uint4*>(src[j] + koff + kk * kstride);
      }
    }
  }

  __device__ __forceinline__ void store(S* lds) const {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      if ((MG * KG) % NT == 0 || kg[j] < KG) {
        uint4 t[VEC];
        transpose_block(reg[j], t);
#pragma unroll
        for (int jj = 0; jj < VEC; ++jj) {
          const int row = mg[j] * VEC + jj;
          *reinterpret_cast<uint4*>(lds + row * BK + swz(row, kg[j]) * VEC) = t[jj];
        }
      }
    }
  }
};

// generic: one element at a time, any strides, edges in every direction
template <typename T, int ROWS, int BK, int NT, int SIDE>
struct Loader<T, ROWS, BK, NT, kGeneric, SIDE> {
  using S = typename Traits<T>::S;
  static constexpr int VEC = Traits<T>::VEC;
  static constexpr int RPP = NT / BK;
  static constexpr int NE = (ROWS + RPP - 1) / RPP;
  static_assert(NT % BK == 0, "tile shape");
  static constexpr bool kDirect = false;

  int64_t rowoff[NE];
  bool rowok[NE];
  S reg[NE];
  int kk, r0;

  __device__ __forceinline__ void init(const ContractArgs& p, int tid, uint32_t row0, int64_t boff) {
    kk = tid % BK;
    r0 = tid / BK;
    const GroupArgs& g = SIDE == 0 ? p.gm : p.gn;
    const uint32_t extent = SIDE == 0 ? p.M : p.N;
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      const uint32_t r = row0 + r0 + i * RPP;
      rowok[i] = r < extent && r0 + i * RPP < ROWS;
      rowoff[i] = rowok[i] ? boff + group_offset<SIDE>(g, r) : 0;
    }
  }
  template <bool ASM>
  __device__ __forceinline__ void issue(S*, int64_t) const {}

  __device__ __forceinline__ void load(const ContractArgs& p, uint32_t k0, int64_t) {
    const S* base = static_cast<const S*>(SIDE == 0 ? p.a : p.b);
    const uint32_t k = k0 + kk;
    const bool kok = k < p.K;
    const int64_t koff = kok ? group_offset<SIDE>(p.gk, k) : 0;
#pragma unroll
    for (int i = 0; i < NE; ++i) reg[i] = (kok && rowok[i]) ? base[rowoff[i] + koff] : S(0);
  }

  __device__ __forceinline__ void store(S* lds) const {
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      const int row = r0 + i * RPP;
      if (row < ROWS) lds[row * BK + swz(row, kk / VEC) * VEC + kk % VEC] = reg[i];
    }
  }
};

// ---- epilogue ------------------------------------------------------------------
// Group descriptors read from the kernel argument segment (the ContractArgs parameter
// sits at its start) through a constant-address-space pointer, in a loop over the
// sub-axes that is not unrolled: the loads are uniform scalar loads issued where the
// offsets are computed (the epilogue), and no descriptor is held in scalar registers
// through the K loop.
typedef const __attribute__((address_space(4))) ContractArgs* KArgs;
typedef const __attribute__((address_space(4))) GroupArgs* KGroup;

__device__ __forceinline__ KArgs kernel_args() {
#if defined(__HIP_DEVICE_COMPILE__)
  return (KArgs)__builtin_amdgcn_kernarg_segment_ptr();
#else
  return nullptr;  // host pass: parsed, never executed
#endif
}

template <int WHICH>
__device__ __forceinline__ int64_t group_offset_k(KGroup g, uint32_t i) {
  int64_t off = 0;
  const int n = g->n;
#pragma nounroll
  for (int d = n - 1; d >= 0; --d) {
    FastDiv f;
    f.d = g->div[d].d;
    f.m = g->div[d].m;
    f.l = g->div[d].l;
    uint32_t r;
    i = f.divmod(i, r);
    off += int64_t(r) * (WHICH == 0 ? g->sa[d] : (WHICH == 1 ? g->sb[d] : g->sc[d]));
  }
  return off;
}

// group_offset_k, or (G > 0) group_offset_d's bounded walk, unrolled
template <int WHICH, int G>
__device__ __forceinline__ int64_t group_offset_kd(KGroup g, uint32_t i) {
  if constexpr (G == 0) {
    return group_offset_k<WHICH>(g, i);
  } else {
    int64_t off = 0;
#pragma unroll
    for (int d = G - 1; d > 0; --d) {
      FastDiv f;
      f.d = g->div[d].d;
      f.m = g->div[d].m;
      f.l = g->div[d].l;
      uint32_t r;
      i = f.divmod(i, r);
      off += int64_t(r) * (WHICH == 0 ? g->sa[d] : (WHICH == 1 ? g->sb[d] : g->sc[d]));
    }
    return off + int64_t(i) * (WHICH == 0 ? g->sa[0] : (WHICH == 1 ? g->sb[0] : g->sc[0]));
  }
}

// Work-group barrier that waits for this wave's LDS operations only: global stores
// issued before it stay in flight.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// LDS bytes the epilogue needs: the staged slice plus the row / column offset tables
template <typename S, int BM, int BN, int WM>
constexpr int epilogue_bytes() {
  return WM * 32 * (BN + 16 / int(sizeof(S))) * int(sizeof(S)) + (BM + BN) * 8;
}

// acc[i][j] holds C^T of a 32x32 block.  The output offset of every tile row and
// column is computed once (one thread each) into LDS tables; then pass i stages rows
// {wm*WTM + i*32 + 0..31 : wm} (WM*32 rows x BN columns, converted to the element
// type) in LDS as [row][n], and the whole work-group writes them out: 16-byte stores
// along n when n is the output's contiguous axis, element stores otherwise.  `lds`
// holds at least epilogue_bytes(); the caller has drained every copy into LDS and
// synchronised the work-group.
template <typename T, int BM, int BN, int WM, int WN, int FM, int FN, bool BIAS>
__device__ __forceinline__ void store_tile(const ContractArgs& p, void* lds, const f32x16 (&acc)[FM][FN], uint32_t m0,
                                           uint32_t n0, int64_t boff_c) {
  using S = typename Traits<T>::S;
  constexpr int NT = WM * WN * 64;
  constexpr int VEC = 16 / int(sizeof(S));
  constexpr int WTM = BM / WM;
  constexpr int WTN = BN / WN;
  constexpr int SROWS = WM * 32;
  constexpr int SLD = BN + VEC;  // staging row pitch (elements)
  S* stage = static_cast<S*>(lds);
  int64_t* row_off = reinterpret_cast<int64_t*>(static_cast<char*>(lds) + SROWS * SLD * int(sizeof(S)));
  int64_t* col_off = row_off + BM;
  const int tid = threadIdx.x;
  const int lane = tid % 64;
  const int wave = tid / 64;
  const int wm = wave / WN;
  const int wn = wave % WN;
  S* C = static_cast<S*>(p.c);
  const KArgs kp = kernel_args();
  for (int r = tid; r < BM; r += NT) {
    const uint32_t m = m0 + r;
    row_off[r] = m < p.M ? boff_c + group_offset_k<2>(&kp->gm, m) : -1;
  }
  for (int c = tid; c < BN; c += NT) {
    const uint32_t n = n0 + c;
    col_off[c] = n < p.N ? group_offset_k<2>(&kp->gn, n) : -1;
  }
  // BIAS: the bias of this lane's columns (es_contract_bias), added before the one rounding
  float bv[FN][4][4];
#pragma unroll
  for (int j = 0; j < FN; ++j)
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t n = n0 + wn * WTN + j * 32 + 8 * g + 4 * (lane / 32) + r;
        bv[j][g][r] = BIAS ? bias_at<T>(p, n) : 0.f;
      }
  // without a bias nothing is added (bv is then unused and folds away)
  auto biased = [&](float v, int j, int g, int r) { return BIAS ? v + bv[j][g][r] : v; };
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int srow = wm * 32 + lane % 32;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int scol = wn * WTN + j * 32 + 8 * g + 4 * (lane / 32);
        S* dst = stage + srow * SLD + scol;
        if constexpr (sizeof(S) == 4) {
          *reinterpret_cast<float4*>(dst) =
              float4{biased(acc[i][j][4 * g], j, g, 0), biased(acc[i][j][4 * g + 1], j, g, 1),
                     biased(acc[i][j][4 * g + 2], j, g, 2), biased(acc[i][j][4 * g + 3], j, g, 3)};
        } else {
          const float v0 = biased(acc[i][j][4 * g], j, g, 0), v1 = biased(acc[i][j][4 * g + 1], j, g, 1);
          const float v2 = biased(acc[i][j][4 * g + 2], j, g, 2), v3 = biased(acc[i][j][4 * g + 3], j, g, 3);
          *reinterpret_cast<uint2*>(dst) = uint2{Traits<T>::pack2(v0, v1), Traits<T>::pack2(v2, v3)};
        }
      }
    }
    lds_barrier();
    // staged row r is tile row (r / 32) * WTM + i * 32 + r % 32
    if (p.vstore == 1) {
      constexpr int CV = BN / VEC;  // vectors per staged row
      for (int v = tid; v < SROWS * CV; v += NT) {
        const int r = v / CV;
        const int cv = v - r * CV;
        const int64_t ro = row_off[(r / 32) * WTM + i * 32 + r % 32];
        const int64_t co = col_off[cv * VEC];
        // nontemporal: the output is not read again by this kernel, so it is not kept in L2
        if (ro >= 0 && co >= 0)
          __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(stage + r * SLD + cv * VEC),
                                      reinterpret_cast<u32x4*>(C + ro + co));
      }
    } else {
      for (int v = tid; v < SROWS * BN; v += NT) {
        const int r = v / BN;
        const int cn = v - r * BN;
        const int64_t ro = row_off[(r / 32) * WTM + i * 32 + r % 32];
        const int64_t co = col_off[cn];
        if (ro >= 0 && co >= 0) C[ro + co] = stage[r * SLD + cn];
      }
    }
    lds_barrier();
  }
}

// Epilogue for an fp32 output (ContractArgs::out_f32, the partial results of a split-K
// 16-bit contraction): no staging and no rounding.  acc[i][j][4g + r] is column
// wn*WTN + j*32 + 8g + 4*(lane/32) + r of tile row wm*WTM + i*32 + lane%32, so each lane
// writes 4 consecutive columns: one 16-byte store when n is the output's contiguous axis
// (vstore == 1: those 4 floats are contiguous and 16-byte aligned), element stores
// otherwise.  Row and column offsets come from LDS tables as in store_tile.
template <typename T, int BM, int BN, int WM, int WN, int FM, int FN, bool BIAS>
__device__ __forceinline__ void store_tile_f32(const ContractArgs& p, void* lds, const f32x16 (&acc)[FM][FN],
                                               uint32_t m0, uint32_t n0, int64_t boff_c) {
  using S = typename Traits<T>::S;
  constexpr int NT = WM * WN * 64;
  constexpr int WTM = BM / WM;
  constexpr int WTN = BN / WN;
  int64_t* row_off = static_cast<int64_t*>(lds);
  int64_t* col_off = row_off + BM;
  const int tid = threadIdx.x;
  const int lane = tid % 64;
  const int wave = tid / 64;
  const int wm = wave / WN;
  const int wn = wave % WN;
  float* C = static_cast<float*>(p.c);
  const KArgs kp = kernel_args();
  for (int r = tid; r < BM; r += NT) {
    const uint32_t m = m0 + r;
    row_off[r] = m < p.M ? boff_c + group_offset_k<2>(&kp->gm, m) : -1;
  }
  for (int c = tid; c < BN; c += NT) {
    const uint32_t n = n0 + c;
    col_off[c] = n < p.N ? group_offset_k<2>(&kp->gn, n) : -1;
  }
  lds_barrier();
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int64_t ro = row_off[wm * WTM + i * 32 + lane % 32];
    if (ro < 0) continue;
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c = wn * WTN + j * 32 + 8 * g + 4 * (lane / 32);
        f32x4 v{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
        if constexpr (BIAS) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const uint32_t n = n0 + c + r;
            v[r] += bias_at<T>(p, n);
          }
        }
        if (p.vstore == 1) {
          const int64_t co = col_off[c];
          if (co >= 0) *reinterpret_cast<f32x4*>(C + ro + co) = v;
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int64_t co = col_off[c + r];
            if (co >= 0) C[ro + co] = v[r];
          }
        }
      }
  }
}

// ---- the kernel ----------------------------------------------------------------
// PF > 1: K-contiguous operands also pull K tile kt + PF into L2 (a 4-byte LDS-DMA
// per 128-byte row into a scratch slot), so the copies of tile kt + 1 find it there.
template <typename T, int BM, int BN, int WM, int WN, int LA, int LB, int PF>
__global__ __launch_bounds__(WM * WN * 64, 1) void contract_kernel(const ContractArgs p) {
  using S = typename Traits<T>::S;
  constexpr int NT = WM * WN * 64;
  constexpr int VEC = Traits<T>::VEC;
  constexpr int BK = kRowBytes / int(sizeof(S));
  constexpr int KSTEP = 2 * VEC;  // k consumed per fragment read
  constexpr int NS = BK / KSTEP;  // fragment steps per K tile
  constexpr int WTM = BM / WM;
  constexpr int WTN = BN / WN;
  constexpr int FM = WTM / 32;
  constexpr int FN = WTN / 32;
  constexpr int STAGE = (BM + BN) * BK;  // elements per LDS stage
  constexpr bool kGen = LA == kGeneric || LB == kGeneric;
  static_assert(FM >= 1 && FN >= 1, "tile shape");

  __shared__ __attribute__((aligned(1024))) S lds[2 * STAGE];
  __shared__ __attribute__((aligned(256))) uint32_t sink[64];

  const int tid = threadIdx.x;
  const int lane = tid % 64;
  const int wave = tid / 64;
  const int wm = wave / WN;
  const int wn = wave % WN;

  // work-group -> tile.  The hardware deals work-groups to the 8 XCDs round
  // robin; give each XCD a contiguous run of tiles (N fastest) so tiles that
  // share an M panel of A meet in the same L2.
  uint32_t bidx, tm, tn;
  tile_of(p, blockIdx.x, bidx, tm, tn);
  const uint32_t m0 = tm * BM;
  const uint32_t n0 = tn * BN;

  const int64_t boff_a = group_offset<0>(p.gb, bidx);
  const int64_t boff_b = group_offset<1>(p.gb, bidx);
  const int64_t boff_c = group_offset<2>(p.gb, bidx);

  Loader<T, BM, BK, NT, LA, 0> la;
  Loader<T, BN, BK, NT, LB, 1> lb;
  la.init(p, tid, m0, boff_a);
  lb.init(p, tid, n0, boff_b);

  constexpr bool kAsmCopies = LA == kKContig && LB == kKContig;  // see Loader::issue
  // L2 touch addresses: one per 128-byte row of the K-contiguous tiles
  constexpr bool kTouch = PF > 1 && (LA == kKContig || LB == kKContig);
  constexpr int kTouchRows = (LA == kKContig ? BM : 0) + (LB == kKContig ? BN : 0);
  constexpr int kTouches = kTouch ? (kTouchRows + NT - 1) / NT : 0;
  const S* touch_src[kTouches > 0 ? kTouches : 1];
  if constexpr (kTouch) {
#pragma unroll
    for (int q = 0; q < kTouches; ++q) {
      int row = tid + q * NT;
      if (row >= kTouchRows) row = kTouchRows - 1;
      const bool on_a = LA == kKContig && row < BM;
      const int r = LA == kKContig ? (on_a ? row : row - BM) : row;
      const uint32_t lim = (on_a ? p.M : p.N) - 1;
      const uint32_t g = min((on_a ? m0 : n0) + r, lim);
      touch_src[q] = static_cast<const S*>(on_a ? p.a : p.b) + (on_a ? boff_a : boff_b) +
                     (on_a ? group_offset<0>(p.gm, g) : group_offset<1>(p.gn, g));
    }
  }
  auto touch = [&](int64_t koff_a, int64_t koff_b) {
    if constexpr (kTouch) {
#pragma unroll
      for (int q = 0; q < kTouches; ++q) {
        const int row = tid + q * NT;
        const bool on_a = LA == kKContig && row < BM;
        if constexpr (kAsmCopies)
          touch_to_lds(touch_src[q] + (on_a ? koff_a : koff_b), lds_address(sink));
        else
          __builtin_amdgcn_global_load_lds((const void*)(touch_src[q] + (on_a ? koff_a : koff_b)), (lds_void*)sink, 4,
                                           0, 0);
      }
    }
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const uint32_t nk = (p.K + BK - 1) / BK;
  KWalk<kKLevels> kw;  // offset of the next tile to fetch
  kw.start(p);
  KWalk<kKLevels> tw;  // offset of the next tile to touch
  tw.start(p);
  if (nk > 0) {
    la.template issue<kAsmCopies>(&lds[0], kw.off_a);
    lb.template issue<kAsmCopies>(&lds[BM * BK], kw.off_b);
    la.load(p, 0, kw.off_a);
    lb.load(p, 0, kw.off_b);
    la.store(&lds[0]);
    lb.store(&lds[BM * BK]);
    if (!kGen) kw.advance();
    if constexpr (kTouch) {
      tw.advance();
#pragma unroll
      for (int d = 1; d < PF; ++d) {
        if (uint32_t(d) < nk) touch(tw.off_a, tw.off_b);
        if (uint32_t(d) < nk) tw.advance();
      }
    }
  }

  // fragment rows of this lane
  int arow[FM], brow[FN];
#pragma unroll
  for (int i = 0; i < FM; ++i) arow[i] = wm * WTM + i * 32 + lane % 32;
#pragma unroll
  for (int j = 0; j < FN; ++j) brow[j] = wn * WTN + j * 32 + lane % 32;

  for (uint32_t kt = 0; kt < nk; ++kt) {
    // Tile kt's copies must have landed.  Vector-memory loads complete in issue
    // order; the only loads issued after them are the touches of the previous
    // iteration (its staged register loads were consumed by its LDS stores), so
    // leaving exactly that many outstanding is enough.
    if (kTouch && kt >= 1 && kt - 1 + PF < nk) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kTouches) : "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      S* nxt = &lds[(cur ^ 1) * STAGE];
      la.template issue<kAsmCopies>(nxt, kw.off_a);
      lb.template issue<kAsmCopies>(nxt + BM * BK, kw.off_b);
      la.load(p, (kt + 1) * BK, kw.off_a);
      lb.load(p, (kt + 1) * BK, kw.off_b);
      if (!kGen) kw.advance();
      if constexpr (kTouch) {
        if (kt + PF < nk) {
          touch(tw.off_a, tw.off_b);
          tw.advance();
        }
      }
    }
    const S* As = &lds[cur * STAGE];
    const S* Bs = As + BM * BK;
    uint4 af[2][FM], bf[2][FN];
    auto frags = [&](int buf, int ks) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[buf][i] = *reinterpret_cast<const uint4*>(As + arow[i] * BK + swz(arow[i], ks * 2 + lane / 32) * VEC);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bf[buf][j] = *reinterpret_cast<const uint4*>(Bs + brow[j] * BK + swz(brow[j], ks * 2 + lane / 32) * VEC);
    };
    frags(0, 0);
#pragma unroll
    for (int ks = 0; ks < NS; ++ks) {
      if (ks + 1 < NS) frags((ks + 1) & 1, ks + 1);
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) Traits<T>::mma(acc[i][j], bf[ks & 1][j], af[ks & 1][i]);
      __builtin_amdgcn_s_setprio(0);
    }
    if (more) {
      S* nxt = &lds[(cur ^ 1) * STAGE];
      la.store(nxt);
      lb.store(nxt + BM * BK);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  static_assert(epilogue_bytes<S, BM, BN, WM>() <= int(sizeof(lds)), "epilogue must fit in LDS");
  if constexpr (sizeof(S) == 2) {
    if (p.out_f32) {
      if (p.bias != nullptr) store_tile_f32<T, BM, BN, WM, WN, FM, FN, true>(p, lds, acc, m0, n0, boff_c);
      else store_tile_f32<T, BM, BN, WM, WN, FM, FN, false>(p, lds, acc, m0, n0, boff_c);
      return;
    }
  }
  if (p.bias != nullptr) store_tile<T, BM, BN, WM, WN, FM, FN, true>(p, lds, acc, m0, n0, boff_c);
  else store_tile<T, BM, BN, WM, WN, FM, FN, false>(p, lds, acc, m0, n0, boff_c);
}

// ---- software-pipelined kernel, both operands K-contiguous (pieces) ----------------
// K walk of contract_pipe's copies.  The loop body has no branches: past the last K
// tile the copies re-fetch the last tile into a stage nobody reads.
template <int L>
struct PipeWalk {
  uint32_t t;  // K tile index of the next copy
  KWalk<L> k;  // its offsets in A and B (oa / ob)
  int64_t oa, ob;

  __device__ __forceinline__ void start(const ContractArgs& p) {
    t = 0;
    k.start(p);
    oa = ob = 0;
  }
  // next tile, or stay on the last one (branch-free)
  __device__ __forceinline__ void advance(uint32_t nk) {
    const bool step = t + 1 < nk;
    int64_t sa, sb;
    uint32_t c[KWalk<L>::W];
    k.next(sa, sb, c);
    oa += step ? sa : 0;
    ob += step ? sb : 0;
#pragma unroll
    for (int l = 0; l < KWalk<L>::W; ++l) k.cnt[l] = step ? c[l] : k.cnt[l];
    t += step ? 1u : 0u;
  }
};

// One 1 KB global -> LDS copy: lane l moves 16 bytes from sbase + voff into LDS byte
// address lds + 16 * l (global_load_lds_dwordx4, scalar-base form).  Issued as inline
// assembly: the compiler then keeps the per-lane offset in one loop-invariant register
// (instead of a 64-bit address it may reuse while the copy still reads it) and does not
// order LDS reads behind the copy; the kernel orders them with explicit
// s_waitcnt vmcnt and barriers.  M0 carries the LDS address; nothing else in the
// kernels that use it touches M0.
__device__ __forceinline__ void copy_to_lds(const void* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds) : "memory");
}


// Copies of a K-contiguous tile for contract_pipe: 32-bit byte offsets of this lane's
// rows from a scalar base (the operand pointer plus the K tile's offset), so each copy
// is one global_load_lds_dwordx4 with a scalar base address.  The host guarantees
// that every offset of the operand fits in 32 bits.
// G > 0: the row group has at most G sub-axes, and a row's offset is formed in 32 bits
// (the same low 32 bits as the 64-bit form).
template <typename S, int ROWS, int NW, int SIDE, int G = 0>
struct PipeCopies {
  static constexpr int RPI = 64 / kChunks;  // rows per copy instruction
  static constexpr int NI = ROWS / RPI / NW;
  static_assert(NI >= 1 && ROWS % (RPI * NW) == 0, "tile shape");
  uint32_t off[NI];
  int region0;

  __device__ __forceinline__ void init(const ContractArgs& p, int wave, int lane, uint32_t row0, int64_t boff) {
    region0 = wave * NI;
    const GroupArgs& g = SIDE == 0 ? p.gm : p.gn;
    const uint32_t lim = (SIDE == 0 ? p.M : p.N) - 1;
    const uint32_t base = uint32_t(boff * int64_t(sizeof(S)));
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int row = (region0 + i) * RPI + lane / kChunks;
      const int chunk = swz(row, lane % kChunks);
      uint32_t r = row0 + row;
      r = r > lim ? lim : r;  // rows past the edge re-read the last row; never stored
      if constexpr (G > 0) off[i] = base + group_offset_d32<SIDE, G>(g, r, sizeof(S)) + uint32_t(chunk * 16);
      else off[i] = uint32_t((boff + group_offset<SIDE>(g, r)) * int64_t(sizeof(S))) + uint32_t(chunk * 16);
    }
  }
  // copy i of this wave's share of the tile at `base` into the LDS tile at byte address `lds`
  __device__ __forceinline__ void issue_one(int i, const void* base, uint32_t lds) const {
    copy_to_lds(base, off[i], lds + uint32_t((region0 + i) * 1024));
  }
};

// The same copy through a buffer resource (es_contract_halo): lane l moves 16 bytes
// from `voff` + `soff` bytes into the range of `srd` (base, stride 0, range, 32-bit data
// format), or zeros when the offset lies past the range (the buffer's range check;
// nothing is read).  The callers keep voff below 2^31 for a row that is read and at or
// above it (with voff + soff below 2^32) for one that is not, and every range is below
// 2^31, so the check gives the same answer whether it counts soff or not.
__device__ __forceinline__ void buffer_copy_to_lds(const u32x4& srd, uint32_t voff, uint32_t soff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %3\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(srd), "s"(soff),
               "s"(lds)
               : "memory");
}

// Copies of A for es_contract_halo: PipeCopies' K-contiguous copies, from the unpadded
// input through a buffer resource.  Tap k = (k_outer, k_inner) of a row at output
// position (o_outer, o_inner) reads input position o_s + dil_s * k_s - pad_s along each
// dim; each lane keeps, for each of its rows, a mask with bit k set when that position
// falls outside [0, extent_s) along some dim.  Such a copy's offset gets bit 31, past
// the buffer's range, and loads zeros.  The K tile's offset rides in the scalar offset.
// G > 0: M has at most G sub-axes (ContractArgs::gdims), walked by G - 1 divisions.
template <typename S, int ROWS, int NW, int G = 0>
struct PipeCopiesHalo {
  static constexpr int RPI = 64 / kChunks;  // rows per copy instruction
  static constexpr int NI = ROWS / RPI / NW;
  static_assert(NI >= 1 && ROWS % (RPI * NW) == 0, "tile shape");
  uint32_t off[NI];      // byte offset of the row's chunk at tap 0, before the shift
  uint32_t outside[NI];  // bit k: tap k reads outside the input
  int region0;

  __device__ __forceinline__ void init(const ContractArgs& p, int wave, int lane, uint32_t row0, int64_t boff) {
    region0 = wave * NI;
    const uint32_t lim = p.M - 1;
    uint32_t outer[NI], inner[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int row = (region0 + i) * RPI + lane / kChunks;
      const int chunk = swz(row, lane % kChunks);
      uint32_t r = row0 + row;
      r = r > lim ? lim : r;  // rows past the edge re-read the last row; never stored
      // one pass over M's sub-axes: the row's offset and its positions along the halo dims
      int64_t goff = boff;
      outer[i] = inner[i] = 0;
      if constexpr (G > 0) {
        // sub-axes G - 1 .. 1 by division (those past gm.n divide by 1), 0 the quotient left
#pragma unroll
        for (int d = G - 1; d >= 0; --d) {
          uint32_t rem = r;
          if (d > 0) r = p.gm.div[d].divmod(r, rem);
          goff += int64_t(rem) * p.gm.sa[d];
          outer[i] = d == p.halo_mlev[0] ? rem : outer[i];
          inner[i] = d == p.halo_mlev[1] ? rem : inner[i];
        }
      } else {
#pragma unroll
        for (int d = ES_MAX_AXES - 1; d >= 0; --d) {
          if (d < p.gm.n) {
            uint32_t rem;
            r = p.gm.div[d].divmod(r, rem);
            goff += int64_t(rem) * p.gm.sa[d];
            outer[i] = d == p.halo_mlev[0] ? rem : outer[i];
            inner[i] = d == p.halo_mlev[1] ? rem : inner[i];
          }
        }
      }
      off[i] = uint32_t(goff * int64_t(sizeof(S))) + uint32_t(chunk * 16);
      // one register for the offset (not a sum the copies would re-add)
      asm volatile("" : "+v"(off[i]));
    }
    // the inside taps of the inner dim, then of both: the inner mask once per inside
    // outer tap (positions below 0 wrap to large unsigned values)
    uint32_t in_inner[NI], inside[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) in_inner[i] = inside[i] = 0;
    for (int k = 0; k < p.halo_taps[1]; ++k) {
      const uint32_t t = uint32_t(k * p.halo_dil[1] - p.halo_pad[1]);
#pragma unroll
      for (int i = 0; i < NI; ++i) in_inner[i] |= uint32_t(inner[i] + t < p.halo_extent[1]) << k;
    }
    for (int k = 0; k < p.halo_taps[0]; ++k) {
      const uint32_t t = uint32_t(k * p.halo_dil[0] - p.halo_pad[0]);
      const int shift = k * p.halo_taps[1];
#pragma unroll
      for (int i = 0; i < NI; ++i) inside[i] |= outer[i] + t < p.halo_extent[0] ? in_inner[i] << shift : 0u;
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) outside[i] = ~inside[i];
  }
  // the vector offset of copy i for a K tile of tap `tap`.  The host keeps off[i] plus
  // any K tile's offset below 2^31 for every row: bit 31 is free for the outside flag,
  // and a flagged offset plus the K tile's offset stays below 2^32.
  __device__ __forceinline__ uint32_t voff(int i, uint32_t tap) const {
    return off[i] | (((outside[i] >> tap) & 1u) << 31);
  }
  // copy i, at vector offset `vo` (voff) and the K tile's offset `kbytes`, into the LDS
  // tile at byte address `lds`
  __device__ __forceinline__ void issue_one(int i, const u32x4& srd, uint32_t vo, uint32_t kbytes,
                                            uint32_t lds) const {
    buffer_copy_to_lds(srd, vo, kbytes, lds + uint32_t((region0 + i) * 1024));
  }
};

// Copies of a tile whose operand is contiguous along its rows (M for A, N for B),
// for contract_pipe.  The tile is stored as blocks of 64 rows: block b is 64 k-rows of
// 128 bytes (rows 64b .. 64b + 63 of one k each), 8 KB, and 16-byte chunk c (8
// consecutive rows) of k-row r sits at chunk position c ^ mn_swz(r).  One copy
// instruction fills 8 k-rows of one block; lane l fetches k-row l / 8 of them, chunk
// position l % 8, so each k-row is one whole 128-byte line of the operand (half lines,
// with blocks of 32 rows, took a K step about 200 cycles longer).  Row runs past the
// edge re-read the last 8 rows (the host guarantees that the row extent is a multiple
// of 8); they are never stored.
__device__ __forceinline__ int mn_swz(int r) { return (((r >> 1) & 1) << 1) | (((r >> 3) & 1) << 2); }

template <typename S, int ROWS, int NW, int SIDE, int G = 0>
struct PipeCopiesMN {
  static constexpr int NI = ROWS / 8 / NW;  // 1 KB copies of this wave per K tile
  static_assert(NI >= 1 && ROWS % (8 * NW) == 0 && ROWS % 64 == 0, "tile shape");
  uint32_t off[NI];
  int region0;

  __device__ __forceinline__ void init(const ContractArgs& p, int wave, int lane, uint32_t row0, int64_t boff) {
    region0 = wave * NI;
    const GroupArgs& g = SIDE == 0 ? p.gm : p.gn;
    const uint32_t last = (SIDE == 0 ? p.M : p.N) - 8;
    const int64_t kstride = SIDE == 0 ? p.ka_inner : p.kb_inner;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int q = region0 + i;  // block q / 8, k-rows 8 (q % 8) .. + 7
      const int kr = (q % 8) * 8 + lane / 8;
      const int chunk = (lane % 8) ^ mn_swz(kr);
      uint32_t r = row0 + uint32_t((q / 8) * 64 + chunk * 8);
      r = r > last ? last : r;
      off[i] = uint32_t((boff + group_offset_d<SIDE, G>(g, r) + int64_t(kr) * kstride) * int64_t(sizeof(S)));
    }
  }
  __device__ __forceinline__ void issue_one(int i, const void* base, uint32_t lds) const {
    copy_to_lds(base, off[i], lds + uint32_t((region0 + i) * 1024));
  }
};

// Fragment reads of contract_pipe: fragment i of a wave is 16 rows (its rows row0 + 16 i
// onwards) by 8 k (k = 32 ks + 8 (lane / 16) .. +7 of the K tile), lane l holding row
// l % 16: the operand layout of v_mfma_f32_16x16x32.  A K-contiguous tile gives each
// lane its 16 bytes in one read.
template <typename S, int LAYOUT>
struct PipeFrag {
  static constexpr int BK = kRowBytes / int(sizeof(S));
  static constexpr int READS = 1;  // LDS read instructions per fragment
  int ofs[2];                      // element offsets of substeps 0 and 1 in the side's tile

  __device__ __forceinline__ void init(int lane, int row0) {
    const int lrow = lane % 16;  // rows row0 + 16 i keep lrow's swizzle key
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) ofs[ks] = (row0 + lrow) * BK + swz(lrow, ks * 4 + lane / 16) * 8;
  }
  __device__ __forceinline__ uint4 read(const S* side, int i, int ks) const {
    return *reinterpret_cast<const uint4*>(side + ofs[ks] + i * 16 * BK);
  }
};

// An MN-contiguous tile (blocks of 64 rows, above) is read with gfx950's transposing
// LDS read ds_read_b64_tr_b16.  Within each 16 lanes, lane j names 4 consecutive
// 16-bit rows of k-row kb + j / 4 starting at row 4 (j % 4), and lane i receives
// element i % 4 of lane 4e + i / 4's four as its element e: lane i then holds k-rows
// kb .. kb + 3 of row i.  Two reads (kb and kb + 4) give one 8-deep fragment.  Each
// half-wave of a read touches 8 k-rows, 4 of each parity, 32 bytes each; k-rows of one
// parity share a 128-byte half of the 256-byte LDS line, and mn_swz gives the 4 of them
// distinct 32-byte chunk pairs (its bits 1 and 2 follow k-row bits 1 and 3), so a
// half-wave reads 64 distinct banks.
template <typename S>
struct PipeFrag<S, kMNContig> {
  static constexpr int READS = 2;
  int base[4];  // byte offsets in the side's tile of fragments with 16-row index i % 4 = 0..3

  __device__ __forceinline__ void init(int lane, int row0) {  // row0: a multiple of 64
    const int j = lane % 16, g = lane / 16, e = j / 4;
    const int t = ((e >> 1) & 1) | ((g & 1) << 1);  // mn_swz(k-row) / 2: the same for + 4, + 32
    const int b = (row0 / 64) * 8192 + (8 * g + e) * 128 + ((j % 4) >> 1) * 16 + (j & 1) * 8;
#pragma unroll
    for (int m = 0; m < 4; ++m) base[m] = b + 32 * (m ^ t);
  }
  __device__ __forceinline__ uint4 read(const S* side, int i, int ks) const {
    typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
    typedef __attribute__((address_space(3))) char lds_char;
    const lds_char* p = (const lds_char*)side + base[i & 3] + (i >> 2) * 8192 + ks * 4096;
    const u32x2 lo = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)p));
    const u32x2 hi = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(p + 512)));
    return make_uint4(lo[0], lo[1], hi[0], hi[1]);
  }
};

// ---- software-pipelined kernel: 256 x BN tiles (BN = 256 or 224), 16-bit types -------
// Four waves (2 x 2) each own 128 x BN/2 as 8 x BN/32 blocks of 16 x 16 on
// v_mfma_f32_16x16x32_{bf16,f16}; a 64-deep K tile is two substeps of 32 k.  Two LDS
// stages, filled by global_load_lds_dwordx4 copies issued a full K tile ahead.  With one
// wave per SIMD nothing hides a stall, so the schedule is explicit, in program order (the
// MFMAs are inline assembly, which the compiler's scheduling groups do not recognise):
//   substep 0: its MFMAs, with the fragment reads of substep 1 spread over the first
//              three quarters of them, so that they have landed by the barrier's LDS
//              wait (spread over all of them: about 1 % slower; issued all ahead of the
//              MFMAs: 2-5 % slower);
//   barrier:   K tile kt+1 has landed (own copies: vmcnt(0); everyone's: the barrier)
//              and nobody reads stage kt any more;
//   substep 1: its MFMAs, with the copies of K tile kt+2 into stage kt spread evenly
//              over them and the fragment reads of K tile kt+1's first substep over
//              their first three quarters (bunching them measured 24 % slower: the
//              copies and reads then queue on LDS).
// Blocks of 16 allow BN = 224 (waves of 128 x 112): an N extent of 7 x 256 = 1792 (one
// tensor-parallel rank's share of a 14336-wide weight) then cuts into 8 tiles instead of
// 7, and 16384 x 1792 into 512 tiles, two whole rounds of one tile per CU, where 256 x 256
// tiles leave a quarter of the CUs idle in the second.
// Lane l of a fragment read holds k = 8 * (l / 16) .. +7 of row l % 16 (one 16-byte LDS
// read); the first MFMA operand is the N-side fragment, so the accumulator holds C^T and
// lane l ends with 4 consecutive n (4 * (l / 16) + 0..3) of m = l % 16.
// MFMAs of contract_pipe as inline assembly with the accumulator tied to the result
// ("+a": read and written in place, in AGPRs).  The builtin is selected in a form
// whose result need not share the accumulator's registers, and with 56 accumulators
// per wave the register allocator then rotated them through the AGPRs with a copy per
// accumulator per K tile (measured 40 % slower than tied).  The compiler cannot see hazards across
// inline assembly, so the kernel avoids them by construction: nothing but these MFMAs
// writes the accumulators (the first MFMA of a tile takes the constant 0 as its
// accumulator, mma_first), the fragment operands come straight from LDS reads, and
// pipe_drain separates the last MFMA from the first VALU read of a result.
template <typename T>
struct PipeMma;

template <>
struct PipeMma<bf16_t> {
  static __device__ __forceinline__ void mma(f32x4& acc, const uint4& nfrag, const uint4& mfrag) {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0"
                 : "+a"(acc)
                 : "v"(__builtin_bit_cast(u32x4, nfrag)), "v"(__builtin_bit_cast(u32x4, mfrag)));
  }
  static __device__ __forceinline__ void mma_first(f32x4& acc, const uint4& nfrag, const uint4& mfrag) {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0"
                 : "=a"(acc)
                 : "v"(__builtin_bit_cast(u32x4, nfrag)), "v"(__builtin_bit_cast(u32x4, mfrag)));
  }
};

template <>
struct PipeMma<f16_t> {
  static __device__ __forceinline__ void mma(f32x4& acc, const uint4& nfrag, const uint4& mfrag) {
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0"
                 : "+a"(acc)
                 : "v"(__builtin_bit_cast(u32x4, nfrag)), "v"(__builtin_bit_cast(u32x4, mfrag)));
  }
  static __device__ __forceinline__ void mma_first(f32x4& acc, const uint4& nfrag, const uint4& mfrag) {
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, 0"
                 : "=a"(acc)
                 : "v"(__builtin_bit_cast(u32x4, nfrag)), "v"(__builtin_bit_cast(u32x4, mfrag)));
  }
};

// After the last MFMA of a tile: 32 wait states (more than any 16x16x32 result needs
// before a VALU read), then every accumulator passes through an empty statement that
// follows them, so no read of a result can be scheduled before the wait.
template <int FM, int FN>
__device__ __forceinline__ void pipe_drain(f32x4 (&acc)[FM][FN]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) asm volatile("" : "+a"(acc[i][j]));
}

// Epilogue of contract_pipe.  The tile is staged in the two (now free) LDS stages,
// wave row 0's rows in stage 0 and wave row 1's in stage 1, in as few passes as fit
// with the row / column offset tables beside them: one pass for 256 x 224 tiles, two of
// 128 rows for 256 x 256.  All four waves stage their accumulators, one barrier, then
// the whole work-group writes the rows out (16-byte streaming stores along n when n is
// the output's contiguous axis, element stores otherwise).  The caller has drained
// every copy into LDS and synchronised the work-group.
template <typename T, int BN, int FM, int FN, bool BIAS, int G = 0>
__device__ __forceinline__ void store_pipe(const ContractArgs& p, typename Traits<T>::S* lds0,
                                           typename Traits<T>::S* lds1, const f32x4 (&acc)[FM][FN], uint32_t m0,
                                           uint32_t n0, int64_t boff_c) {
  using S = typename Traits<T>::S;
  constexpr int BM = 256, WTN = BN / 2, VEC = 8, NT = 256;
  constexpr int SLD = BN + VEC;  // staging row pitch (elements)
  constexpr int STAGE_BYTES = (BM + BN) * kRowBytes;
  constexpr int TABLES = BM * 8;  // the larger table (rows)
  constexpr int P = (16 * FM) * SLD * int(sizeof(S)) + TABLES <= STAGE_BYTES ? 1 : 2;  // passes
  constexpr int BPP = FM / P;   // 16-row blocks per wave row per pass
  constexpr int RR = 16 * BPP;  // rows per stage per pass
  static_assert(FM % P == 0 && RR * SLD * int(sizeof(S)) + TABLES <= STAGE_BYTES, "epilogue fits the stages");
  int64_t* row_off = reinterpret_cast<int64_t*>(reinterpret_cast<char*>(lds0) + RR * SLD * int(sizeof(S)));
  int64_t* col_off = reinterpret_cast<int64_t*>(reinterpret_cast<char*>(lds1) + RR * SLD * int(sizeof(S)));
  const int tid = threadIdx.x;
  const int lane = tid % 64;
  const int wave = tid / 64;
  const int wm = wave / 2;
  const int wn = wave % 2;
  S* region = wm == 0 ? lds0 : lds1;
  S* C = static_cast<S*>(p.c);
  const KArgs kp = kernel_args();
  for (int r = tid; r < BM; r += NT) {
    const uint32_t m = m0 + r;
    row_off[r] = m < p.M ? boff_c + group_offset_kd<2, G>(&kp->gm, m) : -1;
  }
  for (int c = tid; c < BN; c += NT) {
    const uint32_t n = n0 + c;
    col_off[c] = n < p.N ? group_offset_kd<2, G>(&kp->gn, n) : -1;
  }
  // BIAS: the bias of this lane's columns (es_contract_bias), added before the one rounding
  f32x4 bv[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t n = n0 + wn * WTN + j * 16 + 4 * (lane / 16) + r;
      bv[j][r] = BIAS ? bias_at<T>(p, n) : 0.f;
    }
#pragma unroll
  for (int q = 0; q < P; ++q) {
#pragma unroll
    for (int ii = 0; ii < BPP; ++ii)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const f32x4 a = BIAS ? acc[q * BPP + ii][j] + bv[j] : acc[q * BPP + ii][j];
        *reinterpret_cast<uint2*>(region + (ii * 16 + lane % 16) * SLD + wn * WTN + j * 16 + 4 * (lane / 16)) =
            uint2{Traits<T>::pack2(a[0], a[1]), Traits<T>::pack2(a[2], a[3])};
      }
    lds_barrier();
    // staged row rr of stage h is tile row h * 128 + q * RR + rr
    if (p.vstore == 1) {
      constexpr int CV = BN / VEC;  // vectors per row
      for (int v = tid; v < 2 * RR * CV; v += NT) {
        const int h = v / (RR * CV);
        const int rem = v - h * (RR * CV);
        const int rr = rem / CV;
        const int cv = rem - rr * CV;
        const int64_t ro = row_off[h * 128 + q * RR + rr];
        const int64_t co = col_off[cv * VEC];
        // nontemporal: the output is not read again by this kernel, so it is not kept in L2
        if (ro >= 0 && co >= 0)
          __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>((h ? lds1 : lds0) + rr * SLD + cv * VEC),
                                      reinterpret_cast<u32x4*>(C + ro + co));
      }
    } else {
      for (int v = tid; v < 2 * RR * BN; v += NT) {
        const int h = v / (RR * BN);
        const int rem = v - h * (RR * BN);
        const int rr = rem / BN;
        const int cn = rem - rr * BN;
        const int64_t ro = row_off[h * 128 + q * RR + rr];
        const int64_t co = col_off[cn];
        if (ro >= 0 && co >= 0) C[ro + co] = (h ? lds1 : lds0)[rr * SLD + cn];
      }
    }
    if (q + 1 < P) lds_barrier();
  }
}

// The epilogue of contract_pipe when n is the output's contiguous axis (vstore == 1)
// and the output is 16-bit: a kernel instantiation of its own (EPI == 1), since with
// every epilogue in one function the register allocator spilled 36 accumulator
// registers of the 256-wide tile to scratch, about 6 us per launch.  One pass: each
// accumulator is rounded (after the bias) and written to the two freed stages, wave row
// 0's 128 rows in stage 0 and wave row 1's in stage 1, as rows of 512 bytes (a 224-wide
// tile leaves 4 chunks of each unused) whose 16-byte chunk c sits at c ^ (r % 32): the
// 8-byte writes of 16 rows and the 16-byte reads along a row then spread over all banks
// (the padded rows of store_pipe, 464 bytes apart, measured 2.0-2.3 us of tables and
// staging per 224-wide tile on C4); one barrier; the whole work-group writes the tile
// with 16-byte streaming stores.  The offset tables (`tables`, BM + 256 entries) have
// 4 KB of LDS of their own; PRE: the caller formed them before its K loop (as here), so
// the epilogue reads no kernel argument (after 100 us of K loop such a scalar load misses
// every cache, and a few of them in a row measured 1-2 us per tile).  BIAS_LDS: the
// bias, as floats, sits in LDS after the tables (contract_pipe's kBiasLds).  C is the
// output.
template <typename T, int BN, int FM, int FN, bool BIAS, int G = 0, bool PRE = false, bool BIAS_LDS = false>
__device__ __forceinline__ void store_pipe_wide(const ContractArgs& p, typename Traits<T>::S* lds0,
                                                typename Traits<T>::S* lds1, const f32x4 (&acc)[FM][FN],
                                                uint32_t m0, uint32_t n0, int64_t boff_c, int64_t* tables,
                                                typename Traits<T>::S* C) {
  using S = typename Traits<T>::S;
  constexpr int BM = 256, WTN = BN / 2, NT = 256, VEC = 8;
  constexpr int SP = 256;       // staged row pitch (elements): 32 chunks
  constexpr int CH = BN / VEC;  // 16-byte chunks per row
  static_assert(FM * 16 == 128 && FN * 16 == WTN && BN <= SP, "256 x BN tiles of four 128 x BN/2 waves");
  int64_t* row_off = tables;
  int64_t* col_off = tables + BM;
  const int tid = threadIdx.x;
  const int lane = tid % 64;
  const int wave = tid / 64;
  const int wm = wave / 2;
  const int wn = wave % 2;
  // the bias loads go first, so their latency passes while the offset tables are formed
  // (BIAS_LDS: the caller put the tile's bias, as floats, in LDS after the tables)
  const float* bias_lds = reinterpret_cast<const float*>(tables + BM + 256);
  f32x4 bv[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int c = wn * WTN + j * 16 + 4 * (lane / 16) + r;
      bv[j][r] = !BIAS ? 0.f : (BIAS_LDS ? bias_lds[c] : bias_at<T>(p, n0 + c));
    }
  if constexpr (!PRE) {
    const KArgs kp = kernel_args();
    const uint32_t m = m0 + tid, n = n0 + tid;
    row_off[tid] = m < p.M ? boff_c + group_offset_kd<2, G>(&kp->gm, m) : -1;
    if (tid < BN) col_off[tid] = n < p.N ? group_offset_kd<2, G>(&kp->gn, n) : -1;
  }
  S* region = wm == 0 ? lds0 : lds1;
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int col = wn * WTN + j * 16 + 4 * (lane / 16);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int r = i * 16 + lane % 16;  // row within the stage
      const f32x4 a = BIAS ? acc[i][j] + bv[j] : acc[i][j];
      *reinterpret_cast<uint2*>(region + r * SP + ((col / VEC) ^ (r % 32)) * VEC + col % VEC) =
          uint2{Traits<T>::pack2(a[0], a[1]), Traits<T>::pack2(a[2], a[3])};
    }
  }
  lds_barrier();
  for (int v = tid; v < BM * CH; v += NT) {
    const int row = v / CH;
    const int cv = v % CH;
    const int rr = row % 128;
    const int64_t ro = row_off[row];
    const int64_t co = col_off[cv * VEC];
    // nontemporal: the output is not read again by this kernel, so it is not kept in L2
    if (ro >= 0 && co >= 0)
      __builtin_nontemporal_store(
          *reinterpret_cast<const u32x4*>((row < 128 ? lds0 : lds1) + rr * SP + (cv ^ (rr % 32)) * VEC),
          reinterpret_cast<u32x4*>(C + ro + co));
  }
}

// The epilogue of contract_pipe when the output is contiguous along the tile's rows
// (the innermost M sub-axis, ContractArgs::vstore == 2): the tile is staged transposed,
// [column n][row m], and written with 16-byte streaming stores along m.  A lane's four
// consecutive-n values go to four staged rows (four 2-byte LDS writes).  Passes and
// tables as in store_pipe, sized for the transposed stage.
template <typename T, int BN, int FM, int FN, bool BIAS, int G = 0>
__device__ __forceinline__ void store_pipe_t(const ContractArgs& p, typename Traits<T>::S* lds0,
                                             typename Traits<T>::S* lds1, const f32x4 (&acc)[FM][FN], uint32_t m0,
                                             uint32_t n0, int64_t boff_c) {
  using S = typename Traits<T>::S;
  constexpr int BM = 256, WTN = BN / 2, VEC = 8, NT = 256;
  constexpr int STAGE_BYTES = (BM + BN) * kRowBytes;
  constexpr int TABLES = BM * 8;
  constexpr int P = BN * (16 * FM + VEC) * int(sizeof(S)) + TABLES <= STAGE_BYTES ? 1 : 2;  // passes
  constexpr int BPP = FM / P;        // 16-row blocks per wave row per pass
  constexpr int RR = 16 * BPP;       // rows per stage per pass
  constexpr int SLM = RR + VEC;      // staging pitch (elements) of a column
  constexpr int MV = RR / VEC;       // 16-byte vectors per staged column
  static_assert(FM % P == 0 && BN * SLM * int(sizeof(S)) + TABLES <= STAGE_BYTES, "epilogue fits the stages");
  int64_t* row_off = reinterpret_cast<int64_t*>(reinterpret_cast<char*>(lds0) + BN * SLM * int(sizeof(S)));
  int64_t* col_off = reinterpret_cast<int64_t*>(reinterpret_cast<char*>(lds1) + BN * SLM * int(sizeof(S)));
  const int tid = threadIdx.x;
  const int lane = tid % 64;
  const int wave = tid / 64;
  const int wm = wave / 2;
  const int wn = wave % 2;
  S* region = wm == 0 ? lds0 : lds1;
  S* C = static_cast<S*>(p.c);
  const KArgs kp = kernel_args();
  for (int r = tid; r < BM; r += NT) {
    const uint32_t m = m0 + r;
    row_off[r] = m < p.M ? boff_c + group_offset_kd<2, G>(&kp->gm, m) : -1;
  }
  for (int c = tid; c < BN; c += NT) {
    const uint32_t n = n0 + c;
    col_off[c] = n < p.N ? group_offset_kd<2, G>(&kp->gn, n) : -1;
  }
  f32x4 bv[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t n = n0 + wn * WTN + j * 16 + 4 * (lane / 16) + r;
      bv[j][r] = BIAS ? bias_at<T>(p, n) : 0.f;
    }
#pragma unroll
  for (int q = 0; q < P; ++q) {
#pragma unroll
    for (int ii = 0; ii < BPP; ++ii)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const f32x4 a = BIAS ? acc[q * BPP + ii][j] + bv[j] : acc[q * BPP + ii][j];
        const uint32_t lo = Traits<T>::pack2(a[0], a[1]), hi = Traits<T>::pack2(a[2], a[3]);
        S* col = region + (wn * WTN + j * 16 + 4 * (lane / 16)) * SLM + ii * 16 + lane % 16;
        col[0] = S(lo);
        col[SLM] = S(lo >> 16);
        col[2 * SLM] = S(hi);
        col[3 * SLM] = S(hi >> 16);
      }
    lds_barrier();
    // staged column c of stage h holds tile rows h * 128 + q * RR + (0 .. RR) of column c
    for (int v = tid; v < 2 * BN * MV; v += NT) {
      const int h = v / (BN * MV);
      const int rem = v - h * (BN * MV);
      const int c = rem / MV;
      const int mv = rem - c * MV;
      const int64_t ro = row_off[h * 128 + q * RR + mv * VEC];
      const int64_t co = col_off[c];
      if (ro >= 0 && co >= 0)
        __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>((h ? lds1 : lds0) + c * SLM + mv * VEC),
                                    reinterpret_cast<u32x4*>(C + ro + co));
    }
    if (q + 1 < P) lds_barrier();
  }
}

// The epilogue of contract_pipe for an fp32 output (ContractArgs::out_f32): as
// store_tile_f32, for the 16 x 16 blocks of v_mfma_f32_16x16x32, whose acc[i][j] holds
// columns wn*WTN + j*16 + 4*(lane/16) + 0..3 of tile row wm*128 + i*16 + lane%16.  The
// offset tables sit at the start of the two (free) stages.
template <typename T, int BN, int FM, int FN, bool BIAS, bool VEC_ONLY = false, int G = 0>
__device__ __forceinline__ void store_pipe_f32(const ContractArgs& p, typename Traits<T>::S* lds0,
                                               typename Traits<T>::S* lds1, const f32x4 (&acc)[FM][FN],
                                               uint32_t m0, uint32_t n0, int64_t boff_c) {
  using S = typename Traits<T>::S;
  constexpr int BM = 256, WTM = 128, WTN = BN / 2, NT = 256;
  int64_t* row_off = reinterpret_cast<int64_t*>(lds0);
  int64_t* col_off = reinterpret_cast<int64_t*>(lds1);
  const int tid = threadIdx.x;
  const int lane = tid % 64;
  const int wave = tid / 64;
  const int wm = wave / 2;
  const int wn = wave % 2;
  float* C = static_cast<float*>(p.c);
  const KArgs kp = kernel_args();
  for (int r = tid; r < BM; r += NT) {
    const uint32_t m = m0 + r;
    row_off[r] = m < p.M ? boff_c + group_offset_kd<2, G>(&kp->gm, m) : -1;
  }
  for (int c = tid; c < BN; c += NT) {
    const uint32_t n = n0 + c;
    col_off[c] = n < p.N ? group_offset_kd<2, G>(&kp->gn, n) : -1;
  }
  lds_barrier();
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int64_t ro = row_off[wm * WTM + i * 16 + lane % 16];
    if (ro < 0) continue;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int c = wn * WTN + j * 16 + 4 * (lane / 16);
      f32x4 v = acc[i][j];
      if constexpr (BIAS) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t n = n0 + c + r;
          v[r] += bias_at<T>(p, n);
        }
      }
      if (VEC_ONLY || p.vstore == 1) {
        const int64_t co = col_off[c];
        if (co >= 0) *reinterpret_cast<f32x4*>(C + ro + co) = v;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t co = col_off[c + r];
          if (co >= 0) C[ro + co] = v[r];
        }
      }
    }
  }
}

// EPI: 0 = the epilogue chosen at run time (fp32, transposed, vector or element stores);
// 1 = vector stores along n and a 16-bit output (store_pipe_wide; a 224-wide tile's
// stages are then sized for its 512-byte staged rows);
// 2 = 256-wide tiles with an fp32 output, vector stores along n and no bias (split-K
// partials, store_pipe_f32).  Each of
// 1 and 2 is an instantiation of its own: with every epilogue in one function the
// 256-wide kernel spilled accumulators to scratch.
// HALO: A is read by PipeCopiesHalo (es_contract_halo), both operands K-contiguous.
// G > 0: the batch, M and N groups have at most G sub-axes each (ContractArgs::gdims; 1
// or 2, or with a halo 3, for the batch, height and width of a 2-D convolution): every
// row, column and batch offset is an unrolled walk of G - 1 divisions, so the set-up in
// front of the first copies is a few hundred instructions instead of a walk over
// ES_MAX_AXES sub-axes per row with a scalar load per step (the halo kernel of einconv's
// benchmark: 2,605 instructions, 87 waits for scalar loads, 7-10 us per work-group).
// X3 (no halo): one operand, the deep one (1: A, 2: B), gets three LDS stages and the
// other two, so the deep operand's copies start a substep earlier: in step kt its tile
// kt+2 goes, during the first substep, into the stage step kt-1 finished reading, and the
// other operand's tile kt+2 goes, during the second, into the stage the first substep
// finished reading.  The barrier waits for all but the deep operand's last batch (loads
// complete in order).  On a cold cache a copy from HBM takes longer than one K step;
// with one tile of lead the loop waited for it.  Splitting the copies over both
// substeps also keeps the second substep from running long: with all of them in it
// (the deep tile then kt+3), C4 took 193.0 us flushed against 189.9.  The deep operand is the one with more rows of its own to stream
// (A for 16384 x 1792, B for 2048 x 8192).  224-wide tiles: A, with both operands
// K-contiguous.  256-wide tiles (EPI 1): the ring takes all 160 KB of LDS, so the
// epilogue's offset tables wait in registers through the K loop and go to LDS after it.
template <typename T, int BN, int L, int LA, int LB, int EPI = 0, bool HALO = false, int G = 0, int X3 = 0>
__global__ __launch_bounds__(256, 1) void contract_pipe(const ContractArgs p) {
  using S = typename Traits<T>::S;
  constexpr int BM = 256, WM = 2, WN = 2;
  constexpr int VEC = 8;
  constexpr int BK = kRowBytes / int(sizeof(S));  // 64
  constexpr int NS = BK / 32;                      // substeps of 32 k
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 16, FN = WTN / 16;
  constexpr int STAGE = (BM + BN) * BK;
  constexpr int MMAS = FM * FN;  // per substep
  // a substep's FM + FN fragment reads ride on its first three quarters of MFMAs, one per
  // MFMA at most: read r goes out with MFMA q when read_slot(q) <= r < read_slot(q + 1)
  constexpr int RQ = MMAS * 3 / 4;
  static_assert(RQ >= FM + FN, "one fragment read per MFMA at most");
  auto read_slot = [](int q) { return q >= RQ ? FM + FN : (q * (FM + FN)) / RQ; };
  using CopyA = std::conditional_t<
      HALO, PipeCopiesHalo<S, BM, WM * WN, G>,
      std::conditional_t<LA == kMNContig, PipeCopiesMN<S, BM, WM * WN, 0, G>, PipeCopies<S, BM, WM * WN, 0, G>>>;
  static_assert(!HALO || (LA == kKContig && LB == kKContig), "the halo reads K-contiguous operands");
  static_assert(X3 == 0 || (!HALO && (BN == 224 ? X3 == 1 && LA == kKContig && LB == kKContig : EPI == 1 && G > 0)),
                "three stages: A of 224-wide K-contiguous tiles, or either of 256-wide tiles with EPI 1 and bounded groups");
  using CopyB =
      std::conditional_t<LB == kMNContig, PipeCopiesMN<S, BN, WM * WN, 1, G>, PipeCopies<S, BN, WM * WN, 1, G>>;
  using FragA = PipeFrag<S, LA>;
  using FragB = PipeFrag<S, LB>;
  constexpr int NREAD = FM * FragA::READS + FN * FragB::READS;  // LDS read instructions per substep
  constexpr int NCOPY = CopyA::NI + CopyB::NI;  // copies per wave per K tile
  static_assert(sizeof(S) == 2 && NS == 2, "16-bit element types, two substeps per K tile");
  static_assert(WTN % 16 == 0 && FM % 2 == 0, "tile shape");
  static_assert(NCOPY <= MMAS && NREAD <= MMAS, "last substep interleave");
  static_assert((LA == kKContig || WTM % 64 == 0) && (LB == kKContig || WTN % 64 == 0), "MN blocks of 64 rows");

  // EPI 1 stages 128 rows of 256 elements per stage (more than a 224-wide tile's K stage)
  constexpr int STAGE_ALLOC = EPI == 1 && STAGE < 128 * 256 ? 128 * 256 : STAGE;
  // X3: one ring of the A stages then the B stages; the epilogue stages its two halves at
  // its start and 64 KB in
  constexpr int A_TILE = BM * BK, B_TILE = BN * BK;
  constexpr int NA = X3 == 1 ? 3 : 2, NB = X3 == 2 ? 3 : 2;  // stages of A and of B
  constexpr int RING = NA * A_TILE + NB * B_TILE;
  static_assert(X3 == 0 || RING >= 2 * 128 * 256, "the epilogue's two halves fit the ring");
  constexpr int STAGES_BYTES = (X3 ? RING : 2 * STAGE_ALLOC) * int(sizeof(S));
  // the one-pass epilogue's row and column offset tables: LDS of their own when that fits
  // beside the stages, else (a 256-wide ring) the ring's bytes past the staged halves
  // ... and, EPI 1, the tile's bias as floats after them
  constexpr int TABLE_BYTES = (BM + 256) * int(sizeof(int64_t)) + (EPI == 1 ? 256 * int(sizeof(float)) : 0);
  constexpr bool kOwnTables = EPI == 1 && STAGES_BYTES + TABLE_BYTES <= kLdsBytes;
  static_assert(EPI != 1 || kOwnTables || 2 * 128 * 256 * int(sizeof(S)) + TABLE_BYTES <= STAGES_BYTES, "tables fit");
  __shared__ __attribute__((aligned(1024))) char lds_raw[STAGES_BYTES + (kOwnTables ? TABLE_BYTES : 0)];
  S* const lds0 = reinterpret_cast<S*>(lds_raw);
  S* const lds1 = lds0 + (X3 ? 128 * 256 : STAGE_ALLOC);
  int64_t* const ep_tables =
      reinterpret_cast<int64_t*>(lds_raw + (kOwnTables ? STAGES_BYTES : 2 * 128 * 256 * int(sizeof(S))));
  // EPI 1 with bounded groups forms those tables in the prologue (while the first copies
  // are in flight: into LDS, or with no LDS of their own into registers, one row and one
  // column offset per thread, stored after the K loop) and keeps the output pointer and
  // the bias test in scalar registers through the K loop: the epilogue then reads no
  // kernel argument
  constexpr bool kPreTables = EPI == 1 && G > 0;
  // the bias of the tile's columns, loaded ahead of the first copies (so the prologue's
  // wait covers it) and put in LDS beside the tables: the epilogue then reads it from LDS
  // instead of from memory after the K loop (the tables' own LDS only)
  constexpr bool kBiasLds = kPreTables && kOwnTables;
  float* const ep_bias = reinterpret_cast<float*>(ep_tables + BM + 256);
  int64_t reg_row = -1, reg_col = -1;

  const int tid = threadIdx.x;
  const int lane = tid % 64;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
  const int wm = wave / WN;
  const int wn = wave % WN;

  uint32_t bidx, tm, tn;
  tile_of(p, blockIdx.x, bidx, tm, tn);
  const uint32_t m0 = tm * BM;
  const uint32_t n0 = tn * BN;
  const int64_t boff_a = group_offset_d<0, G>(p.gb, bidx);
  const int64_t boff_b = group_offset_d<1, G>(p.gb, bidx);
  const int64_t boff_c = group_offset_d<2, G>(p.gb, bidx);

  CopyA ca;
  CopyB cb;
  ca.init(p, wave, lane, m0, boff_a);
  cb.init(p, wave, lane, n0, boff_b);

  f32x4 acc[FM][FN];  // first written by mma_first

  FragA fa;
  FragB fb;
  fa.init(lane, wm * WTM);
  fb.init(lane, wn * WTN);

  uint4 af[2][FM], bf[2][FN];
  auto frags = [&](const S* stage, int buf, int ks) {
#pragma unroll
    for (int i = 0; i < FM; ++i) af[buf][i] = fa.read(stage, i, ks);
#pragma unroll
    for (int j = 0; j < FN; ++j) bf[buf][j] = fb.read(stage + BM * BK, j, ks);
  };

  const uint32_t nk = (p.K + BK - 1) / BK;  // >= 1: an empty K takes the generic kernel
  PipeWalk<L> w;
  w.start(p);
  const uint32_t lds0_addr = lds_address(lds0);
  const uint32_t lds1_addr = lds_address(lds1);
  // the halo's buffer resource over A
  u32x4 srd = {0u, 0u, 0u, 0u};
  if constexpr (HALO) srd = u32x4{p.halo_srd[0], p.halo_srd[1], p.halo_srd[2], p.halo_srd[3]};
  // HALO: the copies' vector offsets for the K tile at w, formed ahead of the copies
  // (in a step, among substep 0's MFMAs, which have slack; a dependent shift and or in
  // front of each copy in substep 1 took it about 370 cycles longer)
  uint32_t hvoff[HALO ? CopyA::NI : 1];
  // the tap of the K tile at w (K tile t = tap * ctiles + channel tile)
  auto halo_tap = [&]() -> uint32_t {
    if constexpr (HALO) return p.halo_ctiles.div(w.t);
    else return 0u;
  };
  auto halo_voffs = [&]() {
    if constexpr (HALO) {
      const uint32_t tap = halo_tap();
#pragma unroll
      for (int i = 0; i < CopyA::NI; ++i) hvoff[i] = ca.voff(i, tap);
    }
  };
  auto copy = [&](int q, uint32_t stage) {
    if (q < CopyA::NI) {
      if constexpr (HALO) {
        ca.issue_one(q, srd, hvoff[q], uint32_t(w.oa) * uint32_t(sizeof(S)), stage);
      } else {
        ca.issue_one(q, static_cast<const S*>(p.a) + w.oa, stage);
      }
    } else {
      cb.issue_one(q - CopyA::NI, static_cast<const S*>(p.b) + w.ob, stage + uint32_t(BM * BK * sizeof(S)));
    }
  };
  // kBiasLds: the bias loads go out ahead of the first copies; their values reach LDS
  // right after the wait for K tile 0 (the compiler's own wait for them then also covers
  // K tile 1's copies, which were issued right after tile 0's)
  float reg_bias = 0.f;
  auto bias_load = [&]() {
    if constexpr (kBiasLds) {
      if (p.bias != nullptr && tid < BN) reg_bias = bias_at<T>(p, n0 + tid);
    }
  };
  auto bias_store = [&]() {
    if constexpr (kBiasLds) {
      if (tid < BN) ep_bias[tid] = reg_bias;
    }
  };
  // the epilogue's output pointer and bias test (see kPreTables)
  S* out_c;
  uint32_t has_bias;
  auto pre_tables = [&]() {
    out_c = static_cast<S*>(p.c);
    has_bias = p.bias != nullptr ? 1u : 0u;
    if constexpr (kPreTables) {
      const uint32_t m = m0 + tid, n = n0 + tid;
      reg_row = m < p.M ? boff_c + group_offset_d<2, G>(p.gm, m) : -1;
      reg_col = tid < BN && n < p.N ? group_offset_d<2, G>(p.gn, n) : -1;
      if constexpr (kOwnTables) {
        ep_tables[tid] = reg_row;
        if (tid < BN) ep_tables[BM + tid] = reg_col;
      }
      const uint64_t cbits = reinterpret_cast<uint64_t>(out_c);
      uint32_t clo = __builtin_amdgcn_readfirstlane(uint32_t(cbits));
      uint32_t chi = __builtin_amdgcn_readfirstlane(uint32_t(cbits >> 32));
      has_bias = __builtin_amdgcn_readfirstlane(has_bias);
      asm volatile("" : "+s"(clo), "+s"(chi), "+s"(has_bias));
      out_c = reinterpret_cast<S*>((uint64_t(chi) << 32) | clo);
    }
  };
  if constexpr (X3 != 0) {
    // the ring's stages: A stage i at lds0 + i * A_TILE, B stage j after the NA A stages
    const uint32_t ring_addr = lds_address(lds0);
    auto a_stage = [&](uint32_t i) { return lds0 + i * A_TILE; };
    auto b_stage = [&](uint32_t j) { return lds0 + NA * A_TILE + j * B_TILE; };
    PipeWalk<L> wd;  // the deep operand's next K tile to copy
    wd.start(p);
    // both operands copy the same K tile in a step (the deep one in substep 0, the other
    // in substep 1): the other operand's offset is the walk's
    auto other_off = [&]() { return X3 == 1 ? wd.ob : wd.oa; };
    constexpr int NI_D = X3 == 1 ? CopyA::NI : CopyB::NI;  // copies per K tile: deep operand
    constexpr int NI_O = NCOPY - NI_D;                      // ... and the other
    // copy q of the deep (other) operand's next K tile into its stage `st`
    auto copy_d = [&](int q, uint32_t st) {
      if constexpr (X3 == 1)
        ca.issue_one(q, static_cast<const S*>(p.a) + wd.oa, ring_addr + st * uint32_t(A_TILE * sizeof(S)));
      else
        cb.issue_one(q, static_cast<const S*>(p.b) + wd.ob,
                     ring_addr + uint32_t((NA * A_TILE + st * B_TILE) * sizeof(S)));
    };
    auto copy_o = [&](int q, uint32_t st, int64_t off) {
      if constexpr (X3 == 1)
        cb.issue_one(q, static_cast<const S*>(p.b) + off, ring_addr + uint32_t((NA * A_TILE + st * B_TILE) * sizeof(S)));
      else
        ca.issue_one(q, static_cast<const S*>(p.a) + off, ring_addr + st * uint32_t(A_TILE * sizeof(S)));
    };
    // K tiles 0 and 1 of both operands, in the order the barriers count them: D0 O0 | O1 D1
    bias_load();
#pragma unroll
    for (int q = 0; q < NI_D; ++q) copy_d(q, 0);
#pragma unroll
    for (int q = 0; q < NI_O; ++q) copy_o(q, 0, other_off());
    wd.advance(nk);
#pragma unroll
    for (int q = 0; q < NI_O; ++q) copy_o(q, 1, other_off());
#pragma unroll
    for (int q = 0; q < NI_D; ++q) copy_d(q, 1);
    wd.advance(nk);
    pre_tables();
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NCOPY) : "memory");  // K tile 0 landed
    bias_store();
    __syncthreads();
#pragma unroll
    for (int i = 0; i < FM; ++i) af[0][i] = fa.read(a_stage(0), i, 0);
#pragma unroll
    for (int j = 0; j < FN; ++j) bf[0][j] = fb.read(b_stage(0), j, 0);
    // step kt: the deep operand's stage d_cur = kt % 3, the other's o_cur = kt % 2
    auto step3 = [&](uint32_t d_cur, uint32_t d_nxt, uint32_t o_cur, uint32_t o_nxt, auto first) {
      const S* as = a_stage(X3 == 1 ? d_cur : o_cur);
      const S* bs = b_stage(X3 == 1 ? o_cur : d_cur);
      const uint32_t d_far = 3u - d_cur - d_nxt;  // the deep stage step kt - 1 finished with
#pragma unroll
      for (int q = 0; q < MMAS; ++q) {
        if constexpr (decltype(first)::value) PipeMma<T>::mma_first(acc[q / FN][q % FN], bf[0][q % FN], af[0][q / FN]);
        else PipeMma<T>::mma(acc[q / FN][q % FN], bf[0][q % FN], af[0][q / FN]);
        {  // the deep operand's tile kt + 2 into it
          const int c0 = (q * NI_D) / MMAS, c1 = ((q + 1) * NI_D) / MMAS;
          if (c0 != c1) copy_d(c0, d_far);
        }
        const int r0 = read_slot(q), r1 = read_slot(q + 1);
        if (r0 != r1) {
          if (r0 < FM) af[1][r0] = fa.read(as, r0, 1);
          else bf[1][r0 - FM] = fb.read(bs, r0 - FM, 1);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      // K tile kt+1 of both operands landed (the copies still allowed in flight are the
      // deep operand's last batch, tile kt+2); every read of the current stages done
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NI_D) : "memory");
      __syncthreads();
      const S* an = a_stage(X3 == 1 ? d_nxt : o_nxt);
      const S* bn = b_stage(X3 == 1 ? o_nxt : d_nxt);
#pragma unroll
      for (int q = 0; q < MMAS; ++q) {
        PipeMma<T>::mma(acc[q / FN][q % FN], bf[1][q % FN], af[1][q / FN]);
        // the other operand's tile kt + 2 into o_cur
        const int c0 = (q * NI_O) / MMAS, c1 = ((q + 1) * NI_O) / MMAS;
        if (c0 != c1) copy_o(c0, o_cur, other_off());
        const int r0 = read_slot(q), r1 = read_slot(q + 1);
        if (r0 != r1) {
          if (r0 < FM) af[0][r0] = fa.read(an, r0, 0);
          else bf[0][r0 - FM] = fb.read(bn, r0 - FM, 0);
        }
      }
      wd.advance(nk);
      __builtin_amdgcn_sched_barrier(0);
    };
    using First = std::integral_constant<bool, true>;
    using Next = std::integral_constant<bool, false>;
    // the stages repeat every 6 K tiles
    step3(0, 1, 0, 1, First{});
    uint32_t kt = 1;
    for (; kt + 5 < nk; kt += 6) {
      step3(1, 2, 1, 0, Next{});
      step3(2, 0, 0, 1, Next{});
      step3(0, 1, 1, 0, Next{});
      step3(1, 2, 0, 1, Next{});
      step3(2, 0, 1, 0, Next{});
      step3(0, 1, 0, 1, Next{});
    }
    for (; kt < nk; ++kt) step3(kt % 3, (kt + 1) % 3, kt % 2, (kt + 1) % 2, Next{});
  } else {
  bias_load();
  halo_voffs();
#pragma unroll
  for (int q = 0; q < NCOPY; ++q) copy(q, lds0_addr);
  w.advance(nk);
  halo_voffs();
#pragma unroll
  for (int q = 0; q < NCOPY; ++q) copy(q, lds1_addr);
  w.advance(nk);
  pre_tables();
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NCOPY) : "memory");  // K tile 0 of this wave landed
  bias_store();
  __syncthreads();
  frags(lds0, 0, 0);

  // first: the tile's first K tile, whose first MFMAs start the accumulators from 0
  auto step = [&](S* stage_cur, const S* stage_nxt, uint32_t cur_addr, auto first) {
    // substep 0: its MFMAs interleaved with the fragment reads of substep 1 (HALO: and
    // with the offsets of the copies substep 1 issues, one per MFMA from the first)
    const uint32_t tap = halo_tap();
#pragma unroll
    for (int q = 0; q < MMAS; ++q) {
      if constexpr (decltype(first)::value) PipeMma<T>::mma_first(acc[q / FN][q % FN], bf[0][q % FN], af[0][q / FN]);
      else PipeMma<T>::mma(acc[q / FN][q % FN], bf[0][q % FN], af[0][q / FN]);
      if constexpr (HALO) {
        if (q < CopyA::NI) hvoff[q] = ca.voff(q, tap);
      }
      const int r0 = read_slot(q), r1 = read_slot(q + 1);
      if (r0 != r1) {
        if (r0 < FM) af[1][r0] = fa.read(stage_cur, r0, 1);
        else bf[1][r0 - FM] = fb.read(stage_cur + BM * BK, r0 - FM, 1);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    // K tile kt+1 complete for everyone; every read of stage kt done
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    // substep 1: its MFMAs, the copies of K tile kt+2 into this stage and the first
    // fragments of K tile kt+1, interleaved in program order
#pragma unroll
    for (int q = 0; q < MMAS; ++q) {
      PipeMma<T>::mma(acc[q / FN][q % FN], bf[1][q % FN], af[1][q / FN]);
      // copies spread evenly over the substep, fragment reads over read_slot's window
      const int c0 = (q * NCOPY) / MMAS, c1 = ((q + 1) * NCOPY) / MMAS;
      if (c0 != c1) copy(c0, cur_addr);
      const int r0 = read_slot(q), r1 = read_slot(q + 1);
      if (r0 != r1) {
        if (r0 < FM) af[0][r0] = fa.read(stage_nxt, r0, 0);
        else bf[0][r0 - FM] = fb.read(stage_nxt + BM * BK, r0 - FM, 0);
      }
    }
    w.advance(nk);
    __builtin_amdgcn_sched_barrier(0);
  };
  using First = std::integral_constant<bool, true>;
  using Next = std::integral_constant<bool, false>;
  step(lds0, lds1, lds0_addr, First{});
  uint32_t kt = 1;
  for (; kt + 1 < nk; kt += 2) {
    step(lds1, lds0, lds1_addr, Next{});
    step(lds0, lds1, lds0_addr, Next{});
  }
  if (kt < nk) step(lds1, lds0, lds1_addr, Next{});
  }
  pipe_drain(acc);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if constexpr (EPI == 1) {
    if constexpr (kPreTables && !kOwnTables) {
      ep_tables[tid] = reg_row;  // the ring is free: every wave passed the barrier above
      if (tid < BN) ep_tables[BM + tid] = reg_col;
    }
    if (has_bias)
      store_pipe_wide<T, BN, FM, FN, true, G, kPreTables, kBiasLds>(p, lds0, lds1, acc, m0, n0, boff_c, ep_tables,
                                                                    out_c);
    else
      store_pipe_wide<T, BN, FM, FN, false, G, kPreTables>(p, lds0, lds1, acc, m0, n0, boff_c, ep_tables, out_c);
    return;
  }
  if constexpr (EPI == 2) {  // fp32 output with vector stores and no bias (split-K partials)
    store_pipe_f32<T, BN, FM, FN, false, true, G>(p, lds0, lds1, acc, m0, n0, boff_c);
    return;
  }
  if (p.out_f32) {
    if (p.bias != nullptr) store_pipe_f32<T, BN, FM, FN, true, false, G>(p, lds0, lds1, acc, m0, n0, boff_c);
    else store_pipe_f32<T, BN, FM, FN, false, false, G>(p, lds0, lds1, acc, m0, n0, boff_c);
  } else if (p.vstore == 2) {
    if (p.bias != nullptr) store_pipe_t<T, BN, FM, FN, true, G>(p, lds0, lds1, acc, m0, n0, boff_c);
    else store_pipe_t<T, BN, FM, FN, false, G>(p, lds0, lds1, acc, m0, n0, boff_c);
  } else {
    if (p.bias != nullptr) store_pipe<T, BN, FM, FN, true, G>(p, lds0, lds1, acc, m0, n0, boff_c);
    else store_pipe<T, BN, FM, FN, false, G>(p, lds0, lds1, acc, m0, n0, boff_c);
  }
}

// ---- contract_f32_deep: fp32 64 x 64 tiles, four LDS stages --------------------------
// For small fp32 contractions (one 64 x 64 tile per CU) the MFMA work per 32-deep K tile
// is only 1,024 cycles per SIMD, shorter than a load from L2 or HBM.  Here every operand
// is copied global -> LDS by LDS-DMA in its own layout (no register transposes) into one
// of six stages.  A barrier step covers three K tiles: after its barrier the next step's
// three tiles are copied into the stages the previous step used, and its own three are
// computed.  Eight waves: two per 32 x 32 block (one per SIMD pair slot), splitting each
// K tile's four 8-k groups, their partial sums added in the epilogue.  The copies are
// inline assembly (copy_to_lds_v): issued through the builtin, they made the compiler
// wait for all of them, the next step's included, before the step's first LDS read.
// What bounds the loop is the copies' issue: with 1 KB per instruction the CU moves
// about 10 bytes per cycle, and a wave that issues its six copies behind the others'
// waits up to ~2,600 cycles per step for them to be accepted (in-kernel timestamps).
//   K-major tile (operand K-contiguous): 64 rows of 128 bytes, chunks swizzled (swz);
//     a lane's fragment is one 16-byte read of 4 consecutive k (lanes 32-63: k + 4).
//   N-major tile (operand contiguous along its rows): 32 k-rows of 64 floats (256 bytes);
//     a lane's fragment is 4 single-float reads of its row at k, k + 1, k + 2, k + 3.
// Both operands give lane l the same k assignment, so every product is formed once.
template <int LAYOUT, int SIDE, int NW>
struct DeepCopies {
  static constexpr int NI = 8 / NW;  // 1 KB copy instructions per wave per K tile (8 KB tile)
  static_assert(NI >= 1 && NI * NW == 8, "an 8 KB tile in whole 1 KB copies per wave");
  const float* src[NI];
  int region0;
  int64_t kstride;  // N-major: stride of the innermost K sub-axis

  __device__ __forceinline__ void init(const ContractArgs& p, int wave, int lane, uint32_t row0, int64_t boff) {
    region0 = wave * NI;
    const GroupArgs& g = SIDE == 0 ? p.gm : p.gn;
    const float* base = static_cast<const float*>(SIDE == 0 ? p.a : p.b);
    kstride = SIDE == 0 ? p.ka_inner : p.kb_inner;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      if constexpr (LAYOUT == kKContig) {
        // one instruction: 8 rows x 128 bytes; lane l -> row l / 8, stored chunk l % 8
        const uint32_t lim = (SIDE == 0 ? p.M : p.N) - 1;
        const int row = (region0 + i) * 8 + lane / kChunks;
        uint32_t r = row0 + row;
        r = r > lim ? lim : r;  // rows past the edge re-read the last row; never stored
        src[i] = base + boff + group_offset<SIDE>(g, r) + swz(row, lane % kChunks) * 4;
      } else {
        // one instruction: 4 k-rows x 256 bytes; lane l -> k-row l / 16, rows 4 (l % 16) .. + 3
        const uint32_t lim = (SIDE == 0 ? p.M : p.N) - 4;  // last whole group of 4 (extent % 4 == 0)
        const int krow = (region0 + i) * 4 + lane / 16;
        uint32_t r = row0 + 4 * (lane % 16);
        r = r > lim ? lim : r;
        src[i] = base + boff + group_offset<SIDE>(g, r) + int64_t(krow) * kstride;
      }
    }
  }
  __device__ __forceinline__ void issue(float* dst, int64_t koff) const {
#pragma unroll
    for (int i = 0; i < NI; ++i) copy_to_lds_v(src[i] + koff, lds_address(dst + (region0 + i) * 256));
  }
  // this lane's fragment for k group g (8 k) of the wave's 32-row block at `row`
  __device__ __forceinline__ uint4 frag(const float* tile, int lane, int row, int g) const {
    if constexpr (LAYOUT == kKContig) {
      return *reinterpret_cast<const uint4*>(tile + row * 32 + swz(row, g * 2 + lane / 32) * 4);
    } else {
      const float* col = tile + (g * 8 + 4 * (lane / 32)) * 64 + row;
      return uint4{__float_as_uint(col[0]), __float_as_uint(col[64]), __float_as_uint(col[128]),
                   __float_as_uint(col[192])};
    }
  }
};

// Epilogue of contract_f32_deep with KS = 2: the second wave of each block hands its
// partial sums to the first through LDS (fixed order: first + second), the first stages
// the block (with the bias) as [row][n], and all threads write the tile out (16-byte
// stores along n when n is the output's contiguous axis).  Every thread passes every
// barrier.
template <bool BIAS>
__device__ __forceinline__ void store_deep_pair(const ContractArgs& p, float* lds, f32x16 (&acc)[1][1], uint32_t m0,
                                                uint32_t n0, int64_t boff_c) {
  constexpr int BM = 64, BN = 64, NT = 512, SLD = BN + 4;
  const int tid = threadIdx.x;
  const int lane = tid % 64;
  const int wave = tid / 64;
  const int blk = wave % 4, kpart = wave / 4;
  const int wm = blk / 2, wn = blk % 2;
  float* red = lds;                    // 4 blocks x 16 x 64 floats
  float* stage = lds + 4 * 16 * 64;    // 64 x SLD floats
  int64_t* row_off = reinterpret_cast<int64_t*>(stage + BM * SLD);
  int64_t* col_off = row_off + BM;
  const KArgs kp = kernel_args();
  if (tid < BM) {
    const uint32_t m = m0 + tid;
    row_off[tid] = m < p.M ? boff_c + group_offset_k<2>(&kp->gm, m) : -1;
  } else if (tid < BM + BN) {
    const uint32_t n = n0 + tid - BM;
    col_off[tid - BM] = n < p.N ? group_offset_k<2>(&kp->gn, n) : -1;
  }
  if (kpart == 1) {
#pragma unroll
    for (int r = 0; r < 16; ++r) red[(blk * 16 + r) * 64 + lane] = acc[0][0][r];
  }
  __syncthreads();
  if (kpart == 0) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int col = wn * 32 + 8 * g + 4 * (lane / 32);
      f32x4 v;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        v[r] = acc[0][0][4 * g + r] + red[(blk * 16 + 4 * g + r) * 64 + lane];
        if constexpr (BIAS) {
          const uint32_t n = n0 + col + r;
          v[r] += bias_at<float>(p, n);
        }
      }
      *reinterpret_cast<f32x4*>(stage + (wm * 32 + lane % 32) * SLD + col) = v;
    }
  }
  __syncthreads();
  float* C = static_cast<float*>(p.c);
  if (p.vstore == 1) {
    for (int v = tid; v < BM * BN / 4; v += NT) {
      const int row = v / (BN / 4), c4 = v % (BN / 4);
      const int64_t ro = row_off[row], co = col_off[4 * c4];
      if (ro >= 0 && co >= 0)
        __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(stage + row * SLD + 4 * c4),
                                    reinterpret_cast<u32x4*>(C + ro + co));
    }
  } else {
    for (int v = tid; v < BM * BN; v += NT) {
      const int row = v / BN, col = v % BN;
      const int64_t ro = row_off[row], co = col_off[col];
      if (ro >= 0 && co >= 0) C[ro + co] = stage[row * SLD + col];
    }
  }
}

// KS waves per 32 x 32 block (KS = 2: two waves per SIMD, splitting each K tile's four
// 8-k groups between them)
// s_waitcnt vmcnt(n) for a run-time n in [0, 15]
__device__ __forceinline__ void wait_vmcnt(uint32_t n) {
  switch (n) {
#define ES_VMCNT_CASE(N) \
  case N: asm volatile("s_waitcnt vmcnt(" #N ")" ::: "memory"); break;
    ES_VMCNT_CASE(0) ES_VMCNT_CASE(1) ES_VMCNT_CASE(2) ES_VMCNT_CASE(3) ES_VMCNT_CASE(4) ES_VMCNT_CASE(5)
    ES_VMCNT_CASE(6) ES_VMCNT_CASE(7) ES_VMCNT_CASE(8) ES_VMCNT_CASE(9) ES_VMCNT_CASE(10) ES_VMCNT_CASE(11)
    ES_VMCNT_CASE(12) ES_VMCNT_CASE(13) ES_VMCNT_CASE(14)
#undef ES_VMCNT_CASE
    default: asm volatile("s_waitcnt vmcnt(15)" ::: "memory"); break;
  }
}

template <int LA, int LB, int KS>
__global__ __launch_bounds__(256 * KS, 1) void contract_f32_deep(const ContractArgs p) {
  constexpr int BM = 64, BN = 64, BK = 32, NST = 6, TPB = 3;  // LDS stages, K tiles per barrier
  static_assert(NST >= 2 * TPB, "a barrier step's tiles and the next step's copies in separate stages");
  constexpr int NW = 4 * KS;
  constexpr int TILE = BM * BK;  // floats per operand tile (BM == BN)
  constexpr int STAGE = 2 * TILE;
  constexpr int NCOPY = 2 * DeepCopies<LA, 0, NW>::NI;  // copy instructions per thread per K tile
  __shared__ __attribute__((aligned(1024))) float lds[NST * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid % 64;
  const int wave = tid / 64;
  const int blk = wave % 4, kpart = wave / 4;
  const int wm = blk / 2, wn = blk % 2;
  uint32_t bidx, tm, tn;
  tile_of(p, blockIdx.x, bidx, tm, tn);
  const uint32_t m0 = tm * BM, n0 = tn * BN;
  const int64_t boff_a = group_offset<0>(p.gb, bidx);
  const int64_t boff_b = group_offset<1>(p.gb, bidx);
  const int64_t boff_c = group_offset<2>(p.gb, bidx);

  DeepCopies<LA, 0, NW> ca;
  DeepCopies<LB, 1, NW> cb;
  ca.init(p, wave, lane, m0, boff_a);
  cb.init(p, wave, lane, n0, boff_b);

  f32x16 acc[1][1];
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[0][0][r] = 0.f;

  const uint32_t nk = p.K / BK;  // the layouts require whole 32-deep K tiles
  KWalk<kKLevels> kw;
  kw.start(p);
  auto issue = [&](uint32_t t) {
    float* st = lds + (t % NST) * STAGE;
    ca.issue(st, kw.off_a);
    cb.issue(st + TILE, kw.off_b);
    kw.advance();
  };
#pragma unroll
  for (uint32_t t = 0; t < NST - TPB; ++t)
    if (t < nk) issue(t);

  const int arow = wm * 32 + lane % 32;
  const int brow = wn * 32 + lane % 32;
  constexpr int NG = BK / 8 / KS;  // 8-k groups per wave per K tile
  for (uint32_t kt = 0; kt < nk; kt += TPB) {
    // tiles kt .. kt + TPB - 1 landed: the copies still allowed in flight are those of
    // the later tiles issued so far (up to tile kt + NST - TPB - 1)
    static_assert((NST - 2 * TPB) * NCOPY <= 15, "vmcnt immediates");
    const int64_t later = min(int64_t(NST - 2 * TPB), int64_t(nk) - int64_t(kt) - TPB);
    wait_vmcnt(uint32_t(later > 0 ? later : 0) * NCOPY);
    __syncthreads();  // every wave's copies of these tiles landed; every read of the previous step's done
#pragma unroll
    for (int u = 0; u < TPB; ++u)  // into the stages the previous step's tiles used
      if (kt + NST - TPB + u < nk) issue(kt + NST - TPB + u);
#pragma unroll
    for (int u = 0; u < TPB; ++u) {
      if (kt + u >= nk) break;
      const float* As = lds + ((kt + u) % NST) * STAGE;
      const float* Bs = As + TILE;
      uint4 af[2], bf[2];
      af[0] = ca.frag(As, lane, arow, kpart);
      bf[0] = cb.frag(Bs, lane, brow, kpart);
#pragma unroll
      for (int q = 0; q < NG; ++q) {
        if (q + 1 < NG) {
          af[(q + 1) & 1] = ca.frag(As, lane, arow, (q + 1) * KS + kpart);
          bf[(q + 1) & 1] = cb.frag(Bs, lane, brow, (q + 1) * KS + kpart);
        }
        Traits<float>::mma(acc[0][0], bf[q & 1], af[q & 1]);
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if constexpr (KS == 1) {
    static_assert(epilogue_bytes<float, BM, BN, 2>() <= int(sizeof(lds)), "epilogue must fit in LDS");
    if (p.bias != nullptr) store_tile<float, BM, BN, 2, 2, 1, 1, true>(p, lds, acc, m0, n0, boff_c);
    else store_tile<float, BM, BN, 2, 2, 1, 1, false>(p, lds, acc, m0, n0, boff_c);
  } else {
    static_assert((4 * 16 * 64 + 64 * 68) * 4 + 128 * 8 <= int(sizeof(lds)), "epilogue must fit in LDS");
    if (p.bias != nullptr) store_deep_pair<true>(p, lds, acc, m0, n0, boff_c);
    else store_deep_pair<false>(p, lds, acc, m0, n0, boff_c);
  }
}

// ---- contract_f32_pipe: fp32 64 x 64 tiles on four waves, contract_pipe's schedule --
// One 64 x 64 tile per work-group (C1: 256 tiles, one per CU), four waves of 32 x 32,
// each 2 x 2 blocks of v_mfma_f32_16x16x4_f32: four accumulators, so consecutive MFMAs
// never wait on each other's results.  A 32-deep K tile is two substeps of 16 k.  As in
// contract_pipe, substep 0's MFMAs carry the fragment reads of substep 1; one barrier
// (K tile kt+1 landed, every read of stage kt done); substep 1's MFMAs carry the copies
// of K tile kt + NST into the stage just read and the fragment reads of K tile kt+1's
// substep 0.  NST stages of 16 KB, filled by LDS-DMA in each operand's own layout:
//   A (K-contiguous), and B when K-contiguous: 64 rows of 128 bytes, chunk c of row r
//     at c ^ ((r / 2) % 8) (swz); a fragment (4 consecutive k of one row) is one
//     16-byte read;
//   B when N-contiguous: 32 k-rows of 64 floats, 16-byte chunk c of k-row r at
//     c ^ (4 ((r / 4) % 4)); a fragment is 4 single-float reads, and the 4 k-rows a
//     read touches (4 apart) put their 16 lanes on distinct banks.
// Lane l of every fragment holds k = 16 ks + 4 (l / 16) + 0..3 for A and B alike, so
// every product is formed once.  The MFMA's first operand is B's, so the accumulator
// holds C^T: lane l ends with 4 consecutive n of one m, one 16-byte store.
// With one wave per SIMD nothing hides a stall, hence the explicit interleave: the
// simpler schedule (registers ring of loads, one write into LDS and one barrier per K
// tile, then all of the tile's MFMAs) measured 30.5 us on C1 against 29.7 for
// contract_f32_deep, 28.7 with its loads removed.
// Bounded groups only (G sub-axes per group, ContractArgs::gdims) and at most two K
// levels; the host guarantees whole 32-deep K tiles and (N-contiguous B) rows in
// groups of 4.
template <int LAYOUT, int SIDE, int G>
struct F32PipeCopies {  // an 8 KB operand tile: two 1 KB copies per wave
  static constexpr int NI = 2;
  const float* src[NI];
  int region0;
  __device__ __forceinline__ void init(const ContractArgs& p, int wave, int lane, uint32_t row0, int64_t boff) {
    region0 = wave * NI;
    const GroupArgs& g = SIDE == 0 ? p.gm : p.gn;
    const float* base = static_cast<const float*>(SIDE == 0 ? p.a : p.b);
    const int64_t kstride = SIDE == 0 ? p.ka_inner : p.kb_inner;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int q = region0 + i;
      if constexpr (LAYOUT == kKContig) {
        // 8 rows of 128 bytes: lane l -> row 8 q + l / 8, stored chunk l % 8
        const uint32_t lim = (SIDE == 0 ? p.M : p.N) - 1;
        const int row = q * 8 + lane / kChunks;
        uint32_t r = row0 + row;
        r = r > lim ? lim : r;  // rows past the edge re-read the last row; never stored
        src[i] = base + boff + group_offset_d<SIDE, G>(g, r) + swz(row, lane % kChunks) * 4;
      } else {
        // 4 k-rows of 256 bytes: lane l -> k-row 4 q + l / 16 at chunk position l % 16,
        // which holds chunk (l % 16) ^ (4 (q % 4)) of the k-row
        const uint32_t lim = (SIDE == 0 ? p.M : p.N) - 4;  // the last whole group of 4
        const int krow = q * 4 + lane / 16;
        const int chunk = (lane % 16) ^ (4 * (q & 3));
        uint32_t r = row0 + 4 * chunk;
        r = r > lim ? lim : r;
        src[i] = base + boff + group_offset_d<SIDE, G>(g, r) + int64_t(krow) * kstride;
      }
    }
  }
  __device__ __forceinline__ void issue(int i, float* dst, int64_t koff) const {
    copy_to_lds_v(src[i] + koff, lds_address(dst + (region0 + i) * 256));
  }
};

// v_mfma_f32_16x16x4_f32 as inline assembly with the accumulator tied (see PipeMma)
__device__ __forceinline__ void f32_mma(f32x4& acc, float n, float m) {
  asm volatile("v_mfma_f32_16x16x4_f32 %0, %1, %2, %0" : "+a"(acc) : "v"(n), "v"(m));
}
__device__ __forceinline__ void f32_mma_first(f32x4& acc, float n, float m) {
  asm volatile("v_mfma_f32_16x16x4_f32 %0, %1, %2, 0" : "=a"(acc) : "v"(n), "v"(m));
}

template <int LB, int L, int G, int NST = 3>
__global__ __launch_bounds__(256, 1) void contract_f32_pipe(const ContractArgs p) {
  static_assert(G > 0 && NST >= 3, "bounded groups; a stage being read, one landing, one in flight");
  constexpr int TILE = 64 * 32, STAGE = 2 * TILE;  // floats: A's tile, then B's
  constexpr int NCOPY = 4;                          // copies per wave per K tile
  __shared__ __attribute__((aligned(1024))) float lds[NST * STAGE];
  const int tid = threadIdx.x, lane = tid % 64;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
  const int wm = wave / 2, wn = wave % 2;
  uint32_t bidx, tm, tn;
  tile_of(p, blockIdx.x, bidx, tm, tn);
  const uint32_t m0 = tm * 64, n0 = tn * 64;
  const int64_t boff_a = group_offset_d<0, G>(p.gb, bidx);
  const int64_t boff_b = group_offset_d<1, G>(p.gb, bidx);
  const int64_t boff_c = group_offset_d<2, G>(p.gb, bidx);
  F32PipeCopies<kKContig, 0, G> ca;
  F32PipeCopies<LB, 1, G> cb;
  ca.init(p, wave, lane, m0, boff_a);
  cb.init(p, wave, lane, n0, boff_b);
  const uint32_t nk = p.K / 32;  // >= 1: an empty K takes the generic kernel
  PipeWalk<L> w;  // the next K tile to copy (stays on the last one)
  w.start(p);
  auto copy = [&](int q, float* st) {
    if (q < 2) ca.issue(q, st, w.oa);
    else cb.issue(q - 2, st + TILE, w.ob);
  };
  const int g = lane / 16;
  auto read_a = [&](const float* st, int i, int ks) -> f32x4 {
    const int row = wm * 32 + 16 * i + lane % 16;
    return *reinterpret_cast<const f32x4*>(st + row * 32 + swz(row, 4 * ks + g) * 4);
  };
  auto read_b = [&](const float* st, int j, int ks) -> f32x4 {
    if constexpr (LB == kKContig) {
      const int row = wn * 32 + 16 * j + lane % 16;
      return *reinterpret_cast<const f32x4*>(st + TILE + row * 32 + swz(row, 4 * ks + g) * 4);
    } else {
      const int n = wn * 32 + 16 * j + lane % 16;
      const float* b = st + TILE + (16 * ks + 4 * g) * 64 + ((n / 4) ^ (4 * g)) * 4 + n % 4;
      return f32x4{b[0], b[64], b[128], b[192]};
    }
  };
#pragma unroll
  for (int t = 0; t < NST; ++t) {
#pragma unroll
    for (int q = 0; q < NCOPY; ++q) copy(q, lds + t * STAGE);
    w.advance(nk);
  }
  f32x4 acc[2][2];  // first written by f32_mma_first
  f32x4 af[2][2], bf[2][2];
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NST - 1) * NCOPY) : "memory");  // K tile 0 landed
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 2; ++i) af[0][i] = read_a(lds, i, 0);
#pragma unroll
  for (int j = 0; j < 2; ++j) bf[0][j] = read_b(lds, j, 0);
  // MFMA q of a substep: k-step s = q / 4, block (i, j) = ((q / 2) % 2, q % 2)
  auto step = [&](uint32_t kt, auto first) {
    float* cur = lds + (kt % NST) * STAGE;
    const float* nxt = lds + ((kt + 1) % NST) * STAGE;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int s = q / 4, i = (q / 2) % 2, j = q % 2;
      if (decltype(first)::value && s == 0) f32_mma_first(acc[i][j], bf[0][j][s], af[0][i][s]);
      else f32_mma(acc[i][j], bf[0][j][s], af[0][i][s]);
      if (q % 4 == 1) {  // substep 1's fragments: a0, a1, b0, b1
        const int r = q / 4;
        if (r < 2) af[1][r] = read_a(cur, r, 1);
        else bf[1][r - 2] = read_b(cur, r - 2, 1);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NST - 2) * NCOPY) : "memory");  // K tile kt+1 landed
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int s = q / 4, i = (q / 2) % 2, j = q % 2;
      f32_mma(acc[i][j], bf[1][j][s], af[1][i][s]);
      if (q % 4 == 0) copy(q / 4, cur);  // K tile kt + NST into this stage
      if (q % 4 == 2) {                   // K tile kt+1's substep 0 fragments
        const int r = q / 4;
        if (r < 2) af[0][r] = read_a(nxt, r, 0);
        else bf[0][r - 2] = read_b(nxt, r - 2, 0);
      }
    }
    w.advance(nk);
    __builtin_amdgcn_sched_barrier(0);
  };
  step(0u, std::integral_constant<bool, true>{});
  for (uint32_t kt = 1; kt < nk; ++kt) step(kt, std::integral_constant<bool, false>{});
  pipe_drain(acc);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  // lane: acc[i][j] = C[m = wm*32 + 16 i + lane%16][n = wn*32 + 16 j + 4 (lane/16) + 0..3]
  float* C = static_cast<float*>(p.c);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t m = m0 + wm * 32 + 16 * i + lane % 16;
    if (m >= p.M) continue;
    const int64_t ro = boff_c + group_offset_d<2, G>(p.gm, m);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t n = n0 + wn * 32 + 16 * j + 4 * g;
      if (n >= p.N) continue;
      f32x4 v = acc[i][j];
      if (p.bias != nullptr) {
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] += bias_at<float>(p, n + r);
      }
      if (p.vstore == 1) {  // n .. n + 3 contiguous and inside N (N's innermost extent % 4 == 0)
        *reinterpret_cast<f32x4*>(C + ro + group_offset_d<2, G>(p.gn, n)) = v;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n + r < p.N) C[ro + group_offset_d<2, G>(p.gn, n + r)] = v[r];
      }
    }
  }
}

template <int LB, int L, int G>
void launch_f32_pipe(const ContractArgs& p, hipStream_t s) {
  contract_f32_pipe<LB, L, G><<<p.total_tiles, 256, 0, s>>>(p);
}

template <typename T>
int launch_f32_deep(const ContractArgs& p, int la, int lb, hipStream_t s) {
  if constexpr (std::is_same_v<T, float>) {
    constexpr int KS = 2, NT = 256 * KS;
    // contract_f32_pipe: A K-contiguous, bounded groups, at most two K levels
    if (la == kKContig && (lb == kKContig || lb == kMNContig) && p.gdims > 0 && p.gdims <= 2 && p.klevels <= 2) {
      const bool l1 = p.klevels == 1, g1 = p.gdims == 1;
      if (lb == kKContig) {
        if (l1) g1 ? launch_f32_pipe<kKContig, 1, 1>(p, s) : launch_f32_pipe<kKContig, 1, 2>(p, s);
        else g1 ? launch_f32_pipe<kKContig, 2, 1>(p, s) : launch_f32_pipe<kKContig, 2, 2>(p, s);
      } else {
        if (l1) g1 ? launch_f32_pipe<kMNContig, 1, 1>(p, s) : launch_f32_pipe<kMNContig, 1, 2>(p, s);
        else g1 ? launch_f32_pipe<kMNContig, 2, 1>(p, s) : launch_f32_pipe<kMNContig, 2, 2>(p, s);
      }
      set_kernel("contract_f32_pipe_64x64");
      return check_launch("es_contract");
    }
    if (la == kKContig && lb == kKContig) contract_f32_deep<kKContig, kKContig, KS><<<p.total_tiles, NT, 0, s>>>(p);
    else if (la == kKContig) contract_f32_deep<kKContig, kMNContig, KS><<<p.total_tiles, NT, 0, s>>>(p);
    else if (lb == kKContig) contract_f32_deep<kMNContig, kKContig, KS><<<p.total_tiles, NT, 0, s>>>(p);
    else contract_f32_deep<kMNContig, kMNContig, KS><<<p.total_tiles, NT, 0, s>>>(p);
    set_kernel("contract_f32_deep_64x64");
    return check_launch("es_contract");
  }
  return fail(ES_ERR_UNSUPPORTED, "es_contract: the deep fp32 kernel is for f32");
}

// ---- launcher ----------------------------------------------------------------------
// contract_pipe keeps as many K walk levels as the descriptor has (1, 2, or up to 4)
// es_contract_halo: the halo instantiations (both operands K-contiguous); a 256-wide
// tile with vector stores and a 16-bit output takes the one-pass epilogue
template <typename T, int BN, int EPI>
void launch_pipe_halo(const ContractArgs& p, hipStream_t s) {
  // bounded groups: up to three M sub-axes (batch, height, width)
  if (p.gdims > 0) {
    if (p.klevels <= 2) contract_pipe<T, BN, 2, kKContig, kKContig, EPI, true, 3><<<p.total_tiles, 256, 0, s>>>(p);
    else contract_pipe<T, BN, kKLevels, kKContig, kKContig, EPI, true, 3><<<p.total_tiles, 256, 0, s>>>(p);
    return;
  }
  if (p.klevels <= 2) contract_pipe<T, BN, 2, kKContig, kKContig, EPI, true><<<p.total_tiles, 256, 0, s>>>(p);
  else contract_pipe<T, BN, kKLevels, kKContig, kKContig, EPI, true><<<p.total_tiles, 256, 0, s>>>(p);
}

// The bounded-group instantiations (ContractArgs::gdims: at most G sub-axes per batch,
// M and N group; at most two K levels): the 224-wide tile, and the 256-wide tile's two
// one-pass epilogues (16-bit output with vector stores along n; fp32 split-K partials).
// Returns false when the call takes the generic instantiations instead.
template <typename T, int BN, int LA, int LB, int G>
bool launch_pipe_g(const ContractArgs& p, hipStream_t s) {
  const bool l1 = p.klevels == 1;
  if constexpr (BN == 256) {
    if (p.out_f32 && p.vstore == 1 && p.bias == nullptr) {
      if (l1) contract_pipe<T, BN, 1, LA, LB, 2, false, G><<<p.total_tiles, 256, 0, s>>>(p);
      else contract_pipe<T, BN, 2, LA, LB, 2, false, G><<<p.total_tiles, 256, 0, s>>>(p);
      return true;
    }
    if (p.vstore == 1 && !p.out_f32) {
      // the operand with more rows to stream takes a third LDS stage (X3 = 2: B, 1: A)
      if (p.N > p.M) {
        if (l1) contract_pipe<T, BN, 1, LA, LB, 1, false, G, 2><<<p.total_tiles, 256, 0, s>>>(p);
        else contract_pipe<T, BN, 2, LA, LB, 1, false, G, 2><<<p.total_tiles, 256, 0, s>>>(p);
      } else {
        if (l1) contract_pipe<T, BN, 1, LA, LB, 1, false, G, 1><<<p.total_tiles, 256, 0, s>>>(p);
        else contract_pipe<T, BN, 2, LA, LB, 1, false, G, 1><<<p.total_tiles, 256, 0, s>>>(p);
      }
      return true;
    }
    return false;
  } else {
    // 224-wide tiles with both operands K-contiguous give A a third LDS stage (X3 = 1)
    constexpr int X3 = LA == kKContig && LB == kKContig ? 1 : 0;
    if (p.vstore == 1 && !p.out_f32) {
      if (l1) contract_pipe<T, BN, 1, LA, LB, 1, false, G, X3><<<p.total_tiles, 256, 0, s>>>(p);
      else contract_pipe<T, BN, 2, LA, LB, 1, false, G, X3><<<p.total_tiles, 256, 0, s>>>(p);
    } else {
      if (l1) contract_pipe<T, BN, 1, LA, LB, 0, false, G, X3><<<p.total_tiles, 256, 0, s>>>(p);
      else contract_pipe<T, BN, 2, LA, LB, 0, false, G, X3><<<p.total_tiles, 256, 0, s>>>(p);
    }
    return true;
  }
}

// one sub-axis per group (the plain GEMM x[M, K] w[N, K], both operands K-contiguous)
// takes G = 1, where a row's offset is one multiply; up to two take G = 2
template <typename T, int BN, int LA, int LB>
bool launch_pipe_bounded(const ContractArgs& p, hipStream_t s) {
  if (p.gdims == 0 || p.gdims > 2 || p.klevels > 2) return false;
  if constexpr (LA == kKContig && LB == kKContig) {
    if (p.gdims == 1) return launch_pipe_g<T, BN, LA, LB, 1>(p, s);
  }
  return launch_pipe_g<T, BN, LA, LB, 2>(p, s);
}

template <typename T, int BN, int LA, int LB>
void launch_pipe(const ContractArgs& p, hipStream_t s) {
  if constexpr (LA == kKContig && LB == kKContig) {
    if (p.halo_n > 0) {
      if (p.vstore == 1 && !p.out_f32) launch_pipe_halo<T, BN, 1>(p, s);
      else launch_pipe_halo<T, BN, 0>(p, s);
      return;
    }
  }
  if (launch_pipe_bounded<T, BN, LA, LB>(p, s)) return;
  if constexpr (BN == 256) {
    if (p.out_f32 && p.vstore == 1 && p.bias == nullptr) {
      switch (p.klevels) {
        case 1: contract_pipe<T, BN, 1, LA, LB, 2><<<p.total_tiles, 256, 0, s>>>(p); break;
        case 2: contract_pipe<T, BN, 2, LA, LB, 2><<<p.total_tiles, 256, 0, s>>>(p); break;
        default: contract_pipe<T, BN, kKLevels, LA, LB, 2><<<p.total_tiles, 256, 0, s>>>(p); break;
      }
      return;
    }
  }
  if (p.vstore == 1 && !p.out_f32) {
    switch (p.klevels) {
      case 1: contract_pipe<T, BN, 1, LA, LB, 1><<<p.total_tiles, 256, 0, s>>>(p); break;
      case 2: contract_pipe<T, BN, 2, LA, LB, 1><<<p.total_tiles, 256, 0, s>>>(p); break;
      default: contract_pipe<T, BN, kKLevels, LA, LB, 1><<<p.total_tiles, 256, 0, s>>>(p); break;
    }
    return;
  }
  switch (p.klevels) {
    case 1: contract_pipe<T, BN, 1, LA, LB><<<p.total_tiles, 256, 0, s>>>(p); break;
    case 2: contract_pipe<T, BN, 2, LA, LB><<<p.total_tiles, 256, 0, s>>>(p); break;
    default: contract_pipe<T, BN, kKLevels, LA, LB><<<p.total_tiles, 256, 0, s>>>(p); break;
  }
}

template <typename T, int BM, int BN, int WM, int WN, int LA, int LB, int PF>
int launch_one(const ContractArgs& p, hipStream_t s, const char* name) {
  contract_kernel<T, BM, BN, WM, WN, LA, LB, PF><<<p.total_tiles, WM * WN * 64, 0, s>>>(p);
  set_kernel(name);
  return check_launch("es_contract");
}

template <typename T, int BM, int BN, int WM, int WN, int PF>
int launch_layouts(const ContractArgs& p, int la, int lb, hipStream_t s, const char* name) {
  if constexpr (BM == 256 && BN == 256 && sizeof(typename Traits<T>::S) == 2) {
    // contract_pipe when every offset fits 32 bits; an MN-contiguous operand is read
    // through transposing LDS reads (256-wide tiles only)
    if (p.off32) {
      if (la == kKContig && lb == kKContig) {
        if (p.pipe_bn == 224) {
          launch_pipe<T, 224, kKContig, kKContig>(p, s);
          set_kernel(p.halo_n > 0 ? "contract_pipe_256x224_halo" : "contract_pipe_256x224");
        } else {
          launch_pipe<T, 256, kKContig, kKContig>(p, s);
          set_kernel(p.halo_n > 0 ? "contract_pipe_256x256_halo" : "contract_pipe_256x256");
        }
      } else if (la == kKContig && lb == kMNContig) {
        launch_pipe<T, 256, kKContig, kMNContig>(p, s);
        set_kernel("contract_pipe_256x256_mn_b");
      } else if (la == kMNContig && lb == kKContig) {
        launch_pipe<T, 256, kMNContig, kKContig>(p, s);
        set_kernel("contract_pipe_256x256_mn_a");
      } else {
        launch_pipe<T, 256, kMNContig, kMNContig>(p, s);
        set_kernel("contract_pipe_256x256_mn_ab");
      }
      return check_launch("es_contract");
    }
  }
  if (la == kKContig && lb == kKContig) return launch_one<T, BM, BN, WM, WN, kKContig, kKContig, PF>(p, s, name);
  if (la == kKContig && lb == kMNContig) return launch_one<T, BM, BN, WM, WN, kKContig, kMNContig, PF>(p, s, name);
  if (la == kMNContig && lb == kKContig) return launch_one<T, BM, BN, WM, WN, kMNContig, kKContig, PF>(p, s, name);
  if (la == kMNContig && lb == kMNContig) return launch_one<T, BM, BN, WM, WN, kMNContig, kMNContig, 1>(p, s, name);
  return fail(ES_ERR_INVALID, "es_contract: layout combination has no fast kernel");
}

template <typename T>
int launch_typed(const ContractArgs& p, int config, int la, int lb, hipStream_t s) {
  if (la == kGeneric || lb == kGeneric)
    return launch_one<T, 64, 64, 2, 2, kGeneric, kGeneric, 1>(p, s, "contract_generic_64x64");
  // fp32 on 64 x 64 tiles: the four-stage kernel (both layouts by LDS-DMA)
  if (std::is_same_v<T, float> && config == 2 && p.klevels <= kKLevels) return launch_f32_deep<T>(p, la, lb, s);
  switch (config) {
    case 0: return launch_layouts<T, 256, 256, 2, 4, 1>(p, la, lb, s, "contract_256x256");
    case 1: return launch_layouts<T, 128, 128, 2, 2, 1>(p, la, lb, s, "contract_128x128");
    default: return launch_layouts<T, 64, 64, 2, 2, 1>(p, la, lb, s, "contract_64x64");
  }
}

}  // namespace contract
}  // namespace es
