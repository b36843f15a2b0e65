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
__device__ __forceinline__ void tile_of(const ContractArgs& p, uint32_t b, uint32_t& bidx, uint32_t& tm, uint32_t& tn) {
  if (p.total_tiles % 8 == 0) b = (b % 8) * (p.total_tiles / 8) + b / 8;
  const uint32_t per_batch = p.tiles_m * p.tiles_n;
  bidx = b / per_batch;
  const uint32_t rem = b - bidx * per_batch;
  const uint32_t gsize = p.tiles_m * p.group_n;  // tiles per group
  const uint32_t g = rem / gsize;
  const uint32_t r = rem - g * gsize;
  tm = r / p.group_n;
  tn = g * p.group_n + (r - tm * p.group_n);
}

// ---- tile loaders -------------------------------------------------------------
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

  // enqueue the copies of the K tile at element offset `koff` into LDS tile `dst`
  __device__ __forceinline__ void issue(S* dst, int64_t koff) const {
#pragma unroll
    for (int i = 0; i < NI; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(src[i] + koff), (lds_void*)(dst + (region0 + i) * 512 * 2 / sizeof(S)),
                                       16, 0, 0);
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
        bv[j][g][r] = BIAS && n < p.N ? Elem<T>::load(static_cast<const S*>(p.bias)[n]) : 0.f;
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
        __builtin_amdgcn_global_load_lds((const void*)(touch_src[q] + (on_a ? koff_a : koff_b)), (lds_void*)sink, 4, 0,
                                         0);
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
    la.issue(&lds[0], kw.off_a);
    lb.issue(&lds[BM * BK], kw.off_b);
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
      la.issue(nxt, kw.off_a);
      lb.issue(nxt + BM * BK, kw.off_b);
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

__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return uint32_t(uintptr_t((const lds_void*)p));
}

// Copies of a K-contiguous tile for contract_pipe: 32-bit byte offsets of this lane's
// rows from a scalar base (the operand pointer plus the K tile's offset), so each copy
// is one global_load_lds_dwordx4 with a scalar base address.  The host guarantees
// that every offset of the operand fits in 32 bits.
template <typename S, int ROWS, int NW, int SIDE>
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
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int row = (region0 + i) * RPI + lane / kChunks;
      const int chunk = swz(row, lane % kChunks);
      uint32_t r = row0 + row;
      r = r > lim ? lim : r;  // rows past the edge re-read the last row; never stored
      off[i] = uint32_t((boff + group_offset<SIDE>(g, r)) * int64_t(sizeof(S))) + uint32_t(chunk * 16);
    }
  }
  // copy i of this wave's share of the tile at `base` into the LDS tile at byte address `lds`
  __device__ __forceinline__ void issue_one(int i, const void* base, uint32_t lds) const {
    copy_to_lds(base, off[i], lds + uint32_t((region0 + i) * 1024));
  }
};

// Copies of a tile whose operand is contiguous along its rows (M for A, N for B),
// for contract_pipe.  The tile is stored as blocks of 32 rows: block b is 64 k-rows of
// 64 bytes (rows 32b .. 32b + 31 of one k each), 4 KB, and 16-byte chunk c (8
// consecutive rows) of k-row r sits at chunk position c ^ mn_swz(r).  One copy
// instruction fills 16 k-rows of one block; lane l fetches k-row l / 4 of them, chunk
// position l % 4.  Row runs past the edge re-read the last 8 rows (the host guarantees
// that the row extent is a multiple of 8); they are never stored.
__device__ __forceinline__ int mn_swz(int r) { return (((r >> 1) ^ (r >> 3)) & 1) << 1; }

template <typename S, int ROWS, int NW, int SIDE>
struct PipeCopiesMN {
  static constexpr int NI = ROWS / 8 / NW;  // 1 KB copies of this wave per K tile
  static_assert(NI >= 1 && ROWS % (8 * NW) == 0 && ROWS % 32 == 0, "tile shape");
  uint32_t off[NI];
  int region0;

  __device__ __forceinline__ void init(const ContractArgs& p, int wave, int lane, uint32_t row0, int64_t boff) {
    region0 = wave * NI;
    const GroupArgs& g = SIDE == 0 ? p.gm : p.gn;
    const uint32_t last = (SIDE == 0 ? p.M : p.N) - 8;
    const int64_t kstride = SIDE == 0 ? p.ka_inner : p.kb_inner;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int q = region0 + i;
      const int kr = (q % 4) * 16 + lane / 4;
      const int chunk = (lane % 4) ^ mn_swz(kr);
      uint32_t r = row0 + uint32_t((q / 4) * 32 + chunk * 8);
      r = r > last ? last : r;
      off[i] = uint32_t((boff + group_offset<SIDE>(g, r) + int64_t(kr) * kstride) * int64_t(sizeof(S)));
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

// An MN-contiguous tile (blocks of 32 rows, above) is read with gfx950's transposing
// LDS read ds_read_b64_tr_b16.  Within each 16 lanes, lane j names 4 consecutive
// 16-bit rows of k-row kb + j / 4 starting at row 4 (j % 4), and lane i receives
// element i % 4 of lane 4e + i / 4's four as its element e: lane i then holds k-rows
// kb .. kb + 3 of row i.  Two reads (kb and kb + 4) give one 8-deep fragment.  The 16
// k-rows one read touches split evenly over the 32-byte slots of a 256-byte LDS line
// through mn_swz: k-rows that share a slot pair ((r / 2) % 2 and r % 4 equal) differ
// in (r / 8) % 2 and take opposite halves.
template <typename S>
struct PipeFrag<S, kMNContig> {
  static constexpr int READS = 2;
  int base[2];  // byte offsets in the side's tile of fragments with even / odd 16-row index

  __device__ __forceinline__ void init(int lane, int row0) {  // row0: a multiple of 32
    const int j = lane % 16, g = lane / 16, e = j / 4;
    const int half = ((e >> 1) ^ g) & 1;  // mn_swz(8 g + e) / 2: also for k-rows + 4, + 32
    const int b = (row0 / 32) * 4096 + (8 * g + e) * 64 + ((j % 4) >> 1) * 16 + (j & 1) * 8;
    base[0] = b + 32 * half;
    base[1] = b + 32 * (1 - half);
  }
  __device__ __forceinline__ uint4 read(const S* side, int i, int ks) const {
    typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
    typedef __attribute__((address_space(3))) char lds_char;
    const lds_char* p = (const lds_char*)side + base[i & 1] + (i >> 1) * 4096 + ks * 2048;
    const u32x2 lo = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)p));
    const u32x2 hi = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(p + 256)));
    return make_uint4(lo[0], lo[1], hi[0], hi[1]);
  }
};

// ---- software-pipelined kernel: 256 x BN tiles (BN = 256 or 224), 16-bit types -------
// Four waves (2 x 2) each own 128 x BN/2 as 8 x BN/32 blocks of 16 x 16 on
// v_mfma_f32_16x16x32_{bf16,f16}; a 64-deep K tile is two substeps of 32 k.  Two LDS
// stages, filled by global_load_lds_dwordx4 copies issued a full K tile ahead.  With one
// wave per SIMD nothing hides a stall, so the schedule is explicit:
//   substep 0: its MFMAs, with the fragment reads of substep 1 spread evenly over them;
//   barrier:   K tile kt+1 has landed (own copies: vmcnt(0); everyone's: the barrier)
//              and nobody reads stage kt any more;
//   substep 1: its MFMAs, with the copies of K tile kt+2 into stage kt and the fragment
//              reads of K tile kt+1's first substep spread evenly over them (bunching
//              them measured 24 % slower: the copies and reads then queue on LDS).
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
template <typename T, int BN, int FM, int FN, bool BIAS>
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
    row_off[r] = m < p.M ? boff_c + group_offset_k<2>(&kp->gm, m) : -1;
  }
  for (int c = tid; c < BN; c += NT) {
    const uint32_t n = n0 + c;
    col_off[c] = n < p.N ? group_offset_k<2>(&kp->gn, n) : -1;
  }
  // BIAS: the bias of this lane's columns (es_contract_bias), added before the one rounding
  f32x4 bv[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t n = n0 + wn * WTN + j * 16 + 4 * (lane / 16) + r;
      bv[j][r] = BIAS && n < p.N ? Elem<T>::load(static_cast<const S*>(p.bias)[n]) : 0.f;
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

// The epilogue of contract_pipe when the output is contiguous along the tile's rows
// (the innermost M sub-axis, ContractArgs::vstore == 2): the tile is staged transposed,
// [column n][row m], and written with 16-byte streaming stores along m.  A lane's four
// consecutive-n values go to four staged rows (four 2-byte LDS writes).  Passes and
// tables as in store_pipe, sized for the transposed stage.
template <typename T, int BN, int FM, int FN, bool BIAS>
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
    row_off[r] = m < p.M ? boff_c + group_offset_k<2>(&kp->gm, m) : -1;
  }
  for (int c = tid; c < BN; c += NT) {
    const uint32_t n = n0 + c;
    col_off[c] = n < p.N ? group_offset_k<2>(&kp->gn, n) : -1;
  }
  f32x4 bv[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t n = n0 + wn * WTN + j * 16 + 4 * (lane / 16) + r;
      bv[j][r] = BIAS && n < p.N ? Elem<T>::load(static_cast<const S*>(p.bias)[n]) : 0.f;
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

template <typename T, int BN, int L, int LA, int LB>
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
  using CopyA = std::conditional_t<LA == kMNContig, PipeCopiesMN<S, BM, WM * WN, 0>, PipeCopies<S, BM, WM * WN, 0>>;
  using CopyB = std::conditional_t<LB == kMNContig, PipeCopiesMN<S, BN, WM * WN, 1>, PipeCopies<S, BN, WM * WN, 1>>;
  using FragA = PipeFrag<S, LA>;
  using FragB = PipeFrag<S, LB>;
  constexpr int NREAD = FM * FragA::READS + FN * FragB::READS;  // LDS read instructions per substep
  constexpr int NCOPY = CopyA::NI + CopyB::NI;  // copies per wave per K tile
  static_assert(sizeof(S) == 2 && NS == 2, "16-bit element types, two substeps per K tile");
  static_assert(WTN % 16 == 0 && FM % 2 == 0, "tile shape");
  static_assert(NCOPY <= MMAS && NREAD <= MMAS, "last substep interleave");
  static_assert((LA == kKContig || WTM % 32 == 0) && (LB == kKContig || WTN % 32 == 0), "MN blocks of 32 rows");

  __shared__ __attribute__((aligned(1024))) S lds0[STAGE];
  __shared__ __attribute__((aligned(1024))) S lds1[STAGE];

  const int tid = threadIdx.x;
  const int lane = tid % 64;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
  const int wm = wave / WN;
  const int wn = wave % WN;

  uint32_t bidx, tm, tn;
  tile_of(p, blockIdx.x, bidx, tm, tn);
  const uint32_t m0 = tm * BM;
  const uint32_t n0 = tn * BN;
  const int64_t boff_a = group_offset<0>(p.gb, bidx);
  const int64_t boff_b = group_offset<1>(p.gb, bidx);
  const int64_t boff_c = group_offset<2>(p.gb, bidx);

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
  auto copy = [&](int q, uint32_t stage) {
    if (q < CopyA::NI) ca.issue_one(q, static_cast<const S*>(p.a) + w.oa, stage);
    else cb.issue_one(q - CopyA::NI, static_cast<const S*>(p.b) + w.ob, stage + uint32_t(BM * BK * sizeof(S)));
  };
#pragma unroll
  for (int q = 0; q < NCOPY; ++q) copy(q, lds0_addr);
  w.advance(nk);
#pragma unroll
  for (int q = 0; q < NCOPY; ++q) copy(q, lds1_addr);
  w.advance(nk);
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NCOPY) : "memory");  // K tile 0 of this wave landed
  __syncthreads();
  frags(lds0, 0, 0);

  // first: the tile's first K tile, whose first MFMAs start the accumulators from 0
  auto step = [&](S* stage_cur, const S* stage_nxt, uint32_t cur_addr, auto first) {
    // substep 0: its MFMAs interleaved with the fragment reads of substep 1
    frags(stage_cur, 1, 1);
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        if constexpr (decltype(first)::value) PipeMma<T>::mma_first(acc[i][j], bf[0][j], af[0][i]);
        else PipeMma<T>::mma(acc[i][j], bf[0][j], af[0][i]);
      }
#pragma unroll
    for (int q = 0; q < MMAS; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      // the fragment reads spread evenly over the substep
      if ((q * NREAD) / MMAS != ((q + 1) * NREAD) / MMAS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
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
      // copies and fragment reads spread evenly over the substep, alternating
      const int c0 = (q * NCOPY) / MMAS, c1 = ((q + 1) * NCOPY) / MMAS;
      if (c0 != c1) copy(c0, cur_addr);
      const int r0 = (q * (FM + FN)) / MMAS, r1 = ((q + 1) * (FM + FN)) / MMAS;
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
  pipe_drain(acc);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (p.vstore == 2) {
    if (p.bias != nullptr) store_pipe_t<T, BN, FM, FN, true>(p, lds0, lds1, acc, m0, n0, boff_c);
    else store_pipe_t<T, BN, FM, FN, false>(p, lds0, lds1, acc, m0, n0, boff_c);
  } else {
    if (p.bias != nullptr) store_pipe<T, BN, FM, FN, true>(p, lds0, lds1, acc, m0, n0, boff_c);
    else store_pipe<T, BN, FM, FN, false>(p, lds0, lds1, acc, m0, n0, boff_c);
  }
}

// ---- launcher ----------------------------------------------------------------------
// contract_pipe keeps as many K walk levels as the descriptor has (1, 2, or up to 4)
template <typename T, int BN, int LA, int LB>
void launch_pipe(const ContractArgs& p, hipStream_t s) {
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
          set_kernel("contract_pipe_256x224");
        } else {
          launch_pipe<T, 256, kKContig, kKContig>(p, s);
          set_kernel("contract_pipe_256x256");
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
  switch (config) {
    case 0: return launch_layouts<T, 256, 256, 2, 4, 1>(p, la, lb, s, "contract_256x256");
    case 1: return launch_layouts<T, 128, 128, 2, 2, 1>(p, la, lb, s, "contract_128x128");
    default: return launch_layouts<T, 64, 64, 2, 2, 1>(p, la, lb, s, "contract_64x64");
  }
}

}  // namespace contract
}  // namespace es
