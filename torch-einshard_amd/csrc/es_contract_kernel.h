// Kernel template behind es_contract (see es_contract.h for the design).
// Included by one translation unit per element type.
#pragma once

#include "es_contract.h"

namespace es {
namespace contract {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// offset of linear index `i` of a group in the operand selected by `which`
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
  static __device__ __forceinline__ float to_float(S v) { return v; }
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
  static __device__ __forceinline__ float to_float(S v) { return bf16_to_f32(v); }
  static __device__ __forceinline__ S from_float(float v) { return f32_to_bf16(v); }
};

template <>
struct Traits<f16_t> {
  using S = uint16_t;
  static constexpr int VEC = 8;
  static __device__ __forceinline__ void mma(f32x16& acc, const uint4& nfrag, const uint4& mfrag) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, nfrag), __builtin_bit_cast(f16x8, mfrag),
                                                 acc, 0, 0, 0);
  }
  static __device__ __forceinline__ float to_float(S v) { return Elem<f16_t>::load(v); }
  static __device__ __forceinline__ S from_float(float v) { return Elem<f16_t>::store(v); }
};

// ---- register transposes for MN-contiguous tiles -----------------------------
// in[r] holds VEC consecutive mn-elements of k-row r; out[j] holds the VEC
// k-elements of mn-column j.
__device__ __forceinline__ void transpose_block(const uint4 (&in)[8], uint4 (&out)[8]) {
  // 16-bit elements, 8x8
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int p = j / 2;       // dword holding column j in each input row
    const bool hi = j & 1;     // which half
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t a = (&in[2 * q].x)[p];
      const uint32_t b = (&in[2 * q + 1].x)[p];
      // low half <- a's selected half, high half <- b's selected half
      w[q] = hi ? __builtin_amdgcn_perm(b, a, 0x07060302u) : __builtin_amdgcn_perm(b, a, 0x05040100u);
    }
    out[j] = uint4{w[0], w[1], w[2], w[3]};
  }
}

__device__ __forceinline__ void transpose_block(const uint4 (&in)[4], uint4 (&out)[4]) {
  // 32-bit elements, 4x4
#pragma unroll
  for (int j = 0; j < 4; ++j) out[j] = uint4{(&in[0].x)[j], (&in[1].x)[j], (&in[2].x)[j], (&in[3].x)[j]};
}

// ---- tile loaders -------------------------------------------------------------
// SIDE 0 loads the M-side tile from A, SIDE 1 the N-side tile from B.
template <typename T, int ROWS, int BK, int NT, int LAYOUT, int SIDE>
struct Loader;

// K-contiguous: 16-byte vectors along k
template <typename T, int ROWS, int BK, int NT, int SIDE>
struct Loader<T, ROWS, BK, NT, kKContig, SIDE> {
  using S = typename Traits<T>::S;
  static constexpr int VEC = Traits<T>::VEC;
  static constexpr int KV = BK / VEC;
  static constexpr int RPP = NT / KV;  // rows per pass
  static constexpr int NP = (ROWS + RPP - 1) / RPP;
  static_assert(NT % KV == 0, "tile shape");

  int64_t rowoff[NP];
  uint4 reg[NP];
  int kv, r0;

  __device__ __forceinline__ void init(const ContractArgs& p, int tid, uint32_t row0, int64_t boff) {
    kv = tid % KV;
    r0 = tid / KV;
    const GroupArgs& g = SIDE == 0 ? p.gm : p.gn;
    const uint32_t lim = (SIDE == 0 ? p.M : p.N) - 1;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      uint32_t r = row0 + r0 + i * RPP;
      r = r > lim ? lim : r;  // rows past the edge re-read the last row; never stored
      rowoff[i] = boff + group_offset<SIDE>(g, r) + kv * VEC;
    }
  }

  __device__ __forceinline__ void load(const ContractArgs& p, uint32_t k0) {
    const S* base = static_cast<const S*>(SIDE == 0 ? p.a : p.b);
    const int64_t koff = group_offset<SIDE>(p.gk, k0);
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      if (ROWS % RPP == 0 || r0 + i * RPP < ROWS)
        reg[i] = *reinterpret_cast<const uint4*>(base + rowoff[i] + koff);
    }
  }

  __device__ __forceinline__ void store(S* lds, int ldk) const {
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      if (ROWS % RPP == 0 || r0 + i * RPP < ROWS)
        *reinterpret_cast<uint4*>(lds + (r0 + i * RPP) * ldk + kv * VEC) = reg[i];
    }
  }
};

// MN-contiguous: VEC x VEC blocks loaded along mn, transposed in registers
template <typename T, int ROWS, int BK, int NT, int SIDE>
struct Loader<T, ROWS, BK, NT, kMNContig, SIDE> {
  using S = typename Traits<T>::S;
  static constexpr int VEC = Traits<T>::VEC;
  static constexpr int MG = ROWS / VEC;
  static constexpr int KG = BK / VEC;
  static constexpr int NB = (MG * KG + NT - 1) / NT;

  int64_t off[NB];
  uint4 reg[NB][VEC];
  int mg[NB], kg[NB];
  int64_t kstride;

  __device__ __forceinline__ void init(const ContractArgs& p, int tid, uint32_t row0, int64_t boff) {
    const GroupArgs& g = SIDE == 0 ? p.gm : p.gn;
    const uint32_t lim = (SIDE == 0 ? p.M : p.N) - VEC;  // last full group (extent % VEC == 0)
    kstride = SIDE == 0 ? p.ka_inner : p.kb_inner;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int b = tid + j * NT;
      mg[j] = b % MG;
      kg[j] = b / MG;
      uint32_t r = row0 + mg[j] * VEC;
      r = r > lim ? lim : r;
      off[j] = boff + group_offset<SIDE>(g, r) + int64_t(kg[j] * VEC) * kstride;
    }
  }

  __device__ __forceinline__ void load(const ContractArgs& p, uint32_t k0) {
    const S* base = static_cast<const S*>(SIDE == 0 ? p.a : p.b);
    const int64_t koff = group_offset<SIDE>(p.gk, k0);
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      if ((MG * KG) % NT == 0 || kg[j] < KG) {
#pragma unroll
        for (int kk = 0; kk < VEC; ++kk)
          reg[j][kk] = *reinterpret_cast<const uint4*>(base + off[j] + koff + kk * kstride);
      }
    }
  }

  __device__ __forceinline__ void store(S* lds, int ldk) const {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      if ((MG * KG) % NT == 0 || kg[j] < KG) {
        uint4 t[VEC];
        transpose_block(reg[j], t);
#pragma unroll
        for (int jj = 0; jj < VEC; ++jj)
          *reinterpret_cast<uint4*>(lds + (mg[j] * VEC + jj) * ldk + kg[j] * VEC) = t[jj];
      }
    }
  }
};

// generic: one element at a time, any strides, edges in every direction
template <typename T, int ROWS, int BK, int NT, int SIDE>
struct Loader<T, ROWS, BK, NT, kGeneric, SIDE> {
  using S = typename Traits<T>::S;
  static constexpr int RPP = NT / BK;
  static constexpr int NE = (ROWS + RPP - 1) / RPP;
  static_assert(NT % BK == 0, "tile shape");

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

  __device__ __forceinline__ void load(const ContractArgs& p, uint32_t k0) {
    const S* base = static_cast<const S*>(SIDE == 0 ? p.a : p.b);
    const uint32_t k = k0 + kk;
    const bool kok = k < p.K;
    const int64_t koff = kok ? group_offset<SIDE>(p.gk, k) : 0;
#pragma unroll
    for (int i = 0; i < NE; ++i) reg[i] = (kok && rowok[i]) ? base[rowoff[i] + koff] : S(0);
  }

  __device__ __forceinline__ void store(S* lds, int ldk) const {
#pragma unroll
    for (int i = 0; i < NE; ++i)
      if (r0 + i * RPP < ROWS) lds[(r0 + i * RPP) * ldk + kk] = reg[i];
  }
};

// ---- the kernel ----------------------------------------------------------------
template <typename T, int BM, int BN, int BK, int WM, int WN, int LA, int LB>
__global__ __launch_bounds__(WM * WN * 64, 1) void contract_kernel(const ContractArgs p) {
  using S = typename Traits<T>::S;
  constexpr int NT = WM * WN * 64;
  constexpr int VEC = Traits<T>::VEC;
  constexpr int LDK = BK + VEC;  // LDS row pitch (elements): +16 bytes
  constexpr int KSTEP = 2 * VEC; // k consumed per fragment read
  constexpr int WTM = BM / WM;
  constexpr int WTN = BN / WN;
  constexpr int FM = WTM / 32;
  constexpr int FN = WTN / 32;
  static_assert(FM >= 1 && FN >= 1 && BK % KSTEP == 0, "tile shape");

  __shared__ __attribute__((aligned(16))) S lds[2][(BM + BN) * LDK];

  const int tid = threadIdx.x;
  const int lane = tid % 64;
  const int wave = tid / 64;
  const int wm = wave / WN;
  const int wn = wave % WN;

  // work-group -> tile.  The hardware deals work-groups to the 8 XCDs round
  // robin; give each XCD a contiguous run of tiles (N fastest) so tiles that
  // share an M panel of A meet in the same L2.
  uint32_t bid = blockIdx.x;
  if (p.total_tiles % 8 == 0) bid = (bid % 8) * (p.total_tiles / 8) + bid / 8;
  const uint32_t per_batch = p.tiles_m * p.tiles_n;
  const uint32_t bidx = bid / per_batch;
  const uint32_t rem = bid - bidx * per_batch;
  const uint32_t tm = rem / p.tiles_n;
  const uint32_t tn = rem - tm * p.tiles_n;
  const uint32_t m0 = tm * BM;
  const uint32_t n0 = tn * BN;

  const int64_t boff_a = group_offset<0>(p.gb, bidx);
  const int64_t boff_b = group_offset<1>(p.gb, bidx);
  const int64_t boff_c = group_offset<2>(p.gb, bidx);

  Loader<T, BM, BK, NT, LA, 0> la;
  Loader<T, BN, BK, NT, LB, 1> lb;
  la.init(p, tid, m0, boff_a);
  lb.init(p, tid, n0, boff_b);

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const uint32_t nk = (p.K + BK - 1) / BK;
  if (nk > 0) {
    la.load(p, 0);
    lb.load(p, 0);
    la.store(&lds[0][0], LDK);
    lb.store(&lds[0][BM * LDK], LDK);
  }
  __syncthreads();

  for (uint32_t kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      la.load(p, (kt + 1) * BK);
      lb.load(p, (kt + 1) * BK);
    }
    const S* As = &lds[cur][0];
    const S* Bs = &lds[cur][BM * LDK];
#pragma unroll
    for (int ks = 0; ks < BK / KSTEP; ++ks) {
      const int kofs = ks * KSTEP + (lane / 32) * VEC;
      uint4 af[FM], bf[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = *reinterpret_cast<const uint4*>(As + (wm * WTM + i * 32 + lane % 32) * LDK + kofs);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bf[j] = *reinterpret_cast<const uint4*>(Bs + (wn * WTN + j * 32 + lane % 32) * LDK + kofs);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) Traits<T>::mma(acc[i][j], bf[j], af[i]);
    }
    if (more) {
      la.store(&lds[cur ^ 1][0], LDK);
      lb.store(&lds[cur ^ 1][BM * LDK], LDK);
    }
    __syncthreads();
  }

  // ---- epilogue --------------------------------------------------------------
  // acc[i][j] holds C^T of a 32x32 block.  Pass i stages rows
  // {wm*WTM + i*32 + 0..31 : wm} (WM*32 rows x BN columns, converted to the
  // element type) in LDS as [row][n], then the whole work-group writes them
  // out: 16-byte stores along n when n is the output's contiguous axis, element
  // stores otherwise.
  constexpr int SROWS = WM * 32;
  constexpr int SLD = BN + VEC;  // staging row pitch (elements)
  static_assert(SROWS * SLD <= 2 * (BM + BN) * LDK, "staging tile must fit in LDS");
  S* stage = &lds[0][0];
  S* C = static_cast<S*>(p.c);
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
              float4{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
        } else {
          const uint32_t lo = uint32_t(Traits<T>::from_float(acc[i][j][4 * g])) |
                              (uint32_t(Traits<T>::from_float(acc[i][j][4 * g + 1])) << 16);
          const uint32_t hi = uint32_t(Traits<T>::from_float(acc[i][j][4 * g + 2])) |
                              (uint32_t(Traits<T>::from_float(acc[i][j][4 * g + 3])) << 16);
          *reinterpret_cast<uint2*>(dst) = uint2{lo, hi};
        }
      }
    }
    __syncthreads();
    // staged row r is output row m0 + (r / 32) * WTM + i * 32 + r % 32
    if (p.vstore) {
      constexpr int CV = BN / VEC;  // vectors per staged row
      for (int v = tid; v < SROWS * CV; v += NT) {
        const int r = v / CV;
        const int cv = v - r * CV;
        const uint32_t m = m0 + (r / 32) * WTM + i * 32 + r % 32;
        const uint32_t n = n0 + cv * VEC;
        if (m < p.M && n < p.N) {
          const int64_t off = boff_c + group_offset<2>(p.gm, m) + group_offset<2>(p.gn, n);
          *reinterpret_cast<uint4*>(C + off) = *reinterpret_cast<const uint4*>(stage + r * SLD + cv * VEC);
        }
      }
    } else {
      for (int v = tid; v < SROWS * BN; v += NT) {
        const int r = v / BN;
        const int cn = v - r * BN;
        const uint32_t m = m0 + (r / 32) * WTM + i * 32 + r % 32;
        const uint32_t n = n0 + cn;
        if (m < p.M && n < p.N)
          C[boff_c + group_offset<2>(p.gm, m) + group_offset<2>(p.gn, n)] = stage[r * SLD + cn];
      }
    }
    __syncthreads();
  }
}

// ---- launcher ----------------------------------------------------------------------
template <typename T, int BM, int BN, int BK, int WM, int WN, int LA, int LB>
int launch_one(const ContractArgs& p, hipStream_t s, const char* name) {
  contract_kernel<T, BM, BN, BK, WM, WN, LA, LB><<<p.total_tiles, WM * WN * 64, 0, s>>>(p);
  set_kernel(name);
  return check_launch("es_contract");
}

template <typename T, int BM, int BN, int BK, int WM, int WN>
int launch_layouts(const ContractArgs& p, int la, int lb, hipStream_t s, const char* name) {
  if (la == kKContig && lb == kKContig) return launch_one<T, BM, BN, BK, WM, WN, kKContig, kKContig>(p, s, name);
  if (la == kKContig && lb == kMNContig) return launch_one<T, BM, BN, BK, WM, WN, kKContig, kMNContig>(p, s, name);
  if (la == kMNContig && lb == kKContig) return launch_one<T, BM, BN, BK, WM, WN, kMNContig, kKContig>(p, s, name);
  if (la == kMNContig && lb == kMNContig) return launch_one<T, BM, BN, BK, WM, WN, kMNContig, kMNContig>(p, s, name);
  return fail(ES_ERR_INVALID, "es_contract: layout combination has no fast kernel");
}

template <typename T>
int launch_typed(const ContractArgs& p, int config, int la, int lb, hipStream_t s) {
  constexpr int BK = sizeof(typename Traits<T>::S) == 4 ? 32 : 64;
  if (la == kGeneric || lb == kGeneric)
    return launch_one<T, 64, 64, 32, 2, 2, kGeneric, kGeneric>(p, s, "contract_generic_64x64");
  switch (config) {
    case 0: return launch_layouts<T, 256, 256, BK, 2, 2>(p, la, lb, s, "contract_256x256");
    case 1: return launch_layouts<T, 128, 128, BK, 2, 2>(p, la, lb, s, "contract_128x128");
    default: return launch_layouts<T, 64, 64, BK, 2, 2>(p, la, lb, s, "contract_64x64");
  }
}

}  // namespace contract
}  // namespace es
