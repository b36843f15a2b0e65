// es_contract kernels: batched GEMM on gfx950 MFMA over strided label groups.
//
//   C[batch, m, n] = sum_k A[batch, m, k] * B[batch, n, k]
//
// Every group (batch, M, N, K) is a list of sub-axes with their own strides, so
// a permuted operand such as x[a,b,k,c] with M = (k, a) and K = (b, c) is read
// in place: the tile loaders turn a tile index into addresses, no transposed
// copy is ever materialised.
//
// LDS tiles hold 128-byte rows of K (BK = 64 for 16-bit types, 32 for f32) with the
// 16-byte chunk c of row r stored at chunk position c ^ ((r / 2) % 8), so fragment
// reads (32 consecutive rows, one chunk) and tile writes are free of bank conflicts.
// A 16-byte ds_read gives a lane one MFMA fragment:
//   * contract_pipe, bf16/f16: v_mfma_f32_16x16x32 — lane l holds k = 8*(l/16) .. +7
//     of row l%16;
//   * contract_kernel, bf16/f16: v_mfma_f32_32x32x16 — lane l holds k = 8*(l/32) .. +7
//     of row l%32;
//   * contract_kernel, f32: v_mfma_f32_32x32x2 — a 16-byte read gives a lane 4
//     consecutive k; four MFMAs consume them, lanes 0-31 supplying k 0..3 and lanes
//     32-63 k 4..7.  Both operands use the same k assignment, so every product
//     A[m,k]*B[n,k] is formed exactly once (only the summation order differs).
// The MFMA's first operand is the N-side fragment and the second the M-side
// one, so the accumulator holds C^T: each lane ends with 4 consecutive n of
// one m.  The epilogue computes every tile row's and column's output offset once
// into LDS tables, stages 32-row slices of the tile in LDS and writes them with
// 16-byte streaming stores along n when n is the output's contiguous axis.
//
// Kernels:
//   * contract_pipe (16-bit types, both operands K-contiguous, 256 x 256 or 256 x 224
//     tiles): 4 waves of 128 x 128 (or 128 x 112), two LDS stages filled by
//     global_load_lds_dwordx4 copies issued a full K tile ahead, an explicit MFMA /
//     LDS-read / copy interleave (see es_contract_kernel.h).  224-wide tiles are chosen
//     when an N extent cuts into fewer rounds of one tile per CU than with 256-wide
//     ones (N = 1792);
//   * contract_kernel (every other case): WM x WN waves over a BM x BN tile,
//     double-buffered LDS with one barrier per K tile.  Its loaders:
//       - K-contiguous: direct global -> LDS copies;
//       - MN-contiguous: a thread loads a VEC(k) x VEC(m) block with 16-byte loads
//         along m and transposes it in registers (v_perm_b32 for 16-bit types)
//         before 16-byte LDS stores;
//       - generic: element loads with full index decomposition (any strides).
#pragma once

#include "es_common.h"

namespace es {

enum OperandLayout { kKContig = 0, kMNContig = 1, kGeneric = 2 };

constexpr int kKLevels = 4;  // K sub-axes the fast paths walk incrementally

struct GroupArgs {
  int32_t n;
  FastDiv div[ES_MAX_AXES];
  int64_t sa[ES_MAX_AXES];
  int64_t sb[ES_MAX_AXES];
  int64_t sc[ES_MAX_AXES];
};

struct ContractArgs {
  const void* a;
  const void* b;
  void* c;
  uint32_t M, N, K, batch;
  uint32_t tiles_m, tiles_n;
  uint32_t group_n;      // N-tiles per tile group (divides tiles_n; see tile_of)
  uint32_t total_tiles;
  FastDiv tdiv_batch;    // divides by the tiles of one batch entry (tiles_m * tiles_n)
  FastDiv tdiv_group;    // ... of one tile group (tiles_m * group_n)
  FastDiv tdiv_gn;       // ... by group_n
  // the largest sub-axis count of gb, gm and gn when it is at most 3 (at least 1), else 0:
  // the bounded-group instantiations unroll the offset walks to that many (1 or 2; the
  // halo kernel 3)
  int32_t gdims;
  uint32_t pipe_bn;      // 224: contract_pipe's 256 x 224 tiles; 0: 256 x 256
  int32_t vstore;        // 16-byte vector stores: 1 along n; 2 along m (contract_pipe only)
  int32_t off32;         // every byte offset into A and B fits in 32 bits
  int32_t out_f32;       // C is fp32 (unrounded partial results of a 16-bit contraction)
  int64_t ka_inner;      // stride of the innermost K sub-axis in A
  int64_t kb_inner;      // ... in B
  // Incremental K walk of the fast paths (at most kKLevels K sub-axes, the innermost a
  // multiple of BK): level 0 counts K tiles inside the innermost sub-axis, level L > 0
  // the L-th sub-axis out.  Advancing at level L (every level below it wrapping) adds
  // kda[L] / kdb[L] to the tile's offset in A / B.
  uint32_t kcnt[kKLevels];  // extent of each level (unused levels: never wrap)
  uint32_t klevels;         // levels in use: 1, 2, or kKLevels (3 or 4 K sub-axes)
  int64_t kda[kKLevels];
  int64_t kdb[kKLevels];
  const void* bias;      // es_contract_bias: bias[n] added before rounding; else null
  GroupArgs gb, gm, gn, gk;
  // es_contract_halo (halo_n > 0): A is read through a buffer resource whose range is
  // its span, and a row whose input position falls outside the input is loaded from
  // past that range, as zeros.  Dim 0 is the outer spatial dim (n = 2), dim 1 the inner
  // (a 1-D halo uses dim 1 only and leaves dim 0 one tap, always inside).  Tap
  // k_outer * taps[1] + k_inner reads input position o + dil * k - pad along each dim;
  // K tile t belongs to tap t / ctiles.
  // The resource's base is A's pointer less the shift sum(pad * stride) bytes, so that a
  // row's plain offset (its position's offset plus the K tile's) addresses the input;
  // the range ends where A's span does.  Every offset a row inside the input reads
  // lies at or past the shift.
  int32_t halo_n;
  uint32_t halo_srd[4];     // the buffer resource: base, stride 0, range, 32-bit data
  FastDiv halo_ctiles;      // K tiles per tap
  int32_t halo_taps[2];     // taps per dim (taps[0] * taps[1] <= kHaloMaxTaps)
  int32_t halo_dil[2];
  int32_t halo_pad[2];
  uint32_t halo_extent[2];  // input extents (dim 0 of a 1-D halo: 0xffffffff)
  int32_t halo_mlev[2];     // index in gm of each dim's output position (-1: none)
};

// es_contract_halo: an offset past every halo buffer range, whose copy loads zeros; an
// input's span (bytes, plus one vector) stays below it.
constexpr uint32_t kHaloOutside = 0x80000000u;
constexpr uint64_t kHaloSpanLimit = kHaloOutside;
// taps of one halo contraction: each row keeps one bit per tap (set: outside the input)
constexpr int kHaloMaxTaps = 32;

// Launch one contraction; `config` 0 = 256x256, 1 = 128x128, 2 = 64x64.
int launch_contract_f32(const ContractArgs& p, int config, int la, int lb, hipStream_t s);
int launch_contract_bf16(const ContractArgs& p, int config, int la, int lb, hipStream_t s);
int launch_contract_f16(const ContractArgs& p, int config, int la, int lb, hipStream_t s);

}  // namespace es
