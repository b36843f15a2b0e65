// es_gather: the window / halo / permutation / diagonal copy.
//
// A thread moves kUnroll vectors of VB bytes of the dense output.  The output
// coordinate is recovered from the linear vector index with FastDiv (one
// multiply-high per dim).  The source address is linear in the output
// coordinate — input dim j contributes (o[pos_j] + o[win_j] + offset_j) *
// stride_j — so the host folds it into one byte stride per output dim plus a
// constant, and the kernel forms it with one multiply-add per output dim.
// Only the input dims that can leave their range (a window, an offset, or an
// output extent larger than the input) are range-checked; their coordinates are
// summed from the output coordinate through 0 / all-ones masks, without
// branches.  Out-of-range coordinates take the boundary rule (a template
// parameter): the whole element becomes `fill`, or the coordinate is clamped or
// wrapped and the address corrected by (new - old) * stride.
//
// Elements move as raw bits, so the copy is bit-exact for any element type.
// The kernel is HBM-bound: each output byte is written once; a 3x3 window
// re-reads each input element 9 times, from L2.
#include <algorithm>
#include <type_traits>
#include <utility>

#include "es_common.h"

namespace es {
namespace {

constexpr int kMax = ES_MAX_AXES;
constexpr int kThreads = 256;

struct GatherArgs {
  const unsigned char* x;
  unsigned char* out;
  uint64_t fill;  // fill pattern replicated over the vector width (low 8 bytes)
  uint32_t total; // number of output vectors
  int32_t out_rank;
  int32_t inner_shift;  // log2 of the elements per vector along the innermost output dim
  int32_t nchk;         // range-checked input dims
  int64_t base;         // bytes: sum_j offset_j * stride_j
  FastDiv out_div[kMax];  // innermost dim measured in vectors
  int64_t out_stride[kMax];  // bytes per unit of output coordinate d (innermost: per vector)
  // range-checked input dims: coordinate = chk_off + sum_d (o[d] & chk_mask[k][d]),
  // chk_mask 0 or all ones (an output dim feeds an input dim at most once)
  int32_t chk_mask[kMax][kMax];
  int32_t chk_off[kMax];
  int32_t chk_size[kMax];
  uint32_t chk_bias[kMax];  // periodic: a multiple of size making c + bias >= 0
  FastDiv chk_div[kMax];    // periodic: division by size
  int64_t chk_stride[kMax]; // bytes
};

template <int VB>
struct Vec;
template <>
struct Vec<1> { using type = uint8_t; };
template <>
struct Vec<2> { using type = uint16_t; };
template <>
struct Vec<4> { using type = uint32_t; };
template <>
struct Vec<8> { using type = uint2; };
template <>
struct Vec<16> { using type = uint4; };

template <int VB>
__device__ __forceinline__ typename Vec<VB>::type fill_vec(uint64_t f) {
  using V = typename Vec<VB>::type;
  if constexpr (VB == 16) {
    return V{uint32_t(f), uint32_t(f >> 32), uint32_t(f), uint32_t(f >> 32)};
  } else if constexpr (VB == 8) {
    return V{uint32_t(f), uint32_t(f >> 32)};
  } else {
    return V(f);
  }
}

// keep ? a : b one 32-bit component at a time (a whole-vector select of values
// held in an array is lowered through private memory).
template <typename V>
__device__ __forceinline__ V select_vec(bool keep, const V& a, const V& b) {
  if constexpr (sizeof(V) == 16) {
    return V{keep ? a.x : b.x, keep ? a.y : b.y, keep ? a.z : b.z, keep ? a.w : b.w};
  } else if constexpr (sizeof(V) == 8) {
    return V{keep ? a.x : b.x, keep ? a.y : b.y};
  } else {
    return keep ? a : b;
  }
}

// Quotient of n < 2^31 by f: the sum mulhi + n cannot carry out of 32 bits.
__device__ __forceinline__ uint32_t div31(const FastDiv& f, uint32_t n) {
  return (__umulhi(f.m, n) + n) >> f.l;
}

// Source byte offset of output vector v.  R is the (padded) output rank; OffT is
// int32_t when every in-range source offset fits in 31 bits.  M24: the output
// has fewer than 2^31 vectors and every dim size, quotient and byte stride fits
// in 23 (strides 24) bits, so remainders and address terms come from full-rate
// 24-bit multiply-adds (v_mad_i32_i24, v_mad_u32_u24) instead of quarter-rate
// 32-bit multiplies; the wrapped 32-bit sum is exact since the result fits.
// The outermost dim needs no division: v < total leaves its coordinate.
// Branch-free: a constant-boundary element outside the input only sets `outside`.
template <int R, typename OffT, int BOUNDARY, bool M24>
__device__ __forceinline__ OffT source_of(const GatherArgs& p, uint32_t v, bool& outside) {
  int32_t coord[R];
  uint32_t rem = v;
  OffT src = OffT(p.base);
#pragma unroll
  for (int d = R - 1; d >= 0; --d) {
    uint32_t r;
    if (d == 0) {
      r = rem;
    } else if constexpr (M24) {
      const uint32_t q = div31(p.out_div[d], rem);
      r = uint32_t(__mul24(int32_t(q), -int32_t(p.out_div[d].d)) + int32_t(rem));
      rem = q;
    } else {
      rem = p.out_div[d].divmod(rem, r);
    }
    // the innermost dim counts vectors: its coordinate in elements is r << inner_shift
    coord[d] = d == R - 1 ? int32_t(r << p.inner_shift) : int32_t(r);
    if constexpr (M24) {
      // dim 0 (never divided) may have a byte stride of 2^24 or more: a full multiply
      src += d == 0 ? OffT(r) * OffT(p.out_stride[d]) : OffT(__umul24(r, uint32_t(p.out_stride[d])));
    } else {
      src += OffT(r) * OffT(p.out_stride[d]);
    }
  }
  outside = false;
  for (int k = 0; k < p.nchk; ++k) {
    int32_t c = p.chk_off[k];
#pragma unroll
    for (int d = 0; d < R; ++d) c += coord[d] & p.chk_mask[k][d];
    const int32_t n = p.chk_size[k];
    if constexpr (BOUNDARY == ES_BOUNDARY_CONSTANT) {
      outside = outside || uint32_t(c) >= uint32_t(n);
    } else {
      int32_t fixed;
      if constexpr (BOUNDARY == ES_BOUNDARY_REPLICATE) {
        fixed = min(max(c, 0), n - 1);
      } else {
        uint32_t r;
        p.chk_div[k].divmod(uint32_t(c) + p.chk_bias[k], r);
        fixed = int32_t(r);
      }
      src += OffT(fixed - c) * OffT(p.chk_stride[k]);
    }
  }
  return src;
}

// A work-group covers kUnroll * kThreads consecutive output vectors and thread t
// moves vectors t, t + kThreads, ...: stores are coalesced across the wave.  All
// addresses are formed first, then the kUnroll loads are issued back to back (a
// fill element loads from offset 0, always valid, and discards it), so each
// thread keeps kUnroll loads in flight.
constexpr int kUnroll = 4;
constexpr uint32_t kRun = 64;  // consecutive work-groups per XCD

// NT: every input element is read at most once (no window, no broadcast, constant
// boundary), so the input is read with streaming loads.
template <int VB, int R, typename OffT, int BOUNDARY, bool M24, bool NT>
__global__ __launch_bounds__(kThreads) void gather_kernel(const GatherArgs p) {
  using V = typename Vec<VB>::type;
  const uint32_t chunk = kUnroll * kThreads;
  const V fillv = fill_vec<VB>(p.fill);
  // Work-groups are dealt to the 8 XCDs round robin.  Renumber them so each XCD
  // walks runs of kRun consecutive work-groups: neighbouring outputs that re-read
  // the same input rows (a window) then share one L2, while the 8 XCDs still
  // stream through one narrow window of memory together (whole-output bands per
  // XCD measured slower).
  uint32_t blk = blockIdx.x;
  if (gridDim.x % (8 * kRun) == 0) {
    const uint32_t xcd = blk % 8, i = blk / 8;
    blk = (i / kRun) * 8 * kRun + xcd * kRun + i % kRun;
  }
  for (uint32_t base = blk * chunk; base < p.total; base += gridDim.x * chunk) {
    OffT src[kUnroll];
    bool keep[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint32_t v = base + u * kThreads + threadIdx.x;
      const bool valid = v < p.total;
      bool outside;
      const OffT off = source_of<R, OffT, BOUNDARY, M24>(p, valid ? v : 0u, outside);
      keep[u] = valid && !outside;
      src[u] = keep[u] ? off : OffT(0);
    }
    V value[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const V* a = reinterpret_cast<const V*>(p.x + src[u]);
      value[u] = NT ? load_nt(a) : *a;
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint32_t v = base + u * kThreads + threadIdx.x;
      if (v < p.total) store_nt(reinterpret_cast<V*>(p.out) + v, select_vec(keep[u], value[u], fillv));
    }
  }
}

// ---- whole rows -------------------------------------------------------------------
// When the innermost output dim is a plain contiguous run of the input (stride 1, no
// offset, no range check, no window), an output row is one copy of a contiguous input
// run.  Rows are cut into segments of one pass: 2^LPR lanes x kRowUnroll vectors.  A
// segment's source is formed once (source_of at its first vector, with every boundary
// rule) and its lanes move its vectors, lane i taking vectors i, i + 2^LPR, ...  With at
// least 8 lanes per segment each access instruction touches whole 128-byte lines, and the
// index arithmetic is paid once per kRowUnroll vectors instead of once per vector.
// Consecutive waves take consecutive segments, so the waves in flight cover one
// contiguous stretch of the output (long rows handed out whole would put every wave
// at the same offset of its own row: addresses a row apart, which fall into the same
// HBM channels).
constexpr int kRowUnroll = 4;

template <int VB, int R, typename OffT, int BOUNDARY, bool M24, bool NT>
__global__ __launch_bounds__(kThreads) void gather_rows(const GatherArgs p, uint32_t units, uint32_t row_vecs,
                                                        FastDiv segs, int lpr) {
  using V = typename Vec<VB>::type;
  const V fillv = fill_vec<VB>(p.fill);
  const int lane = threadIdx.x % 64;
  const uint32_t wave = blockIdx.x * (kThreads / 64) + threadIdx.x / 64;
  const uint32_t waves = gridDim.x * (kThreads / 64);
  const uint32_t per_wave = 64u >> lpr;  // segments a wave moves at once
  const uint32_t li = uint32_t(lane) & ((1u << lpr) - 1);
  const uint32_t seg_vecs = (1u << lpr) * kRowUnroll;
  for (uint32_t unit = wave * per_wave + (uint32_t(lane) >> lpr); unit < units; unit += waves * per_wave) {
    uint32_t seg;
    const uint32_t row = segs.divmod(unit, seg);
    const uint32_t first = seg * seg_vecs;  // the segment's first vector in its row
    bool outside;
    const OffT src = source_of<R, OffT, BOUNDARY, M24>(p, row * row_vecs + first, outside);
    const V* in = reinterpret_cast<const V*>(p.x + (outside ? OffT(0) : src));
    V* out = reinterpret_cast<V*>(p.out) + size_t(row) * row_vecs + first;
    V value[kRowUnroll];
#pragma unroll
    for (int u = 0; u < kRowUnroll; ++u) {
      const uint32_t v = li + (uint32_t(u) << lpr);
      // a fill segment loads (and discards) offset 0, always valid
      if (first + v < row_vecs) value[u] = NT ? load_nt(in + (outside ? 0 : v)) : in[outside ? 0 : v];
    }
#pragma unroll
    for (int u = 0; u < kRowUnroll; ++u) {
      const uint32_t v = li + (uint32_t(u) << lpr);
      if (first + v < row_vecs) store_nt(out + v, outside ? fillv : value[u]);
    }
  }
}

// index arithmetic of a launch: 64-bit offsets, 32-bit, or 32-bit with 24-bit multiplies
enum class Index { k64, k32, k24 };

struct RowLaunch {
  uint32_t units, row_vecs;
  FastDiv segs;  // segments per row
  int lpr;
  uint32_t blocks;
};

template <int VB, typename OffT, int BOUNDARY, bool M24, bool NT>
void launch_rows_rank(const GatherArgs& p, const RowLaunch& r, hipStream_t s) {
  switch (p.out_rank) {
    case 2:
      gather_rows<VB, 2, OffT, BOUNDARY, M24, NT><<<r.blocks, kThreads, 0, s>>>(p, r.units, r.row_vecs, r.segs, r.lpr);
      break;
    case 4:
      gather_rows<VB, 4, OffT, BOUNDARY, M24, NT><<<r.blocks, kThreads, 0, s>>>(p, r.units, r.row_vecs, r.segs, r.lpr);
      break;
    case 6:
      gather_rows<VB, 6, OffT, BOUNDARY, M24, NT><<<r.blocks, kThreads, 0, s>>>(p, r.units, r.row_vecs, r.segs, r.lpr);
      break;
    default:
      gather_rows<VB, 8, OffT, BOUNDARY, M24, NT><<<r.blocks, kThreads, 0, s>>>(p, r.units, r.row_vecs, r.segs, r.lpr);
      break;
  }
}

// 16-byte vectors only (the rows path is taken for rows of at least 16 of them)
template <int BOUNDARY, bool NT>
void launch_rows_index(const GatherArgs& p, Index index, const RowLaunch& r, hipStream_t s) {
  switch (index) {
    case Index::k64: launch_rows_rank<16, int64_t, BOUNDARY, false, NT>(p, r, s); break;
    case Index::k32: launch_rows_rank<16, int32_t, BOUNDARY, false, NT>(p, r, s); break;
    default: launch_rows_rank<16, int32_t, BOUNDARY, true, NT>(p, r, s); break;
  }
}

template <int VB, typename OffT, int BOUNDARY, bool M24, bool NT = false>
void launch_rank(const GatherArgs& p, uint32_t blocks, hipStream_t s) {
  switch (p.out_rank) {
    case 2: gather_kernel<VB, 2, OffT, BOUNDARY, M24, NT><<<blocks, kThreads, 0, s>>>(p); break;
    case 4: gather_kernel<VB, 4, OffT, BOUNDARY, M24, NT><<<blocks, kThreads, 0, s>>>(p); break;
    case 6: gather_kernel<VB, 6, OffT, BOUNDARY, M24, NT><<<blocks, kThreads, 0, s>>>(p); break;
    default: gather_kernel<VB, 8, OffT, BOUNDARY, M24, NT><<<blocks, kThreads, 0, s>>>(p); break;
  }
}

// 16-byte vectors whose input elements are each read at most once: streaming loads
void launch_stream16(const GatherArgs& p, Index index, uint32_t blocks, hipStream_t s) {
  switch (index) {
    case Index::k64: launch_rank<16, int64_t, ES_BOUNDARY_CONSTANT, false, true>(p, blocks, s); break;
    case Index::k32: launch_rank<16, int32_t, ES_BOUNDARY_CONSTANT, false, true>(p, blocks, s); break;
    default: launch_rank<16, int32_t, ES_BOUNDARY_CONSTANT, true, true>(p, blocks, s); break;
  }
}

template <int VB, int BOUNDARY>
void launch_index(const GatherArgs& p, Index index, uint32_t blocks, hipStream_t s) {
  switch (index) {
    case Index::k64: launch_rank<VB, int64_t, BOUNDARY, false>(p, blocks, s); break;
    case Index::k32: launch_rank<VB, int32_t, BOUNDARY, false>(p, blocks, s); break;
    default: launch_rank<VB, int32_t, BOUNDARY, true>(p, blocks, s); break;
  }
}

template <int VB>
void launch_vb(const GatherArgs& p, Index index, int boundary, uint32_t blocks, hipStream_t s) {
  switch (boundary) {
    case ES_BOUNDARY_REPLICATE: launch_index<VB, ES_BOUNDARY_REPLICATE>(p, index, blocks, s); break;
    case ES_BOUNDARY_PERIODIC: launch_index<VB, ES_BOUNDARY_PERIODIC>(p, index, blocks, s); break;
    default: launch_index<VB, ES_BOUNDARY_CONSTANT>(p, index, blocks, s); break;
  }
}

// ---- transposes -----------------------------------------------------------------
// A pure permutation (every input dim read whole, once, by one output dim) whose
// input unit-stride dim lands on an output dim P other than the innermost one Q
// cannot be read and written with wide accesses at once.  A work-group moves a
// TP x 64 tile of (P, Q) for one combination of the other dims through LDS: it
// reads VEC-element vectors along P (contiguous in the input) and writes them
// along Q (contiguous in the output).  TP adapts to a short P.
constexpr int kTileQ = 64;

struct TransposeArgs {
  const unsigned char* x;
  unsigned char* out;
  uint32_t tiles_p, tiles_q, n_outer;
  uint32_t size_p, size_q;
  int64_t q_in_stride;   // elements
  int64_t p_out_stride;  // elements (output is dense)
  int32_t n_rest;        // other output dims, outermost first
  FastDiv rest_div[kMax];
  int64_t rest_in[kMax];   // input stride of each (elements)
  int64_t rest_out[kMax];  // output stride of each (elements)
};

template <typename E, int VEC>
struct EVec {
  E v[VEC];
};

// VEC elements per access; the host guarantees that size_p and size_q are multiples
// of VEC and that every vector is VEC-element aligned in both tensors.
template <typename E, int VEC, int TP>
__global__ __launch_bounds__(256) void transpose_kernel(const TransposeArgs a) {
  using V = EVec<E, VEC>;
  static_assert(TP % VEC == 0 && kTileQ % VEC == 0, "tile shape");
  __shared__ E tile[kTileQ][TP + 1];
  const E* x = reinterpret_cast<const E*>(a.x);
  E* out = reinterpret_cast<E*>(a.out);
  const uint32_t per_outer = a.tiles_p * a.tiles_q;
  for (uint32_t b = blockIdx.x; b < per_outer * a.n_outer; b += gridDim.x) {
    uint32_t outer = b / per_outer;
    const uint32_t t = b - outer * per_outer;
    const uint32_t tp = t / a.tiles_q, tq = t - tp * a.tiles_q;
    int64_t in_base = 0, out_base = 0;
    for (int d = a.n_rest - 1; d >= 0; --d) {
      uint32_t r;
      outer = a.rest_div[d].divmod(outer, r);
      in_base += int64_t(r) * a.rest_in[d];
      out_base += int64_t(r) * a.rest_out[d];
    }
    const uint32_t p0 = tp * TP, q0 = tq * kTileQ;
    // read: vectors along P, one row of the tile per q; all of a lane's loads are issued
    // before the first LDS write
    constexpr int RV = TP / VEC;  // vectors per q row
    constexpr int RN = (kTileQ * RV + 255) / 256;
    V val[RN];
#pragma unroll
    for (int i = 0; i < RN; ++i) {
      const int v = threadIdx.x + i * 256;
      const int q = v / RV, pv = (v - q * RV) * VEC;
      if (v < kTileQ * RV && p0 + pv < a.size_p && q0 + q < a.size_q)
        val[i] = load_nt(reinterpret_cast<const V*>(x + in_base + int64_t(q0 + q) * a.q_in_stride + p0 + pv));
    }
#pragma unroll
    for (int i = 0; i < RN; ++i) {
      const int v = threadIdx.x + i * 256;
      const int q = v / RV, pv = (v - q * RV) * VEC;
      if (v < kTileQ * RV && p0 + pv < a.size_p && q0 + q < a.size_q) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) tile[q][pv + e] = val[i].v[e];
      }
    }
    __syncthreads();
    // write: vectors along Q, one output row per p
    constexpr int WV = kTileQ / VEC;  // vectors per p row
    for (int v = threadIdx.x; v < TP * WV; v += 256) {
      const int p = v / WV, qv = (v - p * WV) * VEC;
      if (p0 + p < a.size_p && q0 + qv < a.size_q) {
        V val;
#pragma unroll
        for (int e = 0; e < VEC; ++e) val.v[e] = tile[qv + e][p];
        store_nt(reinterpret_cast<V*>(out + out_base + int64_t(p0 + p) * a.p_out_stride + q0 + qv), val);
      }
    }
    __syncthreads();
  }
}

template <typename E, int VEC>
void launch_transpose(const TransposeArgs& a, int tp, uint32_t blocks, hipStream_t s) {
  switch (tp) {
    // tp is at least VEC (the host rounds it up), so each instance sees TP >= VEC
    case 8: transpose_kernel<E, VEC, (VEC > 8 ? VEC : 8)><<<blocks, 256, 0, s>>>(a); break;
    case 16: transpose_kernel<E, VEC, (VEC > 16 ? VEC : 16)><<<blocks, 256, 0, s>>>(a); break;
    case 32: transpose_kernel<E, VEC, 32><<<blocks, 256, 0, s>>>(a); break;
    default: transpose_kernel<E, VEC, 64><<<blocks, 256, 0, s>>>(a); break;
  }
}

// The transpose path of es_gather, or false when the descriptor is not such a transpose.
bool try_transpose(const es_gather_desc* d, const void* x, void* out, hipStream_t s, int& status) {
  const int rank = d->out_rank;
  if (d->in_rank != rank || rank < 2) return false;
  int feeder[kMax];
  for (int i = 0; i < rank; ++i) feeder[i] = -1;
  for (int j = 0; j < rank; ++j) {
    const int p = d->pos[j];
    if (d->win[j] >= 0 || d->offset[j] != 0 || d->in_size[j] != d->out_size[p] || feeder[p] >= 0) return false;
    feeder[p] = j;
  }
  const int q = rank - 1;
  int pdim = -1;
  for (int i = 0; i < rank - 1; ++i)
    if (d->in_stride[feeder[i]] == 1 && d->out_size[i] > 1) pdim = i;
  if (pdim < 0 || d->in_stride[feeder[q]] == 1 || d->out_size[q] < kTileQ / 4) return false;
  TransposeArgs a;
  a.x = static_cast<const unsigned char*>(x);
  a.out = static_cast<unsigned char*>(out);
  a.size_p = uint32_t(d->out_size[pdim]);
  a.size_q = uint32_t(d->out_size[q]);
  a.tiles_q = (a.size_q + kTileQ - 1) / kTileQ;
  a.q_in_stride = d->in_stride[feeder[q]];
  int64_t dense[kMax];
  int64_t run = 1;
  for (int i = rank - 1; i >= 0; --i) {
    dense[i] = run;
    run *= d->out_size[i];
  }
  a.p_out_stride = dense[pdim];
  a.n_rest = 0;
  uint64_t n_outer = 1;
  for (int i = 0; i < rank; ++i) {
    if (i == pdim || i == q) continue;
    a.rest_div[a.n_rest].init(uint32_t(d->out_size[i]));
    a.rest_in[a.n_rest] = d->in_stride[feeder[i]];
    a.rest_out[a.n_rest] = dense[i];
    n_outer *= uint64_t(d->out_size[i]);
    ++a.n_rest;
  }
  for (int i = a.n_rest; i < kMax; ++i) {
    a.rest_div[i].init(1);
    a.rest_in[i] = a.rest_out[i] = 0;
  }
  // 16-byte accesses when every vector is aligned and whole; element accesses otherwise
  const int es_ = d->elem_size;
  const int vec = 16 / es_;
  bool wide = aligned(x, 16) && aligned(out, 16) && a.size_p % vec == 0 && a.size_q % vec == 0 &&
              (a.q_in_stride * es_) % 16 == 0 && (a.p_out_stride * es_) % 16 == 0;
  for (int i = 0; i < a.n_rest && wide; ++i)
    if ((a.rest_in[i] * es_) % 16 != 0 || (a.rest_out[i] * es_) % 16 != 0) wide = false;
  // tile depth along P: the power of two >= size_p, 8 .. 64, at least one vector
  int tp = 8;
  while (tp < 64 && uint32_t(tp) < a.size_p) tp *= 2;
  if (wide && tp < vec) tp = vec;
  a.tiles_p = (a.size_p + tp - 1) / tp;
  const uint64_t blocks64 = n_outer * a.tiles_p * a.tiles_q;
  if (blocks64 > kU32Max) return false;
  a.n_outer = uint32_t(n_outer);
  const uint32_t blocks = uint32_t(blocks64 > 1048576 ? 1048576 : blocks64);
  hipStream_t st = s;
  switch (es_) {
    case 1:
      if (wide) launch_transpose<uint8_t, 16>(a, tp, blocks, st);
      else launch_transpose<uint8_t, 1>(a, tp, blocks, st);
      break;
    case 2:
      if (wide) launch_transpose<uint16_t, 8>(a, tp, blocks, st);
      else launch_transpose<uint16_t, 1>(a, tp, blocks, st);
      break;
    case 4:
      if (wide) launch_transpose<uint32_t, 4>(a, tp, blocks, st);
      else launch_transpose<uint32_t, 1>(a, tp, blocks, st);
      break;
    default:
      if (wide) launch_transpose<uint64_t, 2>(a, tp, blocks, st);
      else launch_transpose<uint64_t, 1>(a, tp, blocks, st);
      break;
  }
  set_kernel("gather_transpose");
  status = check_launch("es_gather");
  return true;
}

// ---- padded transposes --------------------------------------------------------------
// The same tile transpose when some dims carry an offset (a halo, a roll): input
// coordinate = output coordinate + offset, out-of-range coordinates take the boundary
// rule.  Reads are single elements along P (64 lanes cover 64 consecutive input
// elements) because an offset along P breaks vector alignment; writes are WVEC-element
// vectors along Q as in transpose_kernel.  The outer dims' coordinates are resolved once
// per tile.  (A transposing halo is what a channels-first input needs before a
// channels-last convolution.)
struct TransposePadArgs {
  const unsigned char* x;
  unsigned char* out;
  uint64_t fill;  // fill bits of one element
  uint32_t tiles_p, tiles_q, n_outer;
  uint32_t size_p, size_q;  // output extents of P and Q
  int32_t in_p, in_q;       // input extents of the dims feeding P and Q
  int32_t off_p, off_q;     // input coordinate = output coordinate + offset
  int64_t q_in_stride;      // elements (P's input stride is 1)
  int64_t p_out_stride;     // elements (output is dense)
  int32_t n_rest;           // other output dims, outermost first
  FastDiv rest_div[kMax];
  int64_t rest_in[kMax];    // input stride of each (elements)
  int64_t rest_out[kMax];   // output stride of each (elements)
  int32_t rest_size[kMax];  // input extent of each
  int32_t rest_off[kMax];   // offset of each
};

// input coordinate i of an extent-n dim under the boundary rule; a constant boundary
// only flags the element
template <int BOUNDARY>
__device__ __forceinline__ int32_t bound_coord(int32_t i, int32_t n, bool& outside) {
  if (uint32_t(i) < uint32_t(n)) return i;
  if constexpr (BOUNDARY == ES_BOUNDARY_CONSTANT) {
    outside = true;
    return 0;
  } else if constexpr (BOUNDARY == ES_BOUNDARY_REPLICATE) {
    return i < 0 ? 0 : n - 1;
  } else {
    const int32_t r = i % n;
    return r < 0 ? r + n : r;
  }
}

template <typename E, int WVEC, int TP, int BOUNDARY>
__global__ __launch_bounds__(256) void transpose_pad_kernel(const TransposePadArgs a) {
  using V = EVec<E, WVEC>;
  __shared__ E tile[kTileQ][TP + 1];
  const E* x = reinterpret_cast<const E*>(a.x);
  E* out = reinterpret_cast<E*>(a.out);
  const E fill = E(a.fill);
  const uint32_t per_outer = a.tiles_p * a.tiles_q;
  for (uint32_t b = blockIdx.x; b < per_outer * a.n_outer; b += gridDim.x) {
    uint32_t outer = b / per_outer;
    const uint32_t t = b - outer * per_outer;
    const uint32_t tp = t / a.tiles_q, tq = t - tp * a.tiles_q;
    int64_t in_base = 0, out_base = 0;
    bool rest_outside = false;
    for (int d = a.n_rest - 1; d >= 0; --d) {
      uint32_t r;
      outer = a.rest_div[d].divmod(outer, r);
      const int32_t i = bound_coord<BOUNDARY>(int32_t(r) + a.rest_off[d], a.rest_size[d], rest_outside);
      in_base += int64_t(i) * a.rest_in[d];
      out_base += int64_t(r) * a.rest_out[d];
    }
    const uint32_t p0 = tp * TP, q0 = tq * kTileQ;
    // read: one element per lane, consecutive lanes along P; all of a lane's loads are
    // issued before the first LDS write, so they are in flight together
    constexpr int RN = kTileQ * TP / 256;
    E val[RN];
#pragma unroll
    for (int i = 0; i < RN; ++i) {
      const int v = threadIdx.x + i * 256;
      const int q = v / TP, p = v - q * TP;
      bool outside = rest_outside || p0 + p >= a.size_p || q0 + q >= a.size_q;
      const int32_t ip = bound_coord<BOUNDARY>(int32_t(p0 + p) + a.off_p, a.in_p, outside);
      const int32_t iq = bound_coord<BOUNDARY>(int32_t(q0 + q) + a.off_q, a.in_q, outside);
      val[i] = outside ? fill : x[in_base + int64_t(iq) * a.q_in_stride + ip];
    }
#pragma unroll
    for (int i = 0; i < RN; ++i) {
      const int v = threadIdx.x + i * 256;
      tile[v / TP][v % TP] = val[i];
    }
    __syncthreads();
    // write: vectors along Q, one output row per p
    constexpr int WV = kTileQ / WVEC;
    for (int v = threadIdx.x; v < TP * WV; v += 256) {
      const int p = v / WV, qv = (v - p * WV) * WVEC;
      if (p0 + p < a.size_p && q0 + qv < a.size_q) {
        V val;
#pragma unroll
        for (int e = 0; e < WVEC; ++e) val.v[e] = tile[qv + e][p];
        store_nt(reinterpret_cast<V*>(out + out_base + int64_t(p0 + p) * a.p_out_stride + q0 + qv), val);
      }
    }
    __syncthreads();
  }
}

template <typename E, int WVEC, int BOUNDARY>
void launch_transpose_pad_tp(const TransposePadArgs& a, int tp, uint32_t blocks, hipStream_t s) {
  switch (tp) {
    case 8: transpose_pad_kernel<E, WVEC, 8, BOUNDARY><<<blocks, 256, 0, s>>>(a); break;
    case 16: transpose_pad_kernel<E, WVEC, 16, BOUNDARY><<<blocks, 256, 0, s>>>(a); break;
    case 32: transpose_pad_kernel<E, WVEC, 32, BOUNDARY><<<blocks, 256, 0, s>>>(a); break;
    default: transpose_pad_kernel<E, WVEC, 64, BOUNDARY><<<blocks, 256, 0, s>>>(a); break;
  }
}

template <typename E, int WIDE>
void launch_transpose_pad(const TransposePadArgs& a, bool wide, int boundary, int tp, uint32_t blocks, hipStream_t s) {
  switch (boundary) {
    case ES_BOUNDARY_REPLICATE:
      if (wide) launch_transpose_pad_tp<E, WIDE, ES_BOUNDARY_REPLICATE>(a, tp, blocks, s);
      else launch_transpose_pad_tp<E, 1, ES_BOUNDARY_REPLICATE>(a, tp, blocks, s);
      break;
    case ES_BOUNDARY_PERIODIC:
      if (wide) launch_transpose_pad_tp<E, WIDE, ES_BOUNDARY_PERIODIC>(a, tp, blocks, s);
      else launch_transpose_pad_tp<E, 1, ES_BOUNDARY_PERIODIC>(a, tp, blocks, s);
      break;
    default:
      if (wide) launch_transpose_pad_tp<E, WIDE, ES_BOUNDARY_CONSTANT>(a, tp, blocks, s);
      else launch_transpose_pad_tp<E, 1, ES_BOUNDARY_CONSTANT>(a, tp, blocks, s);
      break;
  }
}

// The padded-transpose path of es_gather: every input dim feeds one output dim through
// `pos` (no window), the input's unit-stride dim feeds an output dim P other than the
// innermost one Q, and some dim has an offset or a different extent.
bool try_transpose_pad(const es_gather_desc* d, const void* x, void* out, hipStream_t s, int& status) {
  const int rank = d->out_rank;
  if (d->in_rank != rank || rank < 2) return false;
  int feeder[kMax];
  for (int i = 0; i < rank; ++i) feeder[i] = -1;
  bool padded = false;
  for (int j = 0; j < rank; ++j) {
    const int p = d->pos[j];
    if (d->win[j] >= 0 || feeder[p] >= 0 || d->in_size[j] <= 0) return false;
    if (d->in_size[j] >= (int64_t(1) << 30) || d->out_size[p] >= (int64_t(1) << 30)) return false;
    if (d->offset[j] <= -(int64_t(1) << 30) || d->offset[j] >= (int64_t(1) << 30)) return false;
    if (d->offset[j] != 0 || d->in_size[j] != d->out_size[p]) padded = true;
    feeder[p] = j;
  }
  if (!padded) return false;
  const int q = rank - 1;
  int pdim = -1;
  for (int i = 0; i < rank - 1; ++i)
    if (d->in_stride[feeder[i]] == 1 && d->out_size[i] > 1) pdim = i;
  if (pdim < 0 || d->in_stride[feeder[q]] == 1 || d->out_size[q] < kTileQ / 4) return false;
  TransposePadArgs a;
  a.x = static_cast<const unsigned char*>(x);
  a.out = static_cast<unsigned char*>(out);
  const int es_ = d->elem_size;
  a.fill = es_ < 8 ? (d->fill_bits & ((uint64_t(1) << (8 * es_)) - 1)) : d->fill_bits;
  a.size_p = uint32_t(d->out_size[pdim]);
  a.size_q = uint32_t(d->out_size[q]);
  a.in_p = int32_t(d->in_size[feeder[pdim]]);
  a.in_q = int32_t(d->in_size[feeder[q]]);
  a.off_p = int32_t(d->offset[feeder[pdim]]);
  a.off_q = int32_t(d->offset[feeder[q]]);
  a.tiles_q = (a.size_q + kTileQ - 1) / kTileQ;
  a.q_in_stride = d->in_stride[feeder[q]];
  int64_t dense[kMax];
  int64_t run = 1;
  for (int i = rank - 1; i >= 0; --i) {
    dense[i] = run;
    run *= d->out_size[i];
  }
  a.p_out_stride = dense[pdim];
  a.n_rest = 0;
  uint64_t n_outer = 1;
  for (int i = 0; i < rank; ++i) {
    if (i == pdim || i == q) continue;
    a.rest_div[a.n_rest].init(uint32_t(d->out_size[i]));
    a.rest_in[a.n_rest] = d->in_stride[feeder[i]];
    a.rest_out[a.n_rest] = dense[i];
    a.rest_size[a.n_rest] = int32_t(d->in_size[feeder[i]]);
    a.rest_off[a.n_rest] = int32_t(d->offset[feeder[i]]);
    n_outer *= uint64_t(d->out_size[i]);
    ++a.n_rest;
  }
  for (int i = a.n_rest; i < kMax; ++i) {
    a.rest_div[i].init(1);
    a.rest_in[i] = a.rest_out[i] = 0;
    a.rest_size[i] = 1;
    a.rest_off[i] = 0;
  }
  // 16-byte writes along Q when every vector is aligned and whole
  const int vec = 16 / es_;
  bool wide = aligned(out, 16) && a.size_q % vec == 0 && (a.p_out_stride * es_) % 16 == 0;
  for (int i = 0; i < a.n_rest && wide; ++i)
    if ((a.rest_out[i] * es_) % 16 != 0) wide = false;
  int tp = 8;
  while (tp < 64 && uint32_t(tp) < a.size_p) tp *= 2;
  a.tiles_p = (a.size_p + tp - 1) / tp;
  const uint64_t blocks64 = n_outer * a.tiles_p * a.tiles_q;
  if (blocks64 > kU32Max) return false;
  a.n_outer = uint32_t(n_outer);
  const uint32_t blocks = uint32_t(blocks64 > 1048576 ? 1048576 : blocks64);
  switch (es_) {
    case 1: launch_transpose_pad<uint8_t, 16>(a, wide, d->boundary, tp, blocks, s); break;
    case 2: launch_transpose_pad<uint16_t, 8>(a, wide, d->boundary, tp, blocks, s); break;
    case 4: launch_transpose_pad<uint32_t, 4>(a, wide, d->boundary, tp, blocks, s); break;
    default: launch_transpose_pad<uint64_t, 2>(a, wide, d->boundary, tp, blocks, s); break;
  }
  set_kernel("gather_transpose_pad");
  status = check_launch("es_gather");
  return true;
}

// ---- windows staged through LDS ---------------------------------------------------
// A window re-reads each input element once per window position (9 times for a
// 3x3 window); through the vector memory path each re-read costs as much as a
// fresh load.  When some input dim is windowed, the output is cut into blocks that
// fix every output dim before a split dim D, take a tile of T coordinates of D and
// all of every dim after it.  A block's output is then one contiguous chunk, and
// the input it reads is a box: per input dim, the range of o[pos] + o[win] + offset
// over the block.  A work-group loads its block's box into LDS once, applying the
// boundary rule on the way (LDS holds the padded input), then writes the chunk
// from LDS: the output pass has no range checks, and its LDS address depends only
// on the dims that vary inside the block, lds = sum_{d >= D} (o[d] - first[d]) *
// lstride[d].  One block per work-group: a work-group that went on to a second
// block would wait for its first block's stores (the vector memory counter
// counts stores too) before it could use the second box's loads.
//
// Inside a block every index stays below 2^15, so divisions take one full-rate
// 24-bit multiply (SmallDiv) and addresses 24-bit multiply-adds.
constexpr int64_t kBoxBudget = 32 * 1024;  // LDS bytes per block
constexpr int64_t kChunkMax = 64 * 1024;   // output bytes per block
constexpr int kTileDims = 4;               // box dims of extent > 1; dims varying in a block
constexpr uint32_t kSmallBits = 15;        // block-local indices stay below 2^15
constexpr uint32_t kTileRunMax = 1u << 30;  // consecutive blocks per XCD (whole bands measured best)

// q = n / d for n < 2^kSmallBits: q = (n * m) >> s with s = kSmallBits + ceil(log2 d)
// and m = ceil(2^s / d).  The error n (m d - 2^s) / (d 2^s) < 2^kSmallBits / 2^s <= 1/d
// keeps the floor exact; m <= 2^(kSmallBits + 1), so n * m < 2^32.
struct SmallDiv {
  uint32_t d, m, s;
  __host__ void init(uint32_t divisor) {
    d = divisor < 1 ? 1 : divisor;
    uint32_t l = 0;
    while ((1u << l) < d) ++l;
    s = kSmallBits + l;
    m = uint32_t(((uint64_t(1) << s) + d - 1) / d);
  }
  __device__ __forceinline__ uint32_t div(uint32_t n) const { return __umul24(n, m) >> s; }
};

struct TileArgs {
  const unsigned char* x;
  unsigned char* out;
  uint64_t fill;
  uint32_t blocks;     // real blocks (the grid is padded to whole runs per XCD)
  uint32_t run;        // consecutive blocks per XCD; 0: hardware order
  uint32_t out_vecs;   // output vectors per block
  uint32_t box_vecs;   // vectors in the LDS box
  uint32_t src_limit;  // largest input byte offset a vector may start at
  int32_t nfix;        // block coordinates: k = 0 the tile index of D, then dims D-1, D-2, ...
  int32_t tile;        // T
  int32_t box_shift0;  // log2 of the elements per vector along box dim 0
  int32_t ncon;        // input dims of extent 1 in the box (one coordinate per block)
  FastDiv fix_div[kMax];
  // dims varying inside a block, innermost first (k = 0 counts vectors), merged where
  // contiguous in LDS; the unused ones have extent 1
  SmallDiv loc_div[kTileDims];
  uint32_t loc_lds[kTileDims];  // LDS bytes per unit of coordinate
  // box dims, innermost (in LDS) first, k = 0 counting vectors; the unused ones have
  // extent 1.  Input coordinate lo_k + r, lo_k = box_off[k] + sum_f (fixc[f] &
  // box_feed[k][f]) with fixc[0] = tile index * T.
  SmallDiv box_div[kTileDims];
  int32_t box_off[kTileDims];
  int32_t box_feed[kTileDims][kMax];
  int32_t box_size[kTileDims];     // input extent; 2^30 for a dim that never leaves it
  uint32_t box_bias[kTileDims];    // periodic: a multiple of the extent making coordinates >= 0
  FastDiv box_wrap[kTileDims];     // periodic: division by the extent
  int32_t box_chk[kTileDims];      // periodic: the dim can leave its extent
  int32_t box_stride[kTileDims];   // input bytes per unit of coordinate, below 2^23
  // input dims of extent 1 in the box, with the same fields
  int32_t con_off[kMax];
  int32_t con_feed[kMax][kMax];
  int32_t con_size[kMax];
  uint32_t con_bias[kMax];
  FastDiv con_wrap[kMax];
  int32_t con_chk[kMax];
  int32_t con_stride[kMax];
};

// Coordinate c of a box dim under the boundary rule (constant: only `outside` is set).
template <int BOUNDARY>
__device__ __forceinline__ int32_t bound_coord(int32_t c, int32_t size, uint32_t bias, const FastDiv& wrap,
                                               int32_t chk, bool& outside) {
  if constexpr (BOUNDARY == ES_BOUNDARY_CONSTANT) {
    outside = outside || uint32_t(c) >= uint32_t(size);
  } else if constexpr (BOUNDARY == ES_BOUNDARY_REPLICATE) {
    c = min(max(c, 0), size - 1);
  } else if (chk) {
    uint32_t r;
    wrap.divmod(uint32_t(c) + bias, r);
    c = int32_t(r);
  }
  return c;
}

template <int VB, int BOUNDARY, int NL>
__global__ __launch_bounds__(kThreads) void window_tile_kernel(const TileArgs p) {
  using V = typename Vec<VB>::type;
  extern __shared__ __align__(16) unsigned char box[];
  // runs of p.run consecutive blocks per XCD: neighbouring tiles share input rows
  uint32_t blk = blockIdx.x;
  if (p.run > 0) {
    const uint32_t xcd = blk % 8, i = blk / 8;
    blk = (i / p.run) * 8 * p.run + xcd * p.run + i % p.run;
  }
  if (blk >= p.blocks) return;

  int32_t fixc[kMax];
  {
    uint32_t rem = blk;
#pragma unroll
    for (int f = 0; f < kMax; ++f) {
      fixc[f] = 0;
      if (f < p.nfix) {
        uint32_t r;
        rem = p.fix_div[f].divmod(rem, r);
        fixc[f] = int32_t(r);
      }
    }
    fixc[0] *= p.tile;
  }
  // input dims of extent 1: one coordinate and one address term for the block
  uint32_t base = 0;
  bool block_outside = false;
  for (int k = 0; k < p.ncon; ++k) {
    int32_t c = p.con_off[k];
#pragma unroll
    for (int f = 0; f < kMax; ++f) c += fixc[f] & p.con_feed[k][f];
    c = bound_coord<BOUNDARY>(c, p.con_size[k], p.con_bias[k], p.con_wrap[k], p.con_chk[k], block_outside);
    base += uint32_t(c) * uint32_t(p.con_stride[k]);
  }
  int32_t lo[kTileDims];
#pragma unroll
  for (int k = 0; k < kTileDims; ++k) {
    lo[k] = p.box_off[k];
#pragma unroll
    for (int f = 0; f < kMax; ++f) lo[k] += fixc[f] & p.box_feed[k][f];
  }

  // 1. the box into LDS (dense, box dim 0 innermost).  LDS holds whole groups of
  // kUnroll * kThreads vectors, so every lane writes its slots unconditionally (the
  // slots past the box get fill) and the loads stay back to back.
  const V fillv = fill_vec<VB>(p.fill);
  for (uint32_t first = 0; first < p.box_vecs; first += kUnroll * kThreads) {
    uint32_t src[kUnroll];
    bool keep[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint32_t i = first + u * kThreads + threadIdx.x;
      const bool valid = i < p.box_vecs;
      uint32_t n = valid ? i : 0u;
      uint32_t a = base;
      bool outside = block_outside;
#pragma unroll
      for (int k = 0; k < kTileDims; ++k) {
        uint32_t r = n;
        if (k + 1 < kTileDims) {
          const uint32_t q = p.box_div[k].div(n);
          r = n - __umul24(q, p.box_div[k].d);
          n = q;
        }
        int32_t c = lo[k] + int32_t(k == 0 ? r << p.box_shift0 : r);
        c = bound_coord<BOUNDARY>(c, p.box_size[k], p.box_bias[k], p.box_wrap[k], p.box_chk[k], outside);
        a += uint32_t(__mul24(c, p.box_stride[k]));
      }
      // every in-range vector starts at or below src_limit: the compare only guards the load
      keep[u] = valid && !outside && a <= p.src_limit;
      src[u] = keep[u] ? a : 0u;
    }
    V value[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) value[u] = *reinterpret_cast<const V*>(p.x + src[u]);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      reinterpret_cast<V*>(box)[first + u * kThreads + threadIdx.x] = select_vec(keep[u], value[u], fillv);
  }
  __syncthreads();

  // 2. the block's output chunk from LDS: whole groups of kUnroll vectors per
  // thread (all LDS reads issued before the stores), then the rest one at a time
  auto lds_of = [&](uint32_t n) {
    uint32_t o = 0;
#pragma unroll
    for (int k = 0; k < NL; ++k) {
      uint32_t r = n;
      if (k + 1 < NL) {
        const uint32_t q = p.loc_div[k].div(n);
        r = n - __umul24(q, p.loc_div[k].d);
        n = q;
      }
      o += __umul24(r, p.loc_lds[k]);
    }
    return o;
  };
  V* out = reinterpret_cast<V*>(p.out) + uint64_t(blk) * p.out_vecs;
  const uint32_t full = p.out_vecs - p.out_vecs % (kUnroll * kThreads);
  uint32_t first = 0;
  for (; first < full; first += kUnroll * kThreads) {
    uint32_t off[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) off[u] = lds_of(first + u * kThreads + threadIdx.x);
    V value[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) value[u] = *reinterpret_cast<const V*>(box + off[u]);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) store_nt(out + first + u * kThreads + threadIdx.x, value[u]);
  }
  for (uint32_t i = first + threadIdx.x; i < p.out_vecs; i += kThreads)
    store_nt(out + i, *reinterpret_cast<const V*>(box + lds_of(i)));
}

template <int VB, int BOUNDARY>
void launch_tile_nl(const TileArgs& a, int nl, uint32_t grid, size_t lds, hipStream_t s) {
  switch (nl) {
    case 1: window_tile_kernel<VB, BOUNDARY, 1><<<grid, kThreads, lds, s>>>(a); break;
    case 2: window_tile_kernel<VB, BOUNDARY, 2><<<grid, kThreads, lds, s>>>(a); break;
    case 3: window_tile_kernel<VB, BOUNDARY, 3><<<grid, kThreads, lds, s>>>(a); break;
    default: window_tile_kernel<VB, BOUNDARY, 4><<<grid, kThreads, lds, s>>>(a); break;
  }
}

template <int BOUNDARY>
void launch_tile_vb(const TileArgs& a, int vb, int nl, uint32_t grid, size_t lds, hipStream_t s) {
  switch (vb) {
    case 16: launch_tile_nl<16, BOUNDARY>(a, nl, grid, lds, s); break;
    case 8: launch_tile_nl<8, BOUNDARY>(a, nl, grid, lds, s); break;
    case 4: launch_tile_nl<4, BOUNDARY>(a, nl, grid, lds, s); break;
    case 2: launch_tile_nl<2, BOUNDARY>(a, nl, grid, lds, s); break;
    default: launch_tile_nl<1, BOUNDARY>(a, nl, grid, lds, s); break;
  }
}

// Output dims d > D span [0, size); d == D spans a tile of T; d < D is fixed.
inline int64_t tile_span(const es_gather_desc* d, int dim, int split, int64_t t) {
  if (dim < 0) return 0;
  if (dim > split) return d->out_size[dim] - 1;
  return dim == split ? t - 1 : 0;
}

// The box and block layout of one split (D, T).
struct TileLayout {
  int64_t ext[kMax];        // box extent of each input dim
  int order[kMax];          // box dims of extent > 1, innermost (in LDS) first
  int n_wide;
  int64_t lds_stride[kTileDims];  // elements
  int64_t box_elems;
  int64_t loc_ext[kMax];    // dims varying inside a block, innermost first, merged
  int64_t loc_lds[kMax];    // LDS bytes per unit of their coordinate
  int nl;
};

// Box dims of extent > 1: innermost the input dim feeding the output's innermost dim
// when vectors are wider than an element, else the smallest stride; the rest by
// increasing stride.  Dims varying inside a block: innermost first, a dim whose LDS
// step is the inner one's whole extent merged into it.  False when the kernel's
// fixed dim counts or 24-bit strides do not fit.
bool tile_layout(const es_gather_desc* d, int split, int64_t t, int scale, TileLayout& L) {
  const int es_ = d->elem_size, rank = d->out_rank;
  L.n_wide = 0;
  for (int j = 0; j < d->in_rank; ++j) {
    L.ext[j] = 1 + tile_span(d, d->pos[j], split, t) + tile_span(d, d->win[j], split, t);
    if (L.ext[j] > 1) {
      if (L.n_wide == kTileDims || d->in_stride[j] * es_ >= (int64_t(1) << 23)) return false;
      L.order[L.n_wide++] = j;
    }
  }
  int first = -1;
  for (int k = 0; k < L.n_wide; ++k) {
    const int j = L.order[k];
    const bool feeds_inner = d->pos[j] == rank - 1;
    if (scale > 1 ? feeds_inner : (first < 0 || d->in_stride[j] < d->in_stride[L.order[first]])) first = k;
  }
  if (scale > 1 && first < 0) return false;
  if (first > 0) std::swap(L.order[0], L.order[first]);
  for (int k = 2; k < L.n_wide; ++k)
    for (int m = k; m > 1 && d->in_stride[L.order[m]] < d->in_stride[L.order[m - 1]]; --m)
      std::swap(L.order[m], L.order[m - 1]);
  L.box_elems = 1;
  for (int k = 0; k < kTileDims; ++k) {
    L.lds_stride[k] = k < L.n_wide ? L.box_elems : 0;
    if (k < L.n_wide) L.box_elems *= L.ext[L.order[k]];
  }
  if (scale > 1 && (L.ext[L.order[0]] % scale != 0)) return false;
  L.nl = 0;
  for (int i = rank - 1; i >= split; --i) {
    int64_t extent = i == split ? t : d->out_size[i];
    if (extent == 1 && i != rank - 1) continue;
    int64_t lds = 0;
    for (int k = 0; k < L.n_wide; ++k)
      if (d->pos[L.order[k]] == i || d->win[L.order[k]] == i) lds += L.lds_stride[k];
    lds *= es_;
    if (i == rank - 1) {
      lds *= scale;
      extent /= scale;
    }
    if (L.nl > 0 && lds == L.loc_lds[L.nl - 1] * L.loc_ext[L.nl - 1]) {
      L.loc_ext[L.nl - 1] *= extent;
    } else {
      L.loc_ext[L.nl] = extent;
      L.loc_lds[L.nl++] = lds;
    }
  }
  return L.nl <= kTileDims;
}

struct TilePlan {
  TileArgs a;
  uint32_t grid;
  size_t lds;  // bytes of LDS per block
  int nl;      // dims varying inside a block
};

// Plan the LDS-staged path for a windowed descriptor, or false when no split saves
// enough re-reads or the block does not fit the kernel's index arithmetic.  vb: the
// vector bytes es_gather chose (when wider than an element, the output's innermost
// dim is fed with unit stride by one input dim, never out of range).
bool plan_window_tile(const es_gather_desc* d, const void* x, void* out, int vb, const bool* checked,
                      uint64_t fill, TilePlan& plan) {
  const int es_ = d->elem_size, rank = d->out_rank, scale = vb / es_;
  bool windowed = false;
  int64_t reach = 0;
  for (int j = 0; j < d->in_rank; ++j) {
    windowed = windowed || d->win[j] >= 0;
    if (d->in_size[j] == 0 || d->in_stride[j] < 0) return false;
    reach += (d->in_size[j] - 1) * d->in_stride[j] * es_;
    // every coordinate, offset + o[pos] + o[win], stays far inside 24 bits
    const int64_t far = d->out_size[d->pos[j]] + (d->win[j] >= 0 ? d->out_size[d->win[j]] : 0) +
                        (d->offset[j] < 0 ? -d->offset[j] : d->offset[j]);
    if (far >= (int64_t(1) << 22)) return false;
  }
  // 32-bit input offsets: every in-range offset fits in 30 bits
  if (!windowed || x == nullptr || reach > 0x3fffffffLL) return false;

  // the split (D, T) with the most output bytes per box byte
  const int64_t max_vecs = int64_t(1) << kSmallBits;
  TileLayout L;
  int best_d = -1;
  int64_t best_t = 0, best_chunk = 0, best_box = 0;
  for (int split = 0; split < rank; ++split) {
    int64_t inner = 1;
    for (int i = split + 1; i < rank; ++i) inner *= d->out_size[i];
    const int64_t size = d->out_size[split];
    for (int64_t t = 1; t <= size && t <= 4096; ++t) {
      if (size % t != 0) continue;
      if (split == rank - 1 && t % scale != 0) continue;
      const int64_t chunk = t * inner * es_;
      if (chunk > kChunkMax || chunk / vb > max_vecs) break;
      int64_t elems = 1;
      for (int j = 0; j < d->in_rank && elems * es_ <= kBoxBudget; ++j)
        elems *= 1 + tile_span(d, d->pos[j], split, t) + tile_span(d, d->win[j], split, t);
      const int64_t bytes = elems * es_;
      if (bytes > kBoxBudget || bytes / vb > max_vecs) continue;
      // compare chunk / bytes without division; ties go to the larger chunk
      const bool better = best_d < 0 || chunk * best_box > best_chunk * bytes ||
                          (chunk * best_box == best_chunk * bytes && chunk > best_chunk);
      if (better && tile_layout(d, split, t, scale, L)) {
        best_d = split;
        best_t = t;
        best_chunk = chunk;
        best_box = bytes;
      }
    }
  }
  // at least 1.5 output bytes per box byte, or the staging does not pay
  if (best_d < 0 || 2 * best_chunk < 3 * best_box) return false;
  const int split = best_d;
  const int64_t t = best_t;

  TileArgs& a = plan.a;
  a.x = static_cast<const unsigned char*>(x);
  a.out = static_cast<unsigned char*>(out);
  a.fill = fill;
  a.tile = int32_t(t);
  uint64_t total = 1;
  for (int i = 0; i < rank; ++i) total *= uint64_t(d->out_size[i]);
  const uint64_t per_block = uint64_t(best_chunk / es_);
  if (total / per_block > kU32Max) return false;
  a.blocks = uint32_t(total / per_block);
  a.out_vecs = uint32_t(per_block / scale);
  a.src_limit = uint32_t(reach - (vb - es_) > 0 ? reach - (vb - es_) : 0);

  // block coordinates: the tile index of D, then the dims before it (extent-1 dims dropped)
  int fix_dim[kMax];
  a.nfix = 0;
  fix_dim[a.nfix] = split;
  a.fix_div[a.nfix++].init(uint32_t(d->out_size[split] / t));
  for (int i = split - 1; i >= 0; --i) {
    if (d->out_size[i] == 1) continue;
    fix_dim[a.nfix] = i;
    a.fix_div[a.nfix++].init(uint32_t(d->out_size[i]));
  }
  for (int f = a.nfix; f < kMax; ++f) a.fix_div[f].init(1);

  if (!tile_layout(d, split, t, scale, L)) return false;
  const int n_wide = L.n_wide;
  const int* order = L.order;
  const int64_t* ext = L.ext;
  a.box_shift0 = 0;
  while ((1 << a.box_shift0) < scale) ++a.box_shift0;

  auto periodic_bias = [&](int j) {
    const int64_t n = d->in_size[j];
    const int64_t lowest = d->offset[j] < 0 ? -d->offset[j] : 0;
    return uint32_t(((lowest + n - 1) / n) * n);
  };
  for (int k = 0; k < kTileDims; ++k) {
    for (int f = 0; f < kMax; ++f) a.box_feed[k][f] = 0;
    a.box_off[k] = 0;
    a.box_size[k] = 1 << 30;
    a.box_bias[k] = 0;
    a.box_wrap[k].init(1);
    a.box_chk[k] = 0;
    a.box_stride[k] = 0;
    a.box_div[k].init(1);
    if (k >= n_wide) continue;
    const int j = order[k];
    const int64_t stride = d->in_stride[j] * es_;
    a.box_div[k].init(uint32_t(k == 0 ? ext[j] / scale : ext[j]));
    for (int f = 0; f < a.nfix; ++f)
      if (d->pos[j] == fix_dim[f] || d->win[j] == fix_dim[f]) a.box_feed[k][f] = -1;
    a.box_off[k] = int32_t(d->offset[j]);
    if (checked[j]) {
      a.box_size[k] = int32_t(d->in_size[j]);
      a.box_bias[k] = periodic_bias(j);
      a.box_wrap[k].init(uint32_t(d->in_size[j]));
      a.box_chk[k] = 1;
    }
    a.box_stride[k] = int32_t(stride);
  }
  a.box_vecs = uint32_t(L.box_elems / scale);

  // input dims of extent 1
  a.ncon = 0;
  for (int k = 0; k < kMax; ++k) {
    for (int f = 0; f < kMax; ++f) a.con_feed[k][f] = 0;
    a.con_off[k] = 0;
    a.con_size[k] = 1 << 30;
    a.con_bias[k] = 0;
    a.con_wrap[k].init(1);
    a.con_chk[k] = 0;
    a.con_stride[k] = 0;
  }
  for (int j = 0; j < d->in_rank; ++j) {
    if (ext[j] != 1) continue;
    const int k = a.ncon++;
    for (int f = 0; f < a.nfix; ++f)
      if (d->pos[j] == fix_dim[f] || d->win[j] == fix_dim[f]) a.con_feed[k][f] = -1;
    a.con_off[k] = int32_t(d->offset[j]);
    if (checked[j]) {
      a.con_size[k] = int32_t(d->in_size[j]);
      a.con_bias[k] = periodic_bias(j);
      a.con_wrap[k].init(uint32_t(d->in_size[j]));
      a.con_chk[k] = 1;
    }
    a.con_stride[k] = int32_t(d->in_stride[j] * es_);  // below 2^31: reach fits in 30 bits
  }

  const int nl = L.nl;
  const int64_t* loc_ext = L.loc_ext;
  const int64_t* loc_lds = L.loc_lds;
  for (int k = 0; k < kTileDims; ++k) {
    a.loc_div[k].init(uint32_t(k < nl ? loc_ext[k] : 1));
    a.loc_lds[k] = uint32_t(k < nl ? loc_lds[k] : 0);
  }
  plan.nl = nl;

  uint64_t grid = a.blocks;
  a.run = 0;
  if (grid >= 8) {
    const uint64_t run = std::min<uint64_t>((grid + 7) / 8, kTileRunMax);
    a.run = uint32_t(run);
    grid = (grid + 8 * run - 1) / (8 * run) * (8 * run);
  }
  if (grid > kU32Max) return false;
  plan.grid = uint32_t(grid);
  // LDS for whole groups of kUnroll * kThreads vectors
  const uint64_t group = uint64_t(kUnroll) * kThreads;
  plan.lds = size_t((a.box_vecs + group - 1) / group * group) * size_t(vb);
  // the output pass reads LDS below sum_k (extent_k - 1) * loc_lds[k] + vb
  uint64_t last = 0;
  for (int k = 0; k < nl; ++k) last += uint64_t(loc_ext[k] - 1) * uint64_t(loc_lds[k]);
  if (last + uint64_t(vb) > uint64_t(a.box_vecs) * uint64_t(vb)) return false;
  return true;
}

// The LDS-staged path of es_gather, or false when plan_window_tile declines.
bool try_window_tile(const es_gather_desc* d, const void* x, void* out, int vb, const bool* checked,
                     uint64_t fill, hipStream_t s, int& status) {
  TilePlan plan;
  if (!plan_window_tile(d, x, out, vb, checked, fill, plan)) return false;
  switch (d->boundary) {
    case ES_BOUNDARY_REPLICATE: launch_tile_vb<ES_BOUNDARY_REPLICATE>(plan.a, vb, plan.nl, plan.grid, plan.lds, s); break;
    case ES_BOUNDARY_PERIODIC: launch_tile_vb<ES_BOUNDARY_PERIODIC>(plan.a, vb, plan.nl, plan.grid, plan.lds, s); break;
    default: launch_tile_vb<ES_BOUNDARY_CONSTANT>(plan.a, vb, plan.nl, plan.grid, plan.lds, s); break;
  }
  set_kernel("gather_window_tile");
  status = check_launch("es_gather");
  return true;
}

}  // namespace
}  // namespace es

extern "C" int es_gather(const es_gather_desc* d, const void* x, void* out, void* stream) {
  using namespace es;
  if (d == nullptr) return fail(ES_ERR_INVALID, "es_gather: null descriptor");
  const int es_ = d->elem_size;
  if (es_ != 1 && es_ != 2 && es_ != 4 && es_ != 8)
    return fail(ES_ERR_INVALID, "es_gather: elem_size must be 1, 2, 4 or 8");
  if (d->out_rank < 1 || d->out_rank > kMax || d->in_rank < 0 || d->in_rank > kMax)
    return fail(ES_ERR_INVALID, "es_gather: rank out of range");
  if (d->boundary < ES_BOUNDARY_CONSTANT || d->boundary > ES_BOUNDARY_PERIODIC)
    return fail(ES_ERR_INVALID, "es_gather: unknown boundary");
  uint64_t total = 1;
  for (int i = 0; i < d->out_rank; ++i) {
    if (d->out_size[i] < 0) return fail(ES_ERR_INVALID, "es_gather: negative output size");
    if (d->out_size[i] > 0x3fffffff) return fail(ES_ERR_UNSUPPORTED, "es_gather: output dim too large");
    total *= uint64_t(d->out_size[i]);
  }
  bool any_empty_input = false;
  for (int j = 0; j < d->in_rank; ++j) {
    if (d->pos[j] < 0 || d->pos[j] >= d->out_rank || d->win[j] >= d->out_rank || d->win[j] < -1)
      return fail(ES_ERR_INVALID, "es_gather: pos/win names a missing output dim");
    if (d->win[j] == d->pos[j]) return fail(ES_ERR_INVALID, "es_gather: win and pos name the same output dim");
    if (d->in_size[j] < 0 || d->in_size[j] > 0x3fffffff) return fail(ES_ERR_INVALID, "es_gather: bad input size");
    if (d->offset[j] < -0x3fffffff || d->offset[j] > 0x3fffffff)
      return fail(ES_ERR_UNSUPPORTED, "es_gather: offset too large");
    if (d->in_size[j] == 0) {
      if (d->boundary != ES_BOUNDARY_CONSTANT)
        return fail(ES_ERR_INVALID, "es_gather: cannot pad an empty axis with this boundary");
      any_empty_input = true;
    }
  }
  if (total == 0) return ES_OK;
  if (out == nullptr) return fail(ES_ERR_INVALID, "es_gather: null output");
  if (x == nullptr && !any_empty_input) return fail(ES_ERR_INVALID, "es_gather: null input");

  // which input dims can leave [0, size): a window, an offset, or a longer output
  bool checked[kMax];
  for (int j = 0; j < d->in_rank; ++j) {
    const int64_t reach = d->out_size[d->pos[j]] - 1 + (d->win[j] >= 0 ? d->out_size[d->win[j]] - 1 : 0);
    checked[j] = d->win[j] >= 0 || d->offset[j] != 0 || reach + d->offset[j] >= d->in_size[j] || d->in_size[j] == 0;
  }

  {
    int status = ES_OK;
    if (try_transpose(d, x, out, static_cast<hipStream_t>(stream), status)) return status;
    if (try_transpose_pad(d, x, out, static_cast<hipStream_t>(stream), status)) return status;
  }

  // widest vector: the innermost output dim must feed exactly one input dim,
  // through `pos`, with unit stride, and no window/offset that could split it
  const int inner = d->out_rank - 1;
  int vb = es_;
  for (int cand = 16; cand > es_; cand /= 2) {
    const int64_t per = cand / es_;
    if (d->out_size[inner] % per != 0) continue;
    if (!aligned(x, cand) || !aligned(out, cand)) continue;
    int feeders = 0;
    bool ok = true;
    for (int j = 0; j < d->in_rank && ok; ++j) {
      const bool by_pos = d->pos[j] == inner;
      const bool by_win = d->win[j] == inner;
      if (by_win) ok = false;
      if (by_pos) {
        ++feeders;
        if (d->in_stride[j] != 1 || d->win[j] >= 0) ok = false;
        const bool no_pad = !checked[j];
        const bool whole = d->boundary == ES_BOUNDARY_CONSTANT && d->offset[j] % per == 0 &&
                           d->in_size[j] % per == 0;
        if (!no_pad && !whole) ok = false;
      } else if ((d->in_stride[j] * es_) % cand != 0) {
        ok = false;
      }
    }
    if (ok && feeders == 1) {
      vb = cand;
      break;
    }
  }

  GatherArgs p;
  // fill elements load (and discard) offset 0: point at a valid buffer when the input is empty
  p.x = static_cast<const unsigned char*>(x != nullptr ? x : out);
  p.out = static_cast<unsigned char*>(out);
  uint64_t fill = d->fill_bits;
  if (es_ < 8) fill &= (uint64_t(1) << (8 * es_)) - 1;
  for (int w = es_; w < 8; w *= 2) fill |= fill << (8 * w);
  p.fill = fill;
  // the kernels are instantiated for output ranks 2, 4, 6 and 8: pad with leading
  // dims of extent 1 (they contribute coordinate 0)
  const int rank = d->out_rank <= 2 ? 2 : (d->out_rank <= 4 ? 4 : (d->out_rank <= 6 ? 6 : 8));
  const int pad = rank - d->out_rank;
  p.out_rank = rank;
  const int inner_scale = vb / es_;  // a power of two
  p.inner_shift = 0;
  while ((1 << p.inner_shift) < inner_scale) ++p.inner_shift;
  const uint64_t total_vec = total / uint64_t(inner_scale);
  if (total_vec > kU32Max) return fail(ES_ERR_UNSUPPORTED, "es_gather: output too large (>2^32 vectors)");
  p.total = uint32_t(total_vec);
  p.base = 0;
  for (int i = 0; i < kMax; ++i) {
    p.out_stride[i] = 0;
    const int src_dim = i - pad;  // descriptor dim behind padded dim i
    if (i < rank && src_dim >= 0) {
      int64_t sz = d->out_size[src_dim];
      if (src_dim == inner) sz /= inner_scale;
      p.out_div[i].init(uint32_t(sz));
    } else {
      p.out_div[i].init(1);
    }
  }
  int nchk = 0;
  for (int j = 0; j < d->in_rank; ++j) {
    const int64_t sb = d->in_stride[j] * es_;
    p.out_stride[d->pos[j] + pad] += sb;
    if (d->win[j] >= 0) p.out_stride[d->win[j] + pad] += sb;
    p.base += d->offset[j] * sb;
    if (checked[j]) {
      for (int i = 0; i < kMax; ++i) p.chk_mask[nchk][i] = 0;
      p.chk_mask[nchk][d->pos[j] + pad] = -1;
      if (d->win[j] >= 0) p.chk_mask[nchk][d->win[j] + pad] = -1;
      p.chk_off[nchk] = int32_t(d->offset[j]);
      p.chk_size[nchk] = int32_t(d->in_size[j]);
      p.chk_stride[nchk] = sb;
      const int64_t n = d->in_size[j] > 0 ? d->in_size[j] : 1;
      // smallest coordinate is offset (all output coordinates >= 0)
      const int64_t lowest = d->offset[j] < 0 ? -d->offset[j] : 0;
      const int64_t bias = ((lowest + n - 1) / n) * n;
      if (bias + 0x40000000LL + 0x40000000LL > int64_t(kU32Max))
        return fail(ES_ERR_UNSUPPORTED, "es_gather: periodic reach too large");
      p.chk_bias[nchk] = uint32_t(bias);
      p.chk_div[nchk].init(uint32_t(n));
      ++nchk;
    }
  }
  for (int k = nchk; k < kMax; ++k) {
    for (int i = 0; i < kMax; ++i) p.chk_mask[k][i] = 0;
    p.chk_off[k] = 0;
    p.chk_size[k] = 1;
    p.chk_stride[k] = 0;
    p.chk_bias[k] = 0;
    p.chk_div[k].init(1);
  }
  p.nchk = nchk;

  // the innermost dim steps by whole vectors
  p.out_stride[rank - 1] *= inner_scale;

  // 32-bit source offsets when every in-range offset (and each term of it) fits in 31 bits
  bool off32 = true;
  {
    int64_t reach = 0;
    for (int j = 0; j < d->in_rank; ++j) {
      if (d->in_stride[j] < 0) off32 = false;
      const int64_t n = d->in_size[j] > 0 ? d->in_size[j] : 1;
      reach += (n - 1) * d->in_stride[j] * es_;
    }
    for (int i = 0; i < kMax; ++i)
      if (p.out_stride[i] > 0x7fffffffLL || p.out_stride[i] < 0) off32 = false;
    if (reach > 0x3fffffffLL || p.base < -0x3fffffffLL || p.base > 0x3fffffffLL) off32 = false;
  }
  // 24-bit multiplies: fewer than 2^31 vectors, sizes and quotients below 2^23
  // (v_mad_i32_i24 takes them signed), byte strides below 2^24 (dim 0, which is never
  // divided, takes a full multiply and any stride)
  Index index = off32 ? Index::k32 : Index::k64;
  if (off32 && total_vec < 0x80000000ull) {
    bool m24 = total_vec / p.out_div[rank - 1].d < (1u << 23);
    for (int i = 0; i < rank; ++i) {
      if (p.out_div[i].d >= (1u << 23)) m24 = false;
      if (i > 0 && p.out_stride[i] >= (1 << 24)) m24 = false;  // dim 0: a full multiply
    }
    if (m24) index = Index::k24;
  }
  const uint64_t per_group = uint64_t(kUnroll) * kThreads;
  uint64_t blocks64 = (total_vec + per_group - 1) / per_group;
  // whole runs of kRun work-groups per XCD (the extra groups find no work)
  if (blocks64 >= 8 * kRun) blocks64 = (blocks64 + 8 * kRun - 1) / (8 * kRun) * (8 * kRun);
  const uint32_t blocks = uint32_t(blocks64 > 1048576 ? 1048576 : blocks64);
  hipStream_t s = static_cast<hipStream_t>(stream);
  {
    int status = ES_OK;
    if (try_window_tile(d, x, out, vb, checked, p.fill, s, status)) return status;
  }

  // kernel names: vector bytes, then the index arithmetic (none = 32-bit)
  static const char* const kNames[5][3] = {{"gather_v1_o64", "gather_v1", "gather_v1_m24"},
                                           {"gather_v2_o64", "gather_v2", "gather_v2_m24"},
                                           {"gather_v4_o64", "gather_v4", "gather_v4_m24"},
                                           {"gather_v8_o64", "gather_v8", "gather_v8_m24"},
                                           {"gather_v16_o64", "gather_v16", "gather_v16_m24"}};
  int vb_log = 0;
  while ((1 << vb_log) < vb) ++vb_log;
  // every input element read at most once: a constant boundary, no window, and each
  // output dim feeding exactly one input dim (a permutation, possibly padded)
  bool once = d->boundary == ES_BOUNDARY_CONSTANT;
  for (int o = 0; o < d->out_rank && once; ++o) {
    int feeds = 0;
    for (int j = 0; j < d->in_rank; ++j) feeds += (d->pos[j] == o) + (d->win[j] == o);
    if (feeds != 1) once = false;
  }
  for (int j = 0; j < d->in_rank && once; ++j)
    if (d->win[j] >= 0) once = false;
  // whole rows: the innermost output dim a plain contiguous input run (its input dim
  // unchecked, fed by no window) of 16 to 64 vectors.  Measured against the general
  // kernel: 14 % faster on 512-byte rows with two wrapped dims (a roll), 3 % on a
  // padded 512-byte-row copy; 10 % slower on 4 KB rows and 4 % on 64 KB rows, which the
  // general kernel's XCD runs already stream well.
  if (vb == 16 && total_vec < 0x80000000ull) {
    int feeder = -1;
    bool windowed = false;
    for (int j = 0; j < d->in_rank; ++j) {
      if (d->pos[j] == inner) feeder = j;
      if (d->win[j] == inner) windowed = true;
    }
    const uint64_t row_vecs = uint64_t(d->out_size[inner]) / uint64_t(inner_scale);
    if (feeder >= 0 && !windowed && !checked[feeder] && d->in_stride[feeder] == 1 && row_vecs >= 16 &&
        row_vecs <= 64) {
      RowLaunch r;
      r.lpr = 3;  // at least 8 lanes (128 bytes) per segment
      while (r.lpr < 6 && (uint64_t(1) << r.lpr) * kRowUnroll < row_vecs) ++r.lpr;
      const uint64_t seg_vecs = (uint64_t(1) << r.lpr) * kRowUnroll;
      const uint64_t segs = (row_vecs + seg_vecs - 1) / seg_vecs;
      const uint64_t units = (total_vec / row_vecs) * segs;
      if (units < 0x80000000ull) {
        r.units = uint32_t(units);
        r.row_vecs = uint32_t(row_vecs);
        r.segs.init(uint32_t(segs));
        const uint64_t waves = (units + (64u >> r.lpr) - 1) / (64u >> r.lpr);
        const uint64_t rblocks = (waves + kThreads / 64 - 1) / (kThreads / 64);
        r.blocks = uint32_t(rblocks > 1048576 ? 1048576 : rblocks);
        static const char* const kRowNames[3] = {"gather_rows_o64", "gather_rows", "gather_rows_m24"};
        if (once) {
          launch_rows_index<ES_BOUNDARY_CONSTANT, true>(p, index, r, s);
        } else {
          switch (d->boundary) {
            case ES_BOUNDARY_REPLICATE: launch_rows_index<ES_BOUNDARY_REPLICATE, false>(p, index, r, s); break;
            case ES_BOUNDARY_PERIODIC: launch_rows_index<ES_BOUNDARY_PERIODIC, false>(p, index, r, s); break;
            default: launch_rows_index<ES_BOUNDARY_CONSTANT, false>(p, index, r, s); break;
          }
        }
        set_kernel(kRowNames[int(index)]);
        return check_launch("es_gather");
      }
    }
  }
  switch (vb) {
    case 16:
      if (once) launch_stream16(p, index, blocks, s);
      else launch_vb<16>(p, index, d->boundary, blocks, s);
      break;
    case 8: launch_vb<8>(p, index, d->boundary, blocks, s); break;
    case 4: launch_vb<4>(p, index, d->boundary, blocks, s); break;
    case 2: launch_vb<2>(p, index, d->boundary, blocks, s); break;
    default: launch_vb<1>(p, index, d->boundary, blocks, s); break;
  }
  set_kernel(kNames[vb_log][int(index)]);
  return check_launch("es_gather");
}
