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
  int32_t inner_scale;  // elements per vector along the innermost output dim
  int32_t nchk;         // range-checked input dims
  int64_t base;         // bytes: sum_j offset_j * stride_j
  FastDiv out_div[kMax];  // innermost dim measured in vectors
  int64_t out_stride[kMax];  // bytes per unit of output coordinate d
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

// Source byte offset of output vector v.  R is the (padded) output rank; OffT is
// int32_t when every in-range source offset fits in 31 bits.  Branch-free: a
// constant-boundary element outside the input only sets `outside`.
template <int R, typename OffT, int BOUNDARY>
__device__ __forceinline__ OffT source_of(const GatherArgs& p, uint32_t v, bool& outside) {
  int32_t coord[R];
  uint32_t rem = v;
  OffT src = OffT(p.base);
#pragma unroll
  for (int d = R - 1; d >= 0; --d) {
    uint32_t r;
    rem = p.out_div[d].divmod(rem, r);
    if (d == R - 1) r *= uint32_t(p.inner_scale);
    coord[d] = int32_t(r);
    src += OffT(r) * OffT(p.out_stride[d]);
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

template <int VB, int R, typename OffT, int BOUNDARY>
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
      const OffT off = source_of<R, OffT, BOUNDARY>(p, valid ? v : 0u, outside);
      keep[u] = valid && !outside;
      src[u] = keep[u] ? off : OffT(0);
    }
    V value[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) value[u] = *reinterpret_cast<const V*>(p.x + src[u]);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint32_t v = base + u * kThreads + threadIdx.x;
      if (v < p.total) reinterpret_cast<V*>(p.out)[v] = select_vec(keep[u], value[u], fillv);
    }
  }
}

template <int VB, typename OffT, int BOUNDARY>
void launch_rank(const GatherArgs& p, uint32_t blocks, hipStream_t s) {
  switch (p.out_rank) {
    case 2: gather_kernel<VB, 2, OffT, BOUNDARY><<<blocks, kThreads, 0, s>>>(p); break;
    case 4: gather_kernel<VB, 4, OffT, BOUNDARY><<<blocks, kThreads, 0, s>>>(p); break;
    case 6: gather_kernel<VB, 6, OffT, BOUNDARY><<<blocks, kThreads, 0, s>>>(p); break;
    default: gather_kernel<VB, 8, OffT, BOUNDARY><<<blocks, kThreads, 0, s>>>(p); break;
  }
}

template <int VB, typename OffT>
void launch_off(const GatherArgs& p, int boundary, uint32_t blocks, hipStream_t s) {
  switch (boundary) {
    case ES_BOUNDARY_REPLICATE: launch_rank<VB, OffT, ES_BOUNDARY_REPLICATE>(p, blocks, s); break;
    case ES_BOUNDARY_PERIODIC: launch_rank<VB, OffT, ES_BOUNDARY_PERIODIC>(p, blocks, s); break;
    default: launch_rank<VB, OffT, ES_BOUNDARY_CONSTANT>(p, blocks, s); break;
  }
}

template <int VB>
void launch_vb(const GatherArgs& p, bool off32, int boundary, uint32_t blocks, hipStream_t s) {
  if (off32) launch_off<VB, int32_t>(p, boundary, blocks, s);
  else launch_off<VB, int64_t>(p, boundary, blocks, s);
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
    // read: vectors along P, one row of the tile per q
    constexpr int RV = TP / VEC;  // vectors per q row
    for (int v = threadIdx.x; v < kTileQ * RV; v += 256) {
      const int q = v / RV, pv = (v - q * RV) * VEC;
      if (p0 + pv < a.size_p && q0 + q < a.size_q) {
        const V val = *reinterpret_cast<const V*>(x + in_base + int64_t(q0 + q) * a.q_in_stride + p0 + pv);
#pragma unroll
        for (int e = 0; e < VEC; ++e) tile[q][pv + e] = val.v[e];
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
        *reinterpret_cast<V*>(out + out_base + int64_t(p0 + p) * a.p_out_stride + q0 + qv) = val;
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
  p.inner_scale = vb / es_;
  const uint64_t total_vec = total / uint64_t(p.inner_scale);
  if (total_vec > kU32Max) return fail(ES_ERR_UNSUPPORTED, "es_gather: output too large (>2^32 vectors)");
  p.total = uint32_t(total_vec);
  p.base = 0;
  for (int i = 0; i < kMax; ++i) {
    p.out_stride[i] = 0;
    const int src_dim = i - pad;  // descriptor dim behind padded dim i
    if (i < rank && src_dim >= 0) {
      int64_t sz = d->out_size[src_dim];
      if (src_dim == inner) sz /= p.inner_scale;
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
  const uint64_t per_group = uint64_t(kUnroll) * kThreads;
  uint64_t blocks64 = (total_vec + per_group - 1) / per_group;
  // whole runs of kRun work-groups per XCD (the extra groups find no work)
  if (blocks64 >= 8 * kRun) blocks64 = (blocks64 + 8 * kRun - 1) / (8 * kRun) * (8 * kRun);
  const uint32_t blocks = uint32_t(blocks64 > 1048576 ? 1048576 : blocks64);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (vb) {
    case 16: launch_vb<16>(p, off32, d->boundary, blocks, s); set_kernel("gather_v16"); break;
    case 8: launch_vb<8>(p, off32, d->boundary, blocks, s); set_kernel("gather_v8"); break;
    case 4: launch_vb<4>(p, off32, d->boundary, blocks, s); set_kernel("gather_v4"); break;
    case 2: launch_vb<2>(p, off32, d->boundary, blocks, s); set_kernel("gather_v2"); break;
    default: launch_vb<1>(p, off32, d->boundary, blocks, s); set_kernel("gather_v1"); break;
  }
  return check_launch("es_gather");
}
