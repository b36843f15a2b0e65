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
