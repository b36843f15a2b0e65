// es_gather: the window / halo / permutation / diagonal copy.
//
// One thread moves one vector of VB bytes of the dense output.  The output
// coordinate is recovered from the linear vector index with FastDiv (one
// multiply-high per dim), every input coordinate is an affine function of it
// (base + window offset + constant), and the boundary rule is applied per
// input dim.  Elements are moved as raw bits, so the copy is bit-exact for any
// element type.  The kernel is HBM-bound: each output byte is written once,
// input bytes are re-read from L2/MALL (a 3x3 window reads each input element
// 9 times but the working set of neighbouring rows stays cache resident).
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
  int32_t in_rank;
  int32_t boundary;
  int32_t inner_scale;  // elements per vector along the innermost output dim
  FastDiv out_div[kMax];  // innermost dim measured in vectors
  int64_t in_size[kMax];
  int64_t in_stride_bytes[kMax];
  int64_t offset[kMax];
  int32_t pos[kMax];
  int32_t win[kMax];
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

__device__ __forceinline__ int64_t apply_boundary(int64_t c, int64_t size, int boundary, bool& outside) {
  if (c >= 0 && c < size) return c;
  if (boundary == ES_BOUNDARY_REPLICATE) return c < 0 ? 0 : size - 1;
  if (boundary == ES_BOUNDARY_PERIODIC) {
    int64_t r = c % size;
    return r < 0 ? r + size : r;
  }
  outside = true;
  return 0;
}

template <int VB>
__global__ __launch_bounds__(kThreads) void gather_kernel(const GatherArgs p) {
  using V = typename Vec<VB>::type;
  const uint32_t stride = gridDim.x * kThreads;
  for (uint32_t v = blockIdx.x * kThreads + threadIdx.x; v < p.total; v += stride) {
    int32_t coord[kMax];
    uint32_t rem = v;
#pragma unroll
    for (int d = kMax - 1; d >= 0; --d) {
      if (d < p.out_rank) {
        uint32_t r;
        rem = p.out_div[d].divmod(rem, r);
        coord[d] = r;
      } else {
        coord[d] = 0;
      }
    }
    coord[p.out_rank - 1] *= p.inner_scale;

    bool outside = false;
    int64_t src = 0;
#pragma unroll
    for (int d = 0; d < kMax; ++d) {
      if (d < p.in_rank) {
        int64_t c = int64_t(coord[p.pos[d]]) + p.offset[d];
        if (p.win[d] >= 0) c += coord[p.win[d]];
        c = apply_boundary(c, p.in_size[d], p.boundary, outside);
        src += c * p.in_stride_bytes[d];
      }
    }
    V value = outside ? fill_vec<VB>(p.fill) : *reinterpret_cast<const V*>(p.x + src);
    reinterpret_cast<V*>(p.out)[v] = value;
  }
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
    total *= uint64_t(d->out_size[i]);
  }
  if (total == 0) return ES_OK;
  if (x == nullptr || out == nullptr) return fail(ES_ERR_INVALID, "es_gather: null pointer");
  for (int j = 0; j < d->in_rank; ++j) {
    if (d->pos[j] < 0 || d->pos[j] >= d->out_rank || d->win[j] >= d->out_rank || d->win[j] < -1)
      return fail(ES_ERR_INVALID, "es_gather: pos/win names a missing output dim");
    if (d->in_size[j] <= 0) {
      // an empty input dim can only feed a constant-filled output
      if (d->boundary != ES_BOUNDARY_CONSTANT)
        return fail(ES_ERR_INVALID, "es_gather: cannot pad an empty axis with this boundary");
    }
  }
  // Every output coordinate whose input coordinate may leave [0, size) must be
  // covered by the boundary rule; for the replicate/periodic rules the size
  // must be positive (checked above).  Reads stay inside the input: an in-range
  // coordinate per dim times its stride, summed.

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
        const bool no_pad = d->offset[j] == 0 && d->out_size[inner] <= d->in_size[j];
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
  p.x = static_cast<const unsigned char*>(x);
  p.out = static_cast<unsigned char*>(out);
  uint64_t fill = d->fill_bits;
  if (es_ < 8) fill &= (uint64_t(1) << (8 * es_)) - 1;
  for (int w = es_; w < 8; w *= 2) fill |= fill << (8 * w);
  p.fill = fill;
  p.out_rank = d->out_rank;
  p.in_rank = d->in_rank;
  p.boundary = d->boundary;
  p.inner_scale = vb / es_;
  const uint64_t total_vec = total / uint64_t(p.inner_scale);
  if (total_vec > kU32Max) return fail(ES_ERR_UNSUPPORTED, "es_gather: output too large (>2^32 vectors)");
  p.total = uint32_t(total_vec);
  for (int i = 0; i < kMax; ++i) {
    if (i < d->out_rank) {
      int64_t s = d->out_size[i];
      if (i == inner) s /= p.inner_scale;
      if (uint64_t(s) > kU32Max) return fail(ES_ERR_UNSUPPORTED, "es_gather: dim too large");
      p.out_div[i].init(uint32_t(s));
    } else {
      p.out_div[i].init(1);
    }
    if (i < d->in_rank) {
      p.in_size[i] = d->in_size[i];
      p.in_stride_bytes[i] = d->in_stride[i] * es_;
      p.offset[i] = d->offset[i];
      p.pos[i] = d->pos[i];
      p.win[i] = d->win[i];
    } else {
      p.in_size[i] = 1;
      p.in_stride_bytes[i] = 0;
      p.offset[i] = 0;
      p.pos[i] = 0;
      p.win[i] = -1;
    }
  }
  // an empty input dim: every output element is fill
  for (int j = 0; j < d->in_rank; ++j)
    if (d->in_size[j] <= 0) p.in_size[j] = 0;

  const uint64_t blocks64 = (total_vec + kThreads - 1) / kThreads;
  const uint32_t blocks = uint32_t(blocks64 > 1048576 ? 1048576 : blocks64);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (vb) {
    case 16: gather_kernel<16><<<blocks, kThreads, 0, s>>>(p); set_kernel("gather_v16"); break;
    case 8: gather_kernel<8><<<blocks, kThreads, 0, s>>>(p); set_kernel("gather_v8"); break;
    case 4: gather_kernel<4><<<blocks, kThreads, 0, s>>>(p); set_kernel("gather_v4"); break;
    case 2: gather_kernel<2><<<blocks, kThreads, 0, s>>>(p); set_kernel("gather_v2"); break;
    default: gather_kernel<1><<<blocks, kThreads, 0, s>>>(p); set_kernel("gather_v1"); break;
  }
  return check_launch("es_gather");
}
