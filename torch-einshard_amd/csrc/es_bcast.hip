// es_bcast: out = x * y over a dense output with broadcast strides.
//
// HBM-streaming: one thread handles VEC consecutive elements of the innermost
// output dim (16-byte loads/stores when x and y are contiguous or broadcast
// along it).  The product is formed in fp32 and rounded once, which is what
// torch's mul does for every supported dtype, so results are bit-exact.
//
// The output rank is a template parameter (padded to 2, 4 or 8 with outer dims
// of size 1), so the coordinate decomposition is straight-line code; offsets are
// 32-bit whenever every offset fits in 31 bits.  Operands read exactly once
// (no broadcast dim) and the output are streamed with nontemporal accesses.
#include "es_common.h"

namespace es {
namespace {

constexpr int kMax = ES_MAX_AXES;
constexpr int kThreads = 256;

// N elements moved as one aligned vector access
template <typename S, int N>
struct alignas(sizeof(S) * N) Pack {
  S v[N];
};

struct BcastArgs {
  const void* x;
  const void* y;
  void* out;
  uint32_t total;     // output vectors
  FastDiv div[kMax];  // dims 1 .. R-1 (R-1 innermost, measured in vectors); dim 0 is not divided
  int64_t sx[kMax];   // element strides of x per output dim
  int64_t sy[kMax];
};

// XMODE / YMODE: 1 = contiguous along the innermost dim (vector load),
//                3 = as 1, and every element is read exactly once (streaming load),
//                0 = broadcast along it (one scalar, replicated),
//                2 = strided along it (VEC scalar loads).
// R: padded output rank, dim R-1 innermost.  OffT: int32_t when the output has
// fewer than 2^31 vectors and every offset of x and y fits in 31 bits.
template <typename T, int VEC, int XMODE, int YMODE, int R, typename OffT>
__global__ __launch_bounds__(kThreads) void bcast_kernel(const BcastArgs p) {
  using S = typename Elem<T>::storage;
  const S* x = static_cast<const S*>(p.x);
  const S* y = static_cast<const S*>(p.y);
  S* out = static_cast<S*>(p.out);
  const OffT ix = OffT(p.sx[R - 1]);
  const OffT iy = OffT(p.sy[R - 1]);
  const uint32_t step = gridDim.x * kThreads;
  for (uint32_t v = blockIdx.x * kThreads + threadIdx.x; v < p.total; v += step) {
    uint32_t rem = v;
    OffT ox = 0, oy = 0;
#pragma unroll
    for (int d = R - 1; d >= 1; --d) {
      const uint32_t q = sizeof(OffT) == 4 ? p.div[d].div31(rem) : p.div[d].div(rem);
      const OffT c = OffT(rem - q * p.div[d].d) * OffT(d == R - 1 ? VEC : 1);
      ox += c * OffT(p.sx[d]);
      oy += c * OffT(p.sy[d]);
      rem = q;
    }
    ox += OffT(rem) * OffT(p.sx[0]);  // v < total leaves the outermost coordinate
    oy += OffT(rem) * OffT(p.sy[0]);
    S xs[VEC], ys[VEC];
    Pack<S, VEC> os;
    if constexpr (XMODE == 1 || XMODE == 3) {
      const Pack<S, VEC>* src = reinterpret_cast<const Pack<S, VEC>*>(x + ox);
      const Pack<S, VEC> px = XMODE == 3 ? load_nt(src) : *src;
#pragma unroll
      for (int i = 0; i < VEC; ++i) xs[i] = px.v[i];
    } else if constexpr (XMODE == 0) {
      const S s = x[ox];
#pragma unroll
      for (int i = 0; i < VEC; ++i) xs[i] = s;
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) xs[i] = x[ox + i * ix];
    }
    if constexpr (YMODE == 1 || YMODE == 3) {
      const Pack<S, VEC>* src = reinterpret_cast<const Pack<S, VEC>*>(y + oy);
      const Pack<S, VEC> py = YMODE == 3 ? load_nt(src) : *src;
#pragma unroll
      for (int i = 0; i < VEC; ++i) ys[i] = py.v[i];
    } else if constexpr (YMODE == 0) {
      const S s = y[oy];
#pragma unroll
      for (int i = 0; i < VEC; ++i) ys[i] = s;
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) ys[i] = y[oy + i * iy];
    }
#pragma unroll
    for (int i = 0; i < VEC; ++i) os.v[i] = Elem<T>::store(Elem<T>::load(xs[i]) * Elem<T>::load(ys[i]));
    store_nt(reinterpret_cast<Pack<S, VEC>*>(out) + v, os);
  }
}

// 16-byte vectors, rank 2 or 4, 32-bit offsets: every mode pair
template <typename T, int R>
int launch_fast(const BcastArgs& p, int xmode, int ymode, hipStream_t s, uint32_t blocks) {
  constexpr int VEC = 16 / int(sizeof(typename Elem<T>::storage));
#define ES_BCAST_CASE(XM, YM)                                                    \
  if (xmode == XM && ymode == YM) {                                             \
    bcast_kernel<T, VEC, XM, YM, R, int32_t><<<blocks, kThreads, 0, s>>>(p);    \
    set_kernel("bcast_" #XM #YM);                                               \
    return check_launch("es_bcast");                                            \
  }
  ES_BCAST_CASE(0, 0) ES_BCAST_CASE(0, 1) ES_BCAST_CASE(0, 2) ES_BCAST_CASE(0, 3)
  ES_BCAST_CASE(1, 0) ES_BCAST_CASE(1, 1) ES_BCAST_CASE(1, 2) ES_BCAST_CASE(1, 3)
  ES_BCAST_CASE(2, 0) ES_BCAST_CASE(2, 1) ES_BCAST_CASE(2, 2) ES_BCAST_CASE(2, 3)
  ES_BCAST_CASE(3, 0) ES_BCAST_CASE(3, 1) ES_BCAST_CASE(3, 2) ES_BCAST_CASE(3, 3)
#undef ES_BCAST_CASE
  return fail(ES_ERR_INVALID, "es_bcast: bad stride mode");
}

// everything else: one element per thread, rank 8, 64-bit offsets
template <typename T>
int launch_general(const BcastArgs& p, int xmode, int ymode, hipStream_t s, uint32_t blocks) {
  set_kernel("bcast_scalar");
  if (xmode == 0 && ymode == 0) bcast_kernel<T, 1, 0, 0, kMax, int64_t><<<blocks, kThreads, 0, s>>>(p);
  else if (xmode == 0) bcast_kernel<T, 1, 0, 2, kMax, int64_t><<<blocks, kThreads, 0, s>>>(p);
  else if (ymode == 0) bcast_kernel<T, 1, 2, 0, kMax, int64_t><<<blocks, kThreads, 0, s>>>(p);
  else bcast_kernel<T, 1, 2, 2, kMax, int64_t><<<blocks, kThreads, 0, s>>>(p);
  return check_launch("es_bcast");
}

template <typename T>
int launch_typed(const BcastArgs& p, bool fast, int r, int xmode, int ymode, hipStream_t s, uint32_t blocks) {
  if (!fast) return launch_general<T>(p, xmode, ymode, s, blocks);
  if (r == 2) return launch_fast<T, 2>(p, xmode, ymode, s, blocks);
  return launch_fast<T, 4>(p, xmode, ymode, s, blocks);
}

}  // namespace
}  // namespace es

extern "C" int es_bcast(const es_bcast_desc* d, const void* x, const void* y, void* out, void* stream) {
  using namespace es;
  if (d == nullptr) return fail(ES_ERR_INVALID, "es_bcast: null descriptor");
  const int esz = dtype_size(d->dtype);
  if (esz == 0) return fail(ES_ERR_UNSUPPORTED, "es_bcast: unsupported dtype");
  if (d->rank < 0 || d->rank > kMax) return fail(ES_ERR_INVALID, "es_bcast: rank out of range");
  uint64_t total = 1;
  for (int i = 0; i < d->rank; ++i) {
    if (d->axes[i].size < 0) return fail(ES_ERR_INVALID, "es_bcast: negative size");
    total *= uint64_t(d->axes[i].size);
  }
  if (total == 0) return ES_OK;
  if (x == nullptr || y == nullptr || out == nullptr) return fail(ES_ERR_INVALID, "es_bcast: null pointer");

  // a rank-0 descriptor is a single element: run it as one dim of size 1
  es_axis axes[kMax];
  int rank = d->rank;
  for (int i = 0; i < rank; ++i) axes[i] = d->axes[i];
  if (rank == 0) {
    axes[0] = es_axis{1, 0, 0, 0};
    rank = 1;
  }
  const es_axis& in = axes[rank - 1];

  // 16-byte vectors along the innermost dim, when sizes, strides and pointers allow
  const int max_vec = 16 / esz;
  bool wide = in.size % max_vec == 0 && aligned(out, 16);
  for (int i = 0; i < rank - 1 && wide; ++i)
    if (axes[i].a % max_vec != 0 || axes[i].b % max_vec != 0) wide = false;
  if (in.a == 1 && !aligned(x, 16)) wide = false;
  if (in.b == 1 && !aligned(y, 16)) wide = false;

  // an operand with no broadcast (zero-stride) dim is read exactly once: stream it
  bool x_once = true, y_once = true;
  uint64_t reach_x = 0, reach_y = 0;  // largest |offset| in elements
  for (int i = 0; i < rank; ++i) {
    if (axes[i].size > 1 && axes[i].a == 0) x_once = false;
    if (axes[i].size > 1 && axes[i].b == 0) y_once = false;
    reach_x += uint64_t(axes[i].size - 1) * uint64_t(axes[i].a < 0 ? -axes[i].a : axes[i].a);
    reach_y += uint64_t(axes[i].size - 1) * uint64_t(axes[i].b < 0 ? -axes[i].b : axes[i].b);
  }
  const int xmode = in.a == 1 ? (x_once ? 3 : 1) : (in.a == 0 ? 0 : 2);
  const int ymode = in.b == 1 ? (y_once ? 3 : 1) : (in.b == 0 ? 0 : 2);
  // fast path: 16-byte vectors, rank <= 4, 32-bit offsets; otherwise one element per
  // thread with 64-bit offsets
  const uint64_t lim31 = uint64_t(1) << 31;
  const bool fast = wide && rank <= 4 && total / uint64_t(max_vec) < lim31 && reach_x + max_vec < lim31 &&
                    reach_y + max_vec < lim31;
  const int vec = fast ? max_vec : 1;
  const int r = fast ? (rank <= 2 ? 2 : 4) : kMax;
  const uint64_t total_vec = total / uint64_t(vec);
  if (total_vec > kU32Max) return fail(ES_ERR_UNSUPPORTED, "es_bcast: output too large");

  BcastArgs p;
  p.x = x;
  p.y = y;
  p.out = out;
  p.total = uint32_t(total_vec);
  // descriptor dim i lands at padded dim i + (r - rank); the padding dims have size 1
  for (int j = 0; j < kMax; ++j) {
    const int i = j - (r - rank);
    if (j < r && i >= 0) {
      int64_t s = axes[i].size;
      if (i == rank - 1) s /= vec;
      if (uint64_t(s) > kU32Max) return fail(ES_ERR_UNSUPPORTED, "es_bcast: dim too large");
      p.div[j].init(uint32_t(s));
      p.sx[j] = axes[i].a;
      p.sy[j] = axes[i].b;
    } else {
      p.div[j].init(1);
      p.sx[j] = 0;
      p.sy[j] = 0;
    }
  }
  const uint64_t blocks64 = (total_vec + kThreads - 1) / kThreads;
  const uint32_t blocks = uint32_t(blocks64 > 1048576 ? 1048576 : blocks64);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int xm = fast ? xmode : (xmode == 0 ? 0 : 2);
  const int ym = fast ? ymode : (ymode == 0 ? 0 : 2);
  switch (d->dtype) {
    case ES_F32: return launch_typed<float>(p, fast, r, xm, ym, s, blocks);
    case ES_BF16: return launch_typed<bf16_t>(p, fast, r, xm, ym, s, blocks);
    case ES_F16: return launch_typed<f16_t>(p, fast, r, xm, ym, s, blocks);
  }
  return fail(ES_ERR_UNSUPPORTED, "es_bcast: unsupported dtype");
}
