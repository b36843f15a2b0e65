// es_bcast: out = x * y over a dense output with broadcast strides.
//
// HBM-streaming: one thread handles VEC consecutive elements of the innermost
// output dim (16-byte loads/stores when x and y are contiguous or broadcast
// along it).  The product is formed in fp32 and rounded once, which is what
// torch's mul does for every supported dtype, so results are bit-exact.
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
  uint32_t total;  // vectors
  int32_t rank;
  FastDiv div[kMax];  // innermost dim measured in vectors
  int64_t sx[kMax];
  int64_t sy[kMax];
};

template <typename T, int VEC, int XMODE, int YMODE>
// XMODE / YMODE: 1 = contiguous along the innermost dim (vector load),
//                0 = broadcast along it (one scalar, replicated),
//                2 = strided along it (VEC scalar loads).
__global__ __launch_bounds__(kThreads) void bcast_kernel(const BcastArgs p) {
  using S = typename Elem<T>::storage;
  const S* x = static_cast<const S*>(p.x);
  const S* y = static_cast<const S*>(p.y);
  S* out = static_cast<S*>(p.out);
  const uint32_t step = gridDim.x * kThreads;
  for (uint32_t v = blockIdx.x * kThreads + threadIdx.x; v < p.total; v += step) {
    uint32_t rem = v;
    int64_t ox = 0, oy = 0;
    uint32_t inner = 0;
#pragma unroll
    for (int d = kMax - 1; d >= 0; --d) {
      if (d < p.rank) {
        uint32_t r;
        rem = p.div[d].divmod(rem, r);
        if (d == p.rank - 1) {
          inner = r * VEC;
          ox += int64_t(inner) * p.sx[d];
          oy += int64_t(inner) * p.sy[d];
        } else {
          ox += int64_t(r) * p.sx[d];
          oy += int64_t(r) * p.sy[d];
        }
      }
    }
    const int64_t ix = p.sx[p.rank - 1];
    const int64_t iy = p.sy[p.rank - 1];
    S xs[VEC], ys[VEC];
    Pack<S, VEC> os;
    if constexpr (XMODE == 1) {
      const Pack<S, VEC> px = *reinterpret_cast<const Pack<S, VEC>*>(x + ox);
#pragma unroll
      for (int i = 0; i < VEC; ++i) xs[i] = px.v[i];
    } else if constexpr (XMODE == 0) {
      S s = x[ox];
#pragma unroll
      for (int i = 0; i < VEC; ++i) xs[i] = s;
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) xs[i] = x[ox + i * ix];
    }
    if constexpr (YMODE == 1) {
      const Pack<S, VEC> py = *reinterpret_cast<const Pack<S, VEC>*>(y + oy);
#pragma unroll
      for (int i = 0; i < VEC; ++i) ys[i] = py.v[i];
    } else if constexpr (YMODE == 0) {
      S s = y[oy];
#pragma unroll
      for (int i = 0; i < VEC; ++i) ys[i] = s;
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) ys[i] = y[oy + i * iy];
    }
#pragma unroll
    for (int i = 0; i < VEC; ++i) os.v[i] = Elem<T>::store(Elem<T>::load(xs[i]) * Elem<T>::load(ys[i]));
    reinterpret_cast<Pack<S, VEC>*>(out)[v] = os;
  }
}

template <typename T, int VEC>
int launch_bcast(const BcastArgs& p, int xmode, int ymode, hipStream_t s, uint32_t blocks) {
#define ES_BCAST_CASE(XM, YM)                                             \
  if (xmode == XM && ymode == YM) {                                      \
    bcast_kernel<T, VEC, XM, YM><<<blocks, kThreads, 0, s>>>(p);         \
    set_kernel("bcast_" #XM #YM);                                        \
    return check_launch("es_bcast");                                     \
  }
  ES_BCAST_CASE(1, 1)
  ES_BCAST_CASE(1, 0)
  ES_BCAST_CASE(0, 1)
  ES_BCAST_CASE(0, 0)
  ES_BCAST_CASE(2, 2)
  ES_BCAST_CASE(1, 2)
  ES_BCAST_CASE(2, 1)
  ES_BCAST_CASE(2, 0)
  ES_BCAST_CASE(0, 2)
#undef ES_BCAST_CASE
  return fail(ES_ERR_INVALID, "es_bcast: bad stride mode");
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

  BcastArgs p;
  p.x = x;
  p.y = y;
  p.out = out;
  // a rank-0 descriptor is a single element: run it as one dim of size 1
  es_axis axes[kMax];
  int rank = d->rank;
  for (int i = 0; i < rank; ++i) axes[i] = d->axes[i];
  if (rank == 0) {
    axes[0] = es_axis{1, 0, 0, 0};
    rank = 1;
  }
  p.rank = rank;
  const es_axis& in = axes[rank - 1];

  // vector width along the innermost dim
  const int max_vec = 16 / esz;
  int vec = 1;
  for (int cand = max_vec; cand > 1; cand /= 2) {
    if (in.size % cand != 0) continue;
    if (!aligned(out, cand * esz)) continue;
    bool ok = true;
    for (int i = 0; i < rank - 1 && ok; ++i)
      if (axes[i].a % cand != 0 || axes[i].b % cand != 0) ok = false;
    if (in.a == 1 && !aligned(x, cand * esz)) ok = false;
    if (in.b == 1 && !aligned(y, cand * esz)) ok = false;
    if (ok) {
      vec = cand;
      break;
    }
  }
  const int xmode = in.a == 1 ? 1 : (in.a == 0 ? 0 : 2);
  const int ymode = in.b == 1 ? 1 : (in.b == 0 ? 0 : 2);
  int xm = xmode, ym = ymode;
  if (vec == 1) {  // scalar path: a strided load covers every case
    xm = xmode == 0 ? 0 : 2;
    ym = ymode == 0 ? 0 : 2;
  }
  const uint64_t total_vec = total / uint64_t(vec);
  if (total_vec > kU32Max) return fail(ES_ERR_UNSUPPORTED, "es_bcast: output too large");
  p.total = uint32_t(total_vec);
  for (int i = 0; i < kMax; ++i) {
    if (i < rank) {
      int64_t s = axes[i].size;
      if (i == rank - 1) s /= vec;
      if (uint64_t(s) > kU32Max) return fail(ES_ERR_UNSUPPORTED, "es_bcast: dim too large");
      p.div[i].init(uint32_t(s));
      p.sx[i] = axes[i].a;
      p.sy[i] = axes[i].b;
    } else {
      p.div[i].init(1);
      p.sx[i] = 0;
      p.sy[i] = 0;
    }
  }
  const uint64_t blocks64 = (total_vec + kThreads - 1) / kThreads;
  const uint32_t blocks = uint32_t(blocks64 > 1048576 ? 1048576 : blocks64);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (d->dtype) {
    case ES_F32:
      if (vec == 4) return launch_bcast<float, 4>(p, xm, ym, s, blocks);
      if (vec == 2) return launch_bcast<float, 2>(p, xm, ym, s, blocks);
      return launch_bcast<float, 1>(p, xm, ym, s, blocks);
    case ES_BF16:
      if (vec == 8) return launch_bcast<bf16_t, 8>(p, xm, ym, s, blocks);
      if (vec == 4) return launch_bcast<bf16_t, 4>(p, xm, ym, s, blocks);
      if (vec == 2) return launch_bcast<bf16_t, 2>(p, xm, ym, s, blocks);
      return launch_bcast<bf16_t, 1>(p, xm, ym, s, blocks);
    case ES_F16:
      if (vec == 8) return launch_bcast<f16_t, 8>(p, xm, ym, s, blocks);
      if (vec == 4) return launch_bcast<f16_t, 4>(p, xm, ym, s, blocks);
      if (vec == 2) return launch_bcast<f16_t, 2>(p, xm, ym, s, blocks);
      return launch_bcast<f16_t, 1>(p, xm, ym, s, blocks);
  }
  return fail(ES_ERR_UNSUPPORTED, "es_bcast: unsupported dtype");
}
