// es_reduce: out[keep] = sum over red of x (* y), fp32 accumulation.
//
// Two schedules, chosen by which axis is contiguous in x:
//
//  * column mode — the innermost kept axis is contiguous: a thread owns VEC
//    consecutive outputs and streams down the reduced axes with 16-byte loads
//    (sum over a leading or middle axis: "p b n h -> b n h", "b n h -> b h").
//    When there are few outputs, the reduced range is split over the waves of
//    a work-group (combined through LDS) and over work-groups (partials in the
//    workspace, combined by a second pass in a fixed order).
//  * row mode — the innermost reduced axis is contiguous: one wave reduces one
//    output, lanes stride through the row with 16-byte loads and the wave is
//    combined with cross-lane shuffles ("b n h -> b n").  Long rows with few
//    outputs are split over work-groups the same way.
//
// The summation order is a fixed function of the descriptor (deterministic);
// each thread adds its terms in increasing reduced-index order.  x is read with
// streaming (nontemporal) loads and the result written with streaming stores:
// each element of x is read exactly once.
#include "es_common.h"

namespace es {
namespace {

constexpr int kMax = ES_MAX_AXES;
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kUnroll = 8;  // terms in flight per thread when unrolling
// Unroll only grids with fewer threads than this: a larger grid keeps enough loads
// in flight with one per thread, and spreading one thread's loads over distant
// rows (a sum over a leading axis) was measured to slow it down.
constexpr uint64_t kUnrollBelowThreads = uint64_t(1) << 21;

template <typename S, int N>
struct alignas(sizeof(S) * N) Pack {
  S v[N];
};

struct ReduceArgs {
  const void* x;
  const void* y;
  void* out;
  float* partial;     // [nsplit][n_out] when nsplit > 1
  uint32_t n_out;     // outputs
  uint32_t n_red;     // reduced index space
  uint32_t nsplit;    // work-group split of the reduced space
  uint32_t chunk;     // reduced indices per split
  int32_t unroll;     // load kUnroll terms per thread before adding them
  int32_t n_keep;
  int32_t n_redax;
  FastDiv keep_div[kMax];  // column mode: innermost measured in vectors
  int64_t keep_sx[kMax];
  int64_t keep_sy[kMax];
  FastDiv red_div[kMax];   // row mode: innermost measured in vectors
  int64_t red_sx[kMax];
  int64_t red_sy[kMax];
};

__device__ __forceinline__ void offsets(uint32_t idx, int n, const FastDiv* div, const int64_t* sx,
                                        const int64_t* sy, int64_t& ox, int64_t& oy, int scale_inner) {
  ox = 0;
  oy = 0;
#pragma unroll
  for (int d = kMax - 1; d >= 0; --d) {
    if (d < n) {
      uint32_t r;
      idx = div[d].divmod(idx, r);
      int64_t c = (d == n - 1) ? int64_t(r) * scale_inner : int64_t(r);
      ox += c * sx[d];
      oy += c * sy[d];
    }
  }
}

// ---------------------------------------------------------------------------
// column mode.  Work-group: `waves` rows x (kThreads / waves) column threads.
template <typename T, int VEC, bool HAS_Y, int XMODE, int YMODE>
__global__ __launch_bounds__(kThreads) void reduce_cols(const ReduceArgs p, const int waves) {
  using S = typename Elem<T>::storage;
  const S* x = static_cast<const S*>(p.x);
  const S* y = static_cast<const S*>(p.y);
  __shared__ float red_lds[kThreads * VEC];

  const int cols = kThreads / waves;
  const int tcol = threadIdx.x % cols;
  const int trow = __builtin_amdgcn_readfirstlane(threadIdx.x / cols);
  const uint32_t vcol = blockIdx.x * cols + tcol;  // output vector index
  const uint32_t split = blockIdx.y;
  const uint32_t n_vec = p.n_out / VEC;
  const bool active = vcol < n_vec;

  int64_t kx = 0, ky = 0;
  if (active) offsets(vcol, p.n_keep, p.keep_div, p.keep_sx, p.keep_sy, kx, ky, VEC);
  const int64_t ix = p.n_keep > 0 ? p.keep_sx[p.n_keep - 1] : 0;
  const int64_t iy = p.n_keep > 0 ? p.keep_sy[p.n_keep - 1] : 0;

  float acc[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) acc[i] = 0.f;

  const uint32_t r_begin = split * p.chunk;
  const uint32_t r_end = min(p.n_red, r_begin + p.chunk);
  // term r of this thread: x (and y) at reduced index r
  auto load = [&](uint32_t r, float (&xv)[VEC], float (&yv)[VEC]) {
    int64_t rx, ry;
    offsets(r, p.n_redax, p.red_div, p.red_sx, p.red_sy, rx, ry, 1);
    const int64_t bx = kx + rx;
    if constexpr (XMODE == 1) {
      const Pack<S, VEC> v = load_nt(reinterpret_cast<const Pack<S, VEC>*>(x + bx));
#pragma unroll
      for (int i = 0; i < VEC; ++i) xv[i] = Elem<T>::load(v.v[i]);
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) xv[i] = Elem<T>::load(load_nt(x + bx + i * ix));
    }
    if constexpr (HAS_Y) {
      const int64_t by = ky + ry;
      if constexpr (YMODE == 1) {
        const Pack<S, VEC> v = *reinterpret_cast<const Pack<S, VEC>*>(y + by);
#pragma unroll
        for (int i = 0; i < VEC; ++i) yv[i] = Elem<T>::load(v.v[i]);
      } else if constexpr (YMODE == 0) {
        const float s = Elem<T>::load(y[by]);
#pragma unroll
        for (int i = 0; i < VEC; ++i) yv[i] = s;
      } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) yv[i] = Elem<T>::load(y[by + i * iy]);
      }
    }
  };
  auto add = [&](const float (&xv)[VEC], const float (&yv)[VEC]) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[i] = HAS_Y ? fmaf(xv[i], yv[i], acc[i]) : acc[i] + xv[i];
  };
  if (active) {
    // kUnroll terms are loaded before any is added, so each thread keeps kUnroll
    // loads in flight; they are still added in increasing r
    uint32_t r = r_begin + trow;
    for (; p.unroll && r + (kUnroll - 1) * waves < r_end; r += kUnroll * waves) {
      float xv[kUnroll][VEC], yv[kUnroll][VEC];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) load(r + u * waves, xv[u], yv[u]);
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) add(xv[u], yv[u]);
    }
    for (; r < r_end; r += waves) {
      float xv[VEC], yv[VEC];
      load(r, xv, yv);
      add(xv, yv);
    }
  }

  if (waves > 1) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) red_lds[(trow * cols + tcol) * VEC + i] = acc[i];
    __syncthreads();
    if (trow != 0) return;
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[i] = 0.f;
    for (int w = 0; w < waves; ++w) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) acc[i] += red_lds[(w * cols + tcol) * VEC + i];
    }
  }
  if (!active) return;
  if (p.nsplit > 1) {
    float* dst = p.partial + size_t(split) * p.n_out + size_t(vcol) * VEC;
#pragma unroll
    for (int i = 0; i < VEC; ++i) dst[i] = acc[i];
  } else {
    Pack<S, VEC> o;
#pragma unroll
    for (int i = 0; i < VEC; ++i) o.v[i] = Elem<T>::store(acc[i]);
    store_nt(reinterpret_cast<Pack<S, VEC>*>(p.out) + vcol, o);
  }
}

// ---------------------------------------------------------------------------
// row mode.  One wave per (output, split); kWaves waves per work-group.
template <typename T, int VEC, bool HAS_Y, int YMODE>
__global__ __launch_bounds__(kThreads) void reduce_rows(const ReduceArgs p) {
  using S = typename Elem<T>::storage;
  const S* x = static_cast<const S*>(p.x);
  const S* y = static_cast<const S*>(p.y);
  const int lane = threadIdx.x % 64;
  const uint32_t o = blockIdx.x * kWaves + threadIdx.x / 64;
  const uint32_t split = blockIdx.y;
  if (o >= p.n_out) return;

  int64_t kx, ky;
  offsets(o, p.n_keep, p.keep_div, p.keep_sx, p.keep_sy, kx, ky, 1);

  // reduced space measured in vectors along the contiguous innermost red axis
  const uint32_t n_rvec = p.n_red / VEC;
  const uint32_t r_begin = split * p.chunk;
  const uint32_t r_end = min(n_rvec, r_begin + p.chunk);
  float acc = 0.f;
  auto load = [&](uint32_t r, Pack<S, VEC>& xv, float (&yv)[VEC]) {
    int64_t rx, ry;
    offsets(r, p.n_redax, p.red_div, p.red_sx, p.red_sy, rx, ry, VEC);
    xv = load_nt(reinterpret_cast<const Pack<S, VEC>*>(x + kx + rx));
    if constexpr (HAS_Y) {
      if constexpr (YMODE == 1) {
        const Pack<S, VEC> v = *reinterpret_cast<const Pack<S, VEC>*>(y + ky + ry);
#pragma unroll
        for (int i = 0; i < VEC; ++i) yv[i] = Elem<T>::load(v.v[i]);
      } else {
        const float s = Elem<T>::load(y[ky + ry]);
#pragma unroll
        for (int i = 0; i < VEC; ++i) yv[i] = s;
      }
    }
  };
  auto add = [&](const Pack<S, VEC>& xv, const float (&yv)[VEC]) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      const float v = Elem<T>::load(xv.v[i]);
      acc = HAS_Y ? fmaf(v, yv[i], acc) : acc + v;
    }
  };
  // as in column mode: kUnroll loads in flight, added in increasing r
  uint32_t r = r_begin + lane;
  for (; p.unroll && r + (kUnroll - 1) * 64 < r_end; r += kUnroll * 64) {
    Pack<S, VEC> xv[kUnroll];
    float yv[kUnroll][VEC];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) load(r + u * 64, xv[u], yv[u]);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) add(xv[u], yv[u]);
  }
  for (; r < r_end; r += 64) {
    Pack<S, VEC> xv;
    float yv[VEC];
    load(r, xv, yv);
    add(xv, yv);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (lane != 0) return;
  if (p.nsplit > 1) {
    p.partial[size_t(split) * p.n_out + o] = acc;
  } else {
    static_cast<S*>(p.out)[o] = Elem<T>::store(acc);
  }
}

// ---------------------------------------------------------------------------
// second pass: out[o] = sum_s partial[s][o], s in increasing order.  A narrow output
// (a bias gradient: a few hundred columns over thousands of partials) leaves one
// work-group, so each thread loads 16 partials ahead of adding them in order: the
// loads overlap, the sum stays sequential.
template <typename T>
__global__ __launch_bounds__(kThreads) void reduce_finish(const float* partial, void* out, uint32_t n_out,
                                                          uint32_t nsplit) {
  using S = typename Elem<T>::storage;
  constexpr uint32_t kAhead = 16;
  const uint32_t o = blockIdx.x * kThreads + threadIdx.x;
  if (o >= n_out) return;
  float acc = 0.f;
  uint32_t s = 0;
  for (; s + kAhead <= nsplit; s += kAhead) {
    float v[kAhead];
#pragma unroll
    for (uint32_t u = 0; u < kAhead; ++u) v[u] = partial[size_t(s + u) * n_out + o];
#pragma unroll
    for (uint32_t u = 0; u < kAhead; ++u) acc += v[u];
  }
  for (; s < nsplit; ++s) acc += partial[size_t(s) * n_out + o];
  static_cast<S*>(out)[o] = Elem<T>::store(acc);
}

// ---------------------------------------------------------------------------
// schedule (a pure function of the descriptor)
struct Schedule {
  bool rows = false;
  int vec = 1;
  int waves = 1;
  uint32_t nsplit = 1;
  uint32_t chunk = 0;
  uint32_t grid_x = 1;
  bool unroll = false;
  int xmode = 2, ymode = 2;
  uint64_t n_out = 1, n_red = 1;
};

int plan(const es_reduce_desc* d, const void* x, const void* y, void* out, Schedule& s) {
  const int esz = dtype_size(d->dtype);
  if (esz == 0) return fail(ES_ERR_UNSUPPORTED, "es_reduce: unsupported dtype");
  if (d->n_keep < 0 || d->n_keep > kMax || d->n_red < 0 || d->n_red > kMax)
    return fail(ES_ERR_INVALID, "es_reduce: axis count out of range");
  for (int i = 0; i < d->n_keep; ++i) {
    if (d->keep[i].size < 0) return fail(ES_ERR_INVALID, "es_reduce: negative size");
    s.n_out *= uint64_t(d->keep[i].size);
  }
  for (int i = 0; i < d->n_red; ++i) {
    if (d->red[i].size < 0) return fail(ES_ERR_INVALID, "es_reduce: negative size");
    s.n_red *= uint64_t(d->red[i].size);
  }
  if (s.n_out > kU32Max || s.n_red > kU32Max) return fail(ES_ERR_UNSUPPORTED, "es_reduce: index space too large");
  const bool has_y = d->has_y != 0;
  const int max_vec = 16 / esz;

  // row mode: innermost reduced axis contiguous in x (and y contiguous or broadcast)
  if (d->n_red > 0) {
    const es_axis& r = d->red[d->n_red - 1];
    if (r.a == 1 && (!has_y || r.b == 1 || r.b == 0) &&
        (d->n_keep == 0 || d->keep[d->n_keep - 1].a != 1)) {
      s.rows = true;
      for (int cand = max_vec; cand >= 1; cand /= 2) {
        bool ok = r.size % cand == 0 && (x == nullptr || aligned(x, cand * esz));
        if (has_y && r.b == 1 && y != nullptr && !aligned(y, cand * esz)) ok = false;
        for (int i = 0; i < d->n_red - 1 && ok; ++i)
          if (d->red[i].a % cand || (has_y && d->red[i].b % cand)) ok = false;
        for (int i = 0; i < d->n_keep && ok; ++i)
          if (d->keep[i].a % cand || (has_y && d->keep[i].b % cand)) ok = false;
        if (ok) {
          s.vec = cand;
          break;
        }
      }
      s.ymode = has_y ? (r.b == 0 ? 0 : 1) : 1;
      const uint64_t n_rvec = s.n_red / uint64_t(s.vec);
      const uint64_t groups = (s.n_out + kWaves - 1) / kWaves;
      // split long rows when there are too few outputs to fill the GPU
      uint64_t nsplit = 1;
      while (groups * nsplit < uint64_t(kTargetGroups) && n_rvec / (nsplit * 2) >= 64 * 16) nsplit *= 2;
      s.nsplit = uint32_t(nsplit);
      s.chunk = uint32_t((n_rvec + nsplit - 1) / nsplit);
      s.grid_x = uint32_t(groups);
      s.unroll = groups * nsplit * kThreads < kUnrollBelowThreads;
      return ES_OK;
    }
  }

  // column mode
  s.rows = false;
  const es_axis* in = d->n_keep > 0 ? &d->keep[d->n_keep - 1] : nullptr;
  s.xmode = (in && in->a == 1) ? 1 : 2;
  s.ymode = has_y ? ((in && in->b == 1) ? 1 : ((in == nullptr || in->b == 0) ? 0 : 2)) : 1;
  for (int cand = max_vec; cand >= 1; cand /= 2) {
    if (cand == 1) {
      s.vec = 1;
      break;
    }
    if (in == nullptr || in->size % cand != 0 || s.xmode != 1) continue;
    bool ok = (x == nullptr || aligned(x, cand * esz)) && (out == nullptr || aligned(out, cand * esz));
    if (has_y && s.ymode == 1 && y != nullptr && !aligned(y, cand * esz)) ok = false;
    for (int i = 0; i < d->n_keep - 1 && ok; ++i)
      if (d->keep[i].a % cand || (has_y && d->keep[i].b % cand)) ok = false;
    for (int i = 0; i < d->n_red && ok; ++i)
      if (d->red[i].a % cand || (has_y && d->red[i].b % cand)) ok = false;
    if (ok) {
      s.vec = cand;
      break;
    }
  }
  if (s.vec == 1) {
    s.xmode = 2;
    if (has_y && s.ymode == 1) s.ymode = 2;
  }
  const uint64_t n_vec = s.n_out / uint64_t(s.vec);
  // few outputs: split the reduced range over the waves of a group, then groups
  s.waves = 1;
  if (n_vec < uint64_t(kThreads) * kTargetGroups && s.n_red >= 4) s.waves = 4;
  const int cols = kThreads / s.waves;
  const uint64_t groups = (n_vec + cols - 1) / uint64_t(cols);
  uint64_t nsplit = 1;
  while (groups * nsplit < uint64_t(kTargetGroups) && s.n_red / (nsplit * 2) >= uint64_t(s.waves) * 32) nsplit *= 2;
  s.nsplit = uint32_t(nsplit);
  s.chunk = uint32_t((s.n_red + nsplit - 1) / nsplit);
  s.grid_x = uint32_t(groups);
  s.unroll = groups * nsplit * kThreads < kUnrollBelowThreads;
  return ES_OK;
}

template <typename T, int VEC>
void launch_cols(const ReduceArgs& p, const Schedule& s, bool has_y, hipStream_t st) {
  dim3 grid(s.grid_x, s.nsplit);
  if (!has_y) {
    if (s.xmode == 1) reduce_cols<T, VEC, false, 1, 1><<<grid, kThreads, 0, st>>>(p, s.waves);
    else reduce_cols<T, VEC, false, 2, 1><<<grid, kThreads, 0, st>>>(p, s.waves);
    set_kernel("reduce_cols");
    return;
  }
  set_kernel("reduce_cols_dot");
#define ES_COLS(XM, YM)                                                                  \
  if (s.xmode == XM && s.ymode == YM) {                                                  \
    reduce_cols<T, VEC, true, XM, YM><<<grid, kThreads, 0, st>>>(p, s.waves);            \
    return;                                                                              \
  }
  ES_COLS(1, 1) ES_COLS(1, 0) ES_COLS(1, 2) ES_COLS(2, 1) ES_COLS(2, 0) ES_COLS(2, 2)
#undef ES_COLS
}

template <typename T, int VEC>
void launch_rows(const ReduceArgs& p, const Schedule& s, bool has_y, hipStream_t st) {
  dim3 grid(s.grid_x, s.nsplit);
  if (!has_y) {
    reduce_rows<T, VEC, false, 1><<<grid, kThreads, 0, st>>>(p);
    set_kernel("reduce_rows");
  } else if (s.ymode == 1) {
    reduce_rows<T, VEC, true, 1><<<grid, kThreads, 0, st>>>(p);
    set_kernel("reduce_rows_dot");
  } else {
    reduce_rows<T, VEC, true, 0><<<grid, kThreads, 0, st>>>(p);
    set_kernel("reduce_rows_dot");
  }
}

template <typename T>
void launch_typed(const ReduceArgs& p, const Schedule& s, bool has_y, hipStream_t st) {
  constexpr int kMaxVec = 16 / int(sizeof(typename Elem<T>::storage));
  if (s.rows) {
    if (s.vec == kMaxVec) launch_rows<T, kMaxVec>(p, s, has_y, st);
    else if (s.vec == 4 && kMaxVec > 4) launch_rows<T, 4>(p, s, has_y, st);
    else if (s.vec == 2) launch_rows<T, 2>(p, s, has_y, st);
    else launch_rows<T, 1>(p, s, has_y, st);
  } else {
    if (s.vec == kMaxVec) launch_cols<T, kMaxVec>(p, s, has_y, st);
    else if (s.vec == 4 && kMaxVec > 4) launch_cols<T, 4>(p, s, has_y, st);
    else if (s.vec == 2) launch_cols<T, 2>(p, s, has_y, st);
    else launch_cols<T, 1>(p, s, has_y, st);
  }
  if (s.nsplit > 1) {
    const uint32_t blocks = uint32_t((s.n_out + kThreads - 1) / kThreads);
    reduce_finish<T><<<blocks, kThreads, 0, st>>>(p.partial, p.out, uint32_t(s.n_out), s.nsplit);
  }
}

}  // namespace
}  // namespace es

extern "C" int64_t es_reduce_workspace_bytes(const es_reduce_desc* d) {
  using namespace es;
  if (d == nullptr) return fail(ES_ERR_INVALID, "es_reduce_workspace_bytes: null descriptor");
  Schedule s;
  int st = plan(d, nullptr, nullptr, nullptr, s);
  if (st != ES_OK) return st;
  if (s.n_out == 0) return 0;
  return s.nsplit > 1 ? int64_t(s.nsplit) * int64_t(s.n_out) * 4 : 0;
}

extern "C" int es_reduce(const es_reduce_desc* d, const void* x, const void* y, void* out, void* workspace,
                         int64_t workspace_bytes, void* stream) {
  using namespace es;
  if (d == nullptr) return fail(ES_ERR_INVALID, "es_reduce: null descriptor");
  // the schedule must not depend on pointers beyond what the workspace query
  // saw, so plan once without pointers (sizes) and once with them (vector width)
  Schedule sizing;
  int st = plan(d, nullptr, nullptr, nullptr, sizing);
  if (st != ES_OK) return st;
  if (sizing.n_out == 0) return ES_OK;
  // an empty reduced extent reads nothing (torch hands out null pointers for empty tensors)
  if (out == nullptr || (sizing.n_red > 0 && (x == nullptr || (d->has_y && y == nullptr))))
    return fail(ES_ERR_INVALID, "es_reduce: null pointer");
  Schedule s;
  st = plan(d, x, y, out, s);
  if (st != ES_OK) return st;
  // workspace requirement never grows with pointer alignment: a narrower vector
  // only makes the same split decision or a larger chunk count per split
  s.nsplit = sizing.nsplit;
  s.chunk = s.rows ? uint32_t((s.n_red / s.vec + s.nsplit - 1) / s.nsplit)
                   : uint32_t((s.n_red + s.nsplit - 1) / s.nsplit);
  const int64_t need = s.nsplit > 1 ? int64_t(s.nsplit) * int64_t(s.n_out) * 4 : 0;
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(ES_ERR_WORKSPACE, "es_reduce: workspace too small (need " + std::to_string(need) + " bytes)");

  ReduceArgs p;
  p.x = x;
  p.y = d->has_y ? y : x;
  p.out = out;
  p.partial = static_cast<float*>(workspace);
  p.n_out = uint32_t(s.n_out);
  p.n_red = uint32_t(s.n_red);
  p.nsplit = s.nsplit;
  p.chunk = s.chunk;
  p.unroll = s.unroll ? 1 : 0;
  p.n_keep = d->n_keep;
  p.n_redax = d->n_red;
  for (int i = 0; i < kMax; ++i) {
    if (i < d->n_keep) {
      int64_t sz = d->keep[i].size;
      if (!s.rows && i == d->n_keep - 1) sz /= s.vec;
      p.keep_div[i].init(uint32_t(sz));
      p.keep_sx[i] = d->keep[i].a;
      p.keep_sy[i] = d->has_y ? d->keep[i].b : 0;
    } else {
      p.keep_div[i].init(1);
      p.keep_sx[i] = 0;
      p.keep_sy[i] = 0;
    }
    if (i < d->n_red) {
      int64_t sz = d->red[i].size;
      if (s.rows && i == d->n_red - 1) sz /= s.vec;
      p.red_div[i].init(uint32_t(sz));
      p.red_sx[i] = d->red[i].a;
      p.red_sy[i] = d->has_y ? d->red[i].b : 0;
    } else {
      p.red_div[i].init(1);
      p.red_sx[i] = 0;
      p.red_sy[i] = 0;
    }
  }
  hipStream_t stream_ = static_cast<hipStream_t>(stream);
  const bool has_y = d->has_y != 0;
  switch (d->dtype) {
    case ES_F32: launch_typed<float>(p, s, has_y, stream_); break;
    case ES_BF16: launch_typed<bf16_t>(p, s, has_y, stream_); break;
    case ES_F16: launch_typed<f16_t>(p, s, has_y, stream_); break;
    default: return fail(ES_ERR_UNSUPPORTED, "es_reduce: unsupported dtype");
  }
  return check_launch("es_reduce");
}
