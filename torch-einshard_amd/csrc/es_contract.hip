// es_contract entry point: descriptor validation, operand-layout and tile
// selection, launch.
#include "es_contract.h"

#include <algorithm>
#include <string>

namespace es {
namespace {

constexpr int kMax = ES_MAX_AXES;

int fill_group(GroupArgs& g, int n, const es_axis* axes, uint64_t& extent, const char* name) {
  if (n < 0 || n > kMax) return fail(ES_ERR_INVALID, std::string("es_contract: too many ") + name + " axes");
  g.n = n;
  extent = 1;
  for (int i = 0; i < kMax; ++i) {
    if (i < n) {
      if (axes[i].size < 0) return fail(ES_ERR_INVALID, std::string("es_contract: negative ") + name + " size");
      extent *= uint64_t(axes[i].size);
      if (uint64_t(axes[i].size) > kU32Max) return fail(ES_ERR_UNSUPPORTED, "es_contract: axis too large");
      g.div[i].init(uint32_t(axes[i].size));
      g.sa[i] = axes[i].a;
      g.sb[i] = axes[i].b;
      g.sc[i] = axes[i].c;
    } else {
      g.div[i].init(1);
      g.sa[i] = g.sb[i] = g.sc[i] = 0;
    }
  }
  if (extent > kU32Max) return fail(ES_ERR_UNSUPPORTED, std::string("es_contract: ") + name + " extent >= 2^32");
  return ES_OK;
}

// largest byte offset of an operand: sum over its axes of (size - 1) * |stride|
uint64_t max_offset_bytes(const es_contract_desc* d, int which, int esz) {
  uint64_t off = 0;
  auto add = [&](const es_axis* axes, int n) {
    for (int i = 0; i < n; ++i) {
      const int64_t st = which == 0 ? axes[i].a : axes[i].b;
      if (axes[i].size > 0) off += uint64_t(axes[i].size - 1) * uint64_t(st < 0 ? -st : st);
    }
  };
  add(d->batch, d->n_batch);
  add(which == 0 ? d->m : d->n, which == 0 ? d->n_m : d->n_n);
  add(d->k, d->n_k);
  return off * uint64_t(esz);
}

bool strides_multiple(const es_axis* axes, int n, int skip_last, int which, int64_t q) {
  for (int i = 0; i < n - skip_last; ++i) {
    const int64_t s = which == 0 ? axes[i].a : (which == 1 ? axes[i].b : axes[i].c);
    if (s % q != 0) return false;
  }
  return true;
}

// layout of one operand: `which` 0 = A (rows = M), 1 = B (rows = N)
int operand_layout(const es_contract_desc* d, const void* ptr, int which, int vec, int bk) {
  const es_axis* rows = which == 0 ? d->m : d->n;
  const int nrows = which == 0 ? d->n_m : d->n_n;
  if (!aligned(ptr, 16) || d->n_k == 0) return kGeneric;
  const es_axis& kin = d->k[d->n_k - 1];
  const int64_t kin_stride = which == 0 ? kin.a : kin.b;
  if (kin.size % bk != 0) return kGeneric;
  const bool batch_ok = strides_multiple(d->batch, d->n_batch, 0, which, vec);
  if (!batch_ok) return kGeneric;
  if (kin_stride == 1 && strides_multiple(d->k, d->n_k, 1, which, vec) &&
      strides_multiple(rows, nrows, 0, which, vec))
    return kKContig;
  if (nrows > 0) {
    const es_axis& rin = rows[nrows - 1];
    const int64_t rin_stride = which == 0 ? rin.a : rin.b;
    if (rin_stride == 1 && rin.size % vec == 0 && strides_multiple(rows, nrows, 1, which, vec) &&
        strides_multiple(d->k, d->n_k, 0, which, vec))
      return kMNContig;
  }
  return kGeneric;
}

// N-tiles per tile group (see tile_of in es_contract_kernel.h): each XCD owns
// run = tiles / 8 consecutive logical tiles, a rectangle of group_n N-tiles by
// run / group_n M-tiles when group_n divides tiles_n, run and tiles_m * group_n
// divides into whole runs.  Pick the one touching the fewest A plus B panels.
uint32_t group_width(uint64_t tiles_m, uint64_t tiles_n, uint64_t total) {
  uint32_t best = uint32_t(tiles_n);  // N fastest over the whole row
  if (total % 8 != 0) return best;
  const uint64_t run = total / 8;
  uint64_t best_cost = ~uint64_t(0);
  for (uint64_t gn = 1; gn <= tiles_n; ++gn) {
    if (tiles_n % gn != 0 || run % gn != 0) continue;
    const uint64_t bm = run / gn;
    if ((tiles_m * gn) % run != 0 || bm > tiles_m) continue;
    const uint64_t cost = bm + gn;
    if (cost < best_cost) {
      best_cost = cost;
      best = uint32_t(gn);
    }
  }
  return best;
}

// K walk levels (see ContractArgs::kcnt): level 0 = K tiles of the innermost sub-axis,
// level L = the L-th sub-axis out; advancing at level L resets every level below it.
void k_walk(const es_contract_desc* d, int bk, ContractArgs& p) {
  for (int l = 0; l < kKLevels; ++l) {
    p.kcnt[l] = 0xffffffffu;
    p.kda[l] = p.kdb[l] = 0;
  }
  p.klevels = d->n_k <= 1 ? 1 : (d->n_k == 2 ? 2 : kKLevels);
  if (d->n_k == 0 || d->n_k > kKLevels) return;
  const es_axis& in = d->k[d->n_k - 1];
  const int64_t tiles = in.size / bk;
  int64_t back_a = 0, back_b = 0;  // offset of the last position below the current level
  p.kda[0] = int64_t(bk) * in.a;
  p.kdb[0] = int64_t(bk) * in.b;
  if (d->n_k > 1) p.kcnt[0] = uint32_t(tiles);
  back_a = (tiles - 1) * int64_t(bk) * in.a;
  back_b = (tiles - 1) * int64_t(bk) * in.b;
  for (int l = 1; l < d->n_k; ++l) {
    const es_axis& ax = d->k[d->n_k - 1 - l];
    p.kda[l] = ax.a - back_a;
    p.kdb[l] = ax.b - back_b;
    if (l + 1 < d->n_k) p.kcnt[l] = uint32_t(ax.size);
    back_a += (ax.size - 1) * ax.a;
    back_b += (ax.size - 1) * ax.b;
  }
}

// es_contract_halo's arguments: validate the halo against the descriptor and the
// kernel the contraction takes (the pipelined 16-bit kernel with K-contiguous operands
// on tiles of 256 rows); ES_ERR_UNSUPPORTED when it does not qualify.
int halo_args(const es_contract_desc* d, const es_halo_desc* h, int esz, int la, int lb, int config, int bk,
              ContractArgs& p) {
  const char* who = "es_contract_halo";
  if (h->n < 1 || h->n > 2) return fail(ES_ERR_INVALID, std::string(who) + ": n must be 1 or 2");
  if (d->n_k != h->n + 1)
    return fail(ES_ERR_INVALID, std::string(who) + ": the K group must be the taps followed by the channel");
  for (int s = 0; s < h->n; ++s) {
    const es_halo_dim& g = h->dim[s];
    if (g.m_axis < 0 || g.m_axis >= d->n_m || (s == 1 && g.m_axis == h->dim[0].m_axis))
      return fail(ES_ERR_INVALID, std::string(who) + ": bad m_axis");
    if (g.extent < 1 || g.dilation < 1 || g.pad < 0 || d->k[s].size < 1)
      return fail(ES_ERR_INVALID, std::string(who) + ": bad extent, dilation, pad or tap count");
    if (d->k[s].a != g.dilation * d->m[g.m_axis].a)
      return fail(ES_ERR_INVALID, std::string(who) + ": tap stride must be dilation times the position stride");
  }
  // what the kernel supports
  if (esz != 2 || la != kKContig || lb != kKContig || config != 0 || !p.off32)
    return fail(ES_ERR_UNSUPPORTED, std::string(who) + ": the contraction does not take the pipelined kernel");
  uint64_t span = 1;  // elements up to the last valid input position's channel, plus one
  auto add = [&](const es_axis* axes, int n, bool m_group) {
    for (int i = 0; i < n; ++i) {
      bool spatial = false;
      for (int s = 0; s < h->n && m_group; ++s) spatial = spatial || h->dim[s].m_axis == i;
      if (axes[i].a < 0) return false;
      if (!spatial && axes[i].size > 0) span += uint64_t(axes[i].size - 1) * uint64_t(axes[i].a);
    }
    return true;
  };
  if (!add(d->batch, d->n_batch, false) || !add(d->m, d->n_m, true) || d->k[h->n].a != 1)
    return fail(ES_ERR_UNSUPPORTED, std::string(who) + ": negative strides in A");
  span += uint64_t(d->k[h->n].size - 1);
  int64_t shift = 0;
  for (int s = 0; s < h->n; ++s) {
    const es_halo_dim& g = h->dim[s];
    span += uint64_t(g.extent - 1) * uint64_t(d->m[g.m_axis].a);
    shift += g.pad * d->m[g.m_axis].a;
    if (g.extent > 0xffff || d->m[g.m_axis].size > 0xffff || g.pad > 0xffff || g.dilation * d->k[s].size > 0xffff)
      return fail(ES_ERR_UNSUPPORTED, std::string(who) + ": extents, pads and taps must stay below 65536");
  }
  if (d->k[0].size * (h->n == 2 ? d->k[1].size : 1) > kHaloMaxTaps)
    return fail(ES_ERR_UNSUPPORTED, std::string(who) + ": more than 32 taps");
  const uint64_t span_bytes = span * uint64_t(esz);
  const uint64_t shift_bytes = uint64_t(shift) * uint64_t(esz);
  const uint64_t a_addr = reinterpret_cast<uint64_t>(p.a);
  // every row's offset (positions and taps, read or not) below 2^31 as well: a copy's
  // vector offset then keeps bit 31 free for the outside flag, and adding the K tile's
  // scalar offset cannot wrap
  if (span_bytes + shift_bytes + 64 > uint64_t(kHaloSpanLimit) || a_addr < shift_bytes ||
      max_offset_bytes(d, 0, esz) + 64 > uint64_t(kHaloSpanLimit))
    return fail(ES_ERR_UNSUPPORTED, std::string(who) + ": the input and its halo span 2 GiB or more");
  const int64_t channels = d->k[h->n].size;
  p.halo_n = h->n;
  const uint64_t base = a_addr - shift_bytes;
  p.halo_srd[0] = uint32_t(base);
  p.halo_srd[1] = uint32_t(base >> 32) & 0xffffu;  // stride 0
  p.halo_srd[2] = uint32_t(shift_bytes + span_bytes);
  p.halo_srd[3] = 0x00020000u;                      // 32-bit data format
  p.halo_ctiles.init(uint32_t(channels / bk));
  // slot 1 is the inner dim; a 1-D halo leaves slot 0 always inside
  const int inner = h->n - 1;
  p.halo_taps[1] = int32_t(d->k[inner].size);
  p.halo_taps[0] = h->n == 2 ? int32_t(d->k[0].size) : 1;
  p.halo_dil[1] = int32_t(h->dim[inner].dilation);
  p.halo_pad[1] = int32_t(h->dim[inner].pad);
  p.halo_extent[1] = uint32_t(h->dim[inner].extent);
  p.halo_mlev[1] = h->dim[inner].m_axis;
  if (h->n == 2) {
    p.halo_dil[0] = int32_t(h->dim[0].dilation);
    p.halo_pad[0] = int32_t(h->dim[0].pad);
    p.halo_extent[0] = uint32_t(h->dim[0].extent);
    p.halo_mlev[0] = h->dim[0].m_axis;
  } else {
    p.halo_dil[0] = 0;
    p.halo_pad[0] = 0;
    p.halo_extent[0] = 0xffffffffu;
    p.halo_mlev[0] = -1;
  }
  return ES_OK;
}

}  // namespace
}  // namespace es

namespace es {
namespace {

int contract(const es_contract_desc* d, const void* a, const void* b, const void* bias, void* c, void* stream,
             const es_halo_desc* halo = nullptr) {
  if (d == nullptr) return fail(ES_ERR_INVALID, "es_contract: null descriptor");
  const int esz = dtype_size(d->dtype);
  if (esz == 0) return fail(ES_ERR_UNSUPPORTED, "es_contract: unsupported dtype");

  ContractArgs p;
  uint64_t nb, nm, nn, nk;
  int st;
  if ((st = fill_group(p.gb, d->n_batch, d->batch, nb, "batch")) != ES_OK) return st;
  if ((st = fill_group(p.gm, d->n_m, d->m, nm, "m")) != ES_OK) return st;
  if ((st = fill_group(p.gn, d->n_n, d->n, nn, "n")) != ES_OK) return st;
  if ((st = fill_group(p.gk, d->n_k, d->k, nk, "k")) != ES_OK) return st;
  if (nb * nm * nn == 0) return ES_OK;
  // an empty K reads nothing (torch hands out null data pointers for empty tensors)
  if (c == nullptr || (nk > 0 && (a == nullptr || b == nullptr)))
    return fail(ES_ERR_INVALID, "es_contract: null pointer");
  if (nk > uint64_t(0x7fffffff)) return fail(ES_ERR_UNSUPPORTED, "es_contract: K too large");

  const int vec = 16 / esz;
  const int bk = 128 / esz;  // K tile: 128 bytes per row
  int la = operand_layout(d, a, 0, vec, bk);
  int lb = operand_layout(d, b, 1, vec, bk);
  if (nk == 0) la = lb = kGeneric;  // nothing to load: the generic kernel writes zeros

  p.a = a;
  p.b = b;
  p.c = c;
  p.M = uint32_t(nm);
  p.N = uint32_t(nn);
  p.K = uint32_t(nk);
  p.batch = uint32_t(nb);
  p.ka_inner = d->n_k > 0 ? d->k[d->n_k - 1].a : 0;
  p.kb_inner = d->n_k > 0 ? d->k[d->n_k - 1].b : 0;
  p.bias = bias;
  // an fp32 output is the element type itself for f32 operands
  p.out_f32 = d->out_f32 != 0 && d->dtype != ES_F32 ? 1 : 0;
  // the fast kernels walk K incrementally over at most kKLevels sub-axes
  if (d->n_k > kKLevels) la = lb = kGeneric;
  k_walk(d, bk, p);
  p.off32 = max_offset_bytes(d, 0, esz) + 16 < (uint64_t(1) << 32) && max_offset_bytes(d, 1, esz) + 16 < (uint64_t(1) << 32);
  // vector stores need the output's vectors aligned: 16-byte vectors of the element type,
  // or (out_f32) 4-float runs, whose offsets are then multiples of 8 floats
  p.vstore = 0;
  if (d->n_n > 0) {
    const es_axis& nin = d->n[d->n_n - 1];
    if (nin.c == 1 && nin.size % vec == 0 && aligned(c, 16) && strides_multiple(d->n, d->n_n, 1, 2, vec) &&
        strides_multiple(d->m, d->n_m, 0, 2, vec) && strides_multiple(d->batch, d->n_batch, 0, 2, vec))
      p.vstore = 1;
  }
  // the output contiguous along M instead (contract_pipe stages the tile transposed)
  if (p.vstore == 0 && esz == 2 && d->n_m > 0) {
    const es_axis& min_ = d->m[d->n_m - 1];
    if (min_.c == 1 && min_.size % vec == 0 && aligned(c, 16) && strides_multiple(d->m, d->n_m, 1, 2, vec) &&
        strides_multiple(d->n, d->n_n, 0, 2, vec) && strides_multiple(d->batch, d->n_batch, 0, 2, vec))
      p.vstore = 2;
  }

  // tile: the largest that still gives every CU a tile of its own
  static const int tile_of[3] = {256, 128, 64};
  int config = 2;
  if (la != kGeneric && lb != kGeneric) {
    for (int cfg = 0; cfg < 3; ++cfg) {
      const uint64_t t = uint64_t(tile_of[cfg]);
      const uint64_t tiles = ((nm + t - 1) / t) * ((nn + t - 1) / t) * nb;
      if (tiles >= 256 || cfg == 2) {
        config = cfg;
        break;
      }
    }
  }
  // A 16-bit contraction that contract_pipe can read but with fewer 256-row tiles than
  // CUs: one round of pipelined tiles (some CUs idle) can still beat several rounds of
  // 128 x 128 tiles.  Cycle model per round (MI355X, ~2 GHz under MFMA load): a 64-deep
  // K step of a pipelined 256 x 256 tile takes 2,450 cycles (256 x 224: 7/8 of that plus
  // 5 %) and its prologue and epilogue 23,300; a 128 x 128 tile's step 1,750 and 6,000.
  // Measured: 8192 x 1792 x 4096 took 181 us on 896 tiles of 128 x 128.
  if (config == 1 && esz == 2 && p.off32) {
    const double steps = double((nk + bk - 1) / bk);
    auto rounds = [](uint64_t tiles) { return double((tiles + kCUs - 1) / kCUs); };
    const uint64_t tm256 = (nm + 255) / 256;
    double pipe = rounds(tm256 * ((nn + 255) / 256) * nb) * (2450.0 * steps + 23300.0);
    if (la == kKContig && lb == kKContig)
      pipe = std::min(pipe, rounds(tm256 * ((nn + 223) / 224) * nb) * (2450.0 * 0.875 * 1.05 * steps + 23300.0));
    const double t128 = rounds(((nm + 127) / 128) * ((nn + 127) / 128) * nb) * (1750.0 * steps + 6000.0);
    if (pipe < t128) config = 0;
  }
  const uint64_t t = uint64_t(tile_of[config]);
  const uint64_t tm = (nm + t - 1) / t;
  uint64_t tn = (nn + t - 1) / t;
  // 256 x 224 tiles (contract_pipe) when they take fewer rounds of one tile per CU;
  // a 224-wide tile does 7/8 of the work of a 256-wide one, and its narrower waves read
  // a little more LDS per flop (charged as 5 %)
  p.pipe_bn = 0;
  if (config == 0 && la == kKContig && lb == kKContig && esz == 2 && p.off32) {
    const uint64_t tn224 = (nn + 223) / 224;
    const uint64_t rounds256 = (tm * tn * nb + kCUs - 1) / kCUs;
    const uint64_t rounds224 = (tm * tn224 * nb + kCUs - 1) / kCUs;
    if (rounds224 * 224 * 105 < rounds256 * 256 * 100) {
      p.pipe_bn = 224;
      tn = tn224;
    }
  }
  const uint64_t total = tm * tn * nb;
  if (total > uint64_t(0x7fffffff)) return fail(ES_ERR_UNSUPPORTED, "es_contract: too many tiles");
  p.tiles_m = uint32_t(tm);
  p.tiles_n = uint32_t(tn);
  p.total_tiles = uint32_t(total);
  p.group_n = group_width(tm, tn, total);
  p.tdiv_batch.init(uint32_t(tm * tn));
  p.tdiv_group.init(uint32_t(tm * p.group_n));
  p.tdiv_gn.init(p.group_n);
  {
    const int most = std::max(d->n_batch, std::max(d->n_m, d->n_n));
    p.gdims = most <= 3 ? std::max(most, 1) : 0;
  }
  p.halo_n = 0;
  if (halo != nullptr && (st = halo_args(d, halo, esz, la, lb, config, bk, p)) != ES_OK) return st;

  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (d->dtype) {
    case ES_F32: return launch_contract_f32(p, config, la, lb, s);
    case ES_BF16: return launch_contract_bf16(p, config, la, lb, s);
    case ES_F16: return launch_contract_f16(p, config, la, lb, s);
  }
  return fail(ES_ERR_UNSUPPORTED, "es_contract: unsupported dtype");
}

}  // namespace
}  // namespace es

extern "C" int es_contract(const es_contract_desc* d, const void* a, const void* b, void* c, void* stream) {
  return es::contract(d, a, b, nullptr, c, stream);
}

extern "C" int es_contract_bias(const es_contract_desc* d, const void* a, const void* b, const void* bias, void* c,
                                void* stream) {
  if (bias == nullptr) return es::fail(ES_ERR_INVALID, "es_contract_bias: null bias");
  return es::contract(d, a, b, bias, c, stream);
}

extern "C" int es_contract_halo(const es_contract_desc* d, const es_halo_desc* halo, const void* a, const void* b,
                                const void* bias, void* c, void* stream) {
  if (halo == nullptr) return es::fail(ES_ERR_INVALID, "es_contract_halo: null halo descriptor");
  return es::contract(d, a, b, bias, c, stream, halo);
}
