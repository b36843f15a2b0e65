/*
 * Brute-force CPU restatements used to pin the oracle — TEST INFRASTRUCTURE.
 *
 * brute_einsum: exhaustive fp64 einsum.  Every combination of every label is
 *   visited (an odometer over all labels); each operand is read through its
 *   own per-dim label and element stride, so a label repeated inside one
 *   operand walks its diagonal and a stride of 0 broadcasts.  The product of
 *   the operands is added to the output element named by the output labels.
 *   Cost is the product of all label sizes: tiny shapes only.
 *
 * brute_window: the closed form of einwindow / einhalo
 *   (reference src/torch_einshard/halo.py:347-418 and :27-55):
 *     out[o] = x[c_0, ..., c_{r-1}],  c_d = o[pos[d]] + (win[d] >= 0 ? o[win[d]] : 0) - left[d]
 *   with a coordinate outside [0, n_d) replaced by `fill` (constant), clamped
 *   (replicate) or wrapped (periodic).  Elements are copied as raw bytes.
 */
#include <stdint.h>
#include <string.h>

#define BR_MAX 16

static double load_as_f64(const void* base, int64_t index, int dtype) {
  switch (dtype) {
    case 0: return (double)((const float*)base)[index];
    case 1: { /* bfloat16 */
      uint32_t bits = (uint32_t)((const uint16_t*)base)[index] << 16;
      float f;
      memcpy(&f, &bits, 4);
      return (double)f;
    }
    case 2: { /* float16 */
      uint16_t h = ((const uint16_t*)base)[index];
      int sign = h >> 15, exp = (h >> 10) & 0x1f, man = h & 0x3ff;
      double v;
      if (exp == 0) v = man * (1.0 / (1 << 24));
      else if (exp == 31) v = man ? (0.0 / 0.0) : (1.0 / 0.0);
      else v = (1.0 + man / 1024.0) * (double)(1LL << exp) / (double)(1LL << 15);
      return sign ? -v : v;
    }
    default: return ((const double*)base)[index];
  }
}

/* labels_in: n_inputs x BR_MAX label ids; strides_in: n_inputs x BR_MAX.
 * Returns 0, or -1 on a bad argument. */
int brute_einsum(int n_labels, const int64_t* label_size, int n_inputs, const int* in_rank, const int* labels_in,
                 const int64_t* strides_in, const void* const* data, const int* dtype, int out_rank,
                 const int* out_labels, double* out) {
  if (n_labels < 0 || n_labels > BR_MAX || n_inputs < 1 || n_inputs > 2 || out_rank < 0 || out_rank > BR_MAX)
    return -1;
  int64_t out_count = 1;
  for (int i = 0; i < out_rank; ++i) out_count *= label_size[out_labels[i]];
  for (int64_t i = 0; i < out_count; ++i) out[i] = 0.0;
  int64_t total = 1;
  for (int l = 0; l < n_labels; ++l) {
    if (label_size[l] == 0) return 0;
    total *= label_size[l];
  }
  int64_t idx[BR_MAX] = {0};
  for (int64_t step = 0; step < total; ++step) {
    double prod = 1.0;
    for (int t = 0; t < n_inputs; ++t) {
      int64_t off = 0;
      for (int d = 0; d < in_rank[t]; ++d) off += idx[labels_in[t * BR_MAX + d]] * strides_in[t * BR_MAX + d];
      prod *= load_as_f64(data[t], off, dtype[t]);
    }
    int64_t o = 0;
    for (int i = 0; i < out_rank; ++i) o = o * label_size[out_labels[i]] + idx[out_labels[i]];
    out[o] += prod;
    for (int l = n_labels - 1; l >= 0; --l) { /* odometer, last label fastest */
      if (++idx[l] < label_size[l]) break;
      idx[l] = 0;
    }
  }
  return 0;
}

int brute_window(int elem_size, int in_rank, const int64_t* in_size, const int64_t* in_stride, int out_rank,
                 const int64_t* out_size, const int* pos, const int* win, const int64_t* left, int boundary,
                 const void* fill, const void* x, void* out) {
  if (in_rank < 0 || in_rank > BR_MAX || out_rank < 1 || out_rank > BR_MAX) return -1;
  int64_t total = 1;
  for (int i = 0; i < out_rank; ++i) total *= out_size[i];
  int64_t o[BR_MAX] = {0};
  const unsigned char* src = (const unsigned char*)x;
  unsigned char* dst = (unsigned char*)out;
  for (int64_t e = 0; e < total; ++e) {
    int outside = 0;
    int64_t off = 0;
    for (int d = 0; d < in_rank; ++d) {
      int64_t c = o[pos[d]] - left[d];
      if (win[d] >= 0) c += o[win[d]];
      const int64_t n = in_size[d];
      if (c < 0 || c >= n) {
        if (boundary == 1) c = c < 0 ? 0 : n - 1;
        else if (boundary == 2) { c %= n; if (c < 0) c += n; }
        else outside = 1;
      }
      off += c * in_stride[d];
    }
    memcpy(dst + e * elem_size, outside ? (const unsigned char*)fill : src + off * elem_size, (size_t)elem_size);
    for (int i = out_rank - 1; i >= 0; --i) {
      if (++o[i] < out_size[i]) break;
      o[i] = 0;
    }
  }
  return 0;
}
