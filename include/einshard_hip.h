/*
 * einshard_hip.h — C ABI of libeinshard_hip.so, the MI355X (gfx950) kernels
 * behind torch_einshard's single-device path.
 *
 * The reference runs every local einshard through one call,
 *     torch.einsum(equation, *xs)          (reference: src/torch_einshard/einsum.py:132)
 * and every einwindow / einhalo through
 *     F.pad / index_select per axis        (reference: src/torch_einshard/halo.py:27-55)
 *     Tensor.unfold + permute().contiguous()  (reference: src/torch_einshard/halo.py:405-418)
 * The entry points below replace exactly those calls.  The Python layer
 * (torch_einshard.einsum / torch_einshard.halo) parses the expression, lowers it
 * to one of the descriptors here and calls the matching entry point through
 * ctypes; a maintainer binding from another language would do the same.
 *
 * Conventions
 *   - Pointers are device pointers (HIP), sizes and strides are int64 counts of
 *     ELEMENTS.  Outputs are dense in the order the descriptor lists its axes
 *     unless the descriptor carries explicit output strides (es_contract).
 *   - The caller allocates every buffer (inputs, outputs, workspace); the
 *     library never allocates or frees device memory and keeps no pointer
 *     after a call returns.
 *   - `stream` is a hipStream_t (NULL = the null stream).  Work is enqueued
 *     asynchronously; nothing synchronises the device.
 *   - Every entry point returns ES_OK (0) or a negative es_status; a message
 *     describing the last failure on the calling thread is returned by
 *     es_last_error().  Nothing crosses the ABI as a C++ exception.
 *   - Descriptors are plain structs; axes are listed outermost first.
 */
#ifndef EINSHARD_HIP_H
#define EINSHARD_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ES_ABI_VERSION 3
#define ES_MAX_AXES 8 /* sub-axes per descriptor group (after merging) */

typedef enum {
  ES_OK = 0,
  ES_ERR_INVALID = -1,     /* malformed descriptor, null pointer, bad size */
  ES_ERR_UNSUPPORTED = -2, /* well-formed but not implemented (dtype, rank) */
  ES_ERR_LAUNCH = -3,      /* the HIP runtime rejected a launch */
  ES_ERR_WORKSPACE = -4    /* workspace missing or smaller than required */
} es_status;

typedef enum { ES_F32 = 0, ES_BF16 = 1, ES_F16 = 2 } es_dtype;

typedef enum {
  ES_BOUNDARY_CONSTANT = 0,  /* out-of-range reads produce `fill` (F.pad value=) */
  ES_BOUNDARY_REPLICATE = 1, /* clamp the coordinate into [0, size) */
  ES_BOUNDARY_PERIODIC = 2   /* wrap the coordinate modulo size */
} es_boundary;

/* One iteration axis: extent and strides (elements) in the first input (a),
 * the second input (b) and the output (c); 0 = the operand does not vary. */
typedef struct {
  int64_t size;
  int64_t a, b, c;
} es_axis;

/* ---- gather: window / halo / permutation / diagonal ------------------------
 * out is dense over out_size[0..out_rank).  For every output coordinate o and
 * every input dim d:
 *     i_d = o[pos[d]] + (win[d] >= 0 ? o[win[d]] : 0) + offset[d]
 * If some i_d falls outside [0, in_size[d]) the boundary rule applies (per
 * dim, all dims share the rule); with ES_BOUNDARY_CONSTANT the whole element
 * is `fill`.  Otherwise out[o] = x[sum_d i_d * in_stride[d]].
 * win[d] is -1 or an output dim other than pos[d].
 * Elements are copied as raw bits (elem_size 1, 2, 4 or 8 bytes): bit-exact. */
typedef struct {
  int32_t elem_size;
  int32_t boundary;        /* es_boundary */
  uint64_t fill_bits;      /* fill value, low elem_size bytes, already in the element type */
  int32_t out_rank;
  int32_t in_rank;
  int64_t out_size[ES_MAX_AXES];
  int64_t in_size[ES_MAX_AXES];
  int64_t in_stride[ES_MAX_AXES];
  int64_t offset[ES_MAX_AXES];
  int32_t pos[ES_MAX_AXES];
  int32_t win[ES_MAX_AXES];
} es_gather_desc;

/* Replaces: torch.einsum unary permutation/diagonal (einsum.py:132),
 * _pad_dim + unfold + permute().contiguous() (halo.py:27-55, 402-418) and
 * torch.roll per axis (roll.py:27: offset -(shift mod n) with ES_BOUNDARY_PERIODIC). */
int es_gather(const es_gather_desc* desc, const void* x, void* out, void* stream);

/* ---- broadcast elementwise: out = x * y -------------------------------------
 * out is dense over axes[0..rank); axes[i].a / .b are the strides of x / y
 * (0 = broadcast).  Computed in fp32, rounded once to the element type: the
 * same single rounding as torch's mul, hence bit-exact with it. */
typedef struct {
  int32_t dtype; /* es_dtype */
  int32_t rank;
  es_axis axes[ES_MAX_AXES];
} es_bcast_desc;

/* Replaces: torch.einsum binary with no summed label (einsum.py:132, -> at::mul). */
int es_bcast(const es_bcast_desc* desc, const void* x, const void* y, void* out, void* stream);

/* ---- reduction: out[keep] = sum_red x (* y) ------------------------------
 * out is dense over keep[0..n_keep).  With has_y the summand is x*y (a thin
 * contraction: dot products and matrix-vector products).  Accumulates in fp32,
 * one rounding to the element type at the end.  An empty red extent yields 0.
 * Deterministic: the summation order depends only on the descriptor. */
typedef struct {
  int32_t dtype; /* es_dtype of the output (and of x, y unless in_f32) */
  int32_t has_y;
  int32_t n_keep;
  int32_t n_red;
  int32_t in_f32;   /* nonzero: x is fp32 whatever `dtype` is (without y only); the sum of
                       fp32 partial results rounded once to `dtype` */
  int32_t reserved; /* 0 */
  es_axis keep[ES_MAX_AXES]; /* .a = x stride, .b = y stride */
  es_axis red[ES_MAX_AXES];  /* .a = x stride, .b = y stride */
} es_reduce_desc;

/* Bytes of workspace es_reduce needs for this descriptor (0 = none), or a
 * negative es_status for an invalid descriptor. */
int64_t es_reduce_workspace_bytes(const es_reduce_desc* desc);

/* Replaces: torch.einsum unary with summed labels (einsum.py:132, -> at::sum),
 * and thin binary contractions.  `workspace` must hold
 * es_reduce_workspace_bytes(desc) bytes (may be NULL when that is 0). */
int es_reduce(const es_reduce_desc* desc, const void* x, const void* y, void* out,
              void* workspace, int64_t workspace_bytes, void* stream);

/* es_reduce for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart in
 * the reference: it is es_reduce with the same kernels and results, its split partial
 * sums kept in a library-owned device array of ES_NOALLOC_SCRATCH_BYTES per GPU
 * (allocated with the code object, held until the process ends) instead of a
 * workspace argument.  The call itself allocates nothing.  The limit covers every
 * descriptor: es_reduce splits a reduction only while its grid has fewer than 2048
 * work-groups of 64 columns of at most 8 outputs, so its partials stay below
 * 4096 x 64 x 8 x 4 bytes = 8 MiB; a descriptor needing more would return
 * ES_ERR_WORKSPACE before any launch.  The scratch needs no clearing (every partial
 * is written before it is read), keeps the last call's contents, and is shared by
 * every call on that GPU: calls that overlap on one GPU (other streams, other
 * threads, graph replays in flight together) race on it.  The first call on a device
 * looks up the array's address there; make it outside any graph capture.  A captured
 * call replays like any launch. */
#define ES_NOALLOC_SCRATCH_BYTES (8 * 1024 * 1024)
int es_reduce_noalloc(const es_reduce_desc* desc, const void* x, const void* y, void* out, void* stream);

/* ---- contraction: batched GEMM over strided label groups -------------------
 * C[batch, m, n] = sum_k A[batch, m, k] * B[batch, n, k]
 * with every group given as sub-axes (outermost first).  Strides: A uses .a of
 * batch/m/k, B uses .b of batch/n/k, C uses .c of batch/m/n (explicit output
 * strides).  An empty group has extent 1.  bf16/f16 run on
 * v_mfma_f32_16x16x32_{bf16,f16} (large problems; an operand contiguous along M or
 * N is transposed in the LDS read, ds_read_b64_tr_b16) or
 * v_mfma_f32_32x32x16_{bf16,f16}, f32 on v_mfma_f32_32x32x2_f32; fp32
 * accumulation, one rounding of the result.  Operand layouts are read in place
 * (no transposed copy): either the innermost K sub-axis or the innermost M
 * (resp. N) sub-axis may be the contiguous one. */
typedef struct {
  int32_t dtype; /* es_dtype of A and B (and of C unless out_f32) */
  int32_t n_batch, n_m, n_n, n_k;
  int32_t out_f32; /* nonzero: C is written as fp32, unrounded (split-K partial results of
                      16-bit contractions, summed afterwards by es_reduce with in_f32) */
  es_axis batch[ES_MAX_AXES];
  es_axis m[ES_MAX_AXES];
  es_axis n[ES_MAX_AXES];
  es_axis k[ES_MAX_AXES];
} es_contract_desc;

/* Replaces: torch.einsum binary with contracted labels (einsum.py:132 -> bmm). */
int es_contract(const es_contract_desc* desc, const void* a, const void* b, void* c, void* stream);

/* es_contract plus a bias: C[batch, m, n] = sum_k A * B + bias[n], with n the linear
 * index over the N group and bias a dense vector of N elements of the descriptor's
 * dtype, added in fp32 before the one rounding of the result.
 * Replaces: the convolution with bias inside einconv (conv.py:195,
 * F.conv{1,2,3}d(x, weight, bias, padding=0, dilation=...)), which einconv runs as a
 * contraction over an overlapping strided view of the padded input (no im2col). */
int es_contract_bias(const es_contract_desc* desc, const void* a, const void* b, const void* bias, void* c,
                     void* stream);

/* ---- contraction over a zero halo ----------------------------------------------
 * es_contract (es_contract_bias when bias is not null) whose A is read with zero
 * padding instead of from a padded copy: einconv's implicit GEMM straight from its
 * unpadded input.  The K group is exactly the tap sub-axes 0 .. n-1 followed by the
 * channel sub-axis (innermost, unit stride in A).  For spatial dim s, M sub-axis
 * dim[s].m_axis is the output position o_s and K sub-axis s the tap k_s; A's row for
 * (o, k) is input position i_s = o_s + dilation_s * k_s - pad_s, which the descriptor
 * addresses as if no padding existed (A points at input position 0; M stride along
 * o_s = A's stride along the input dim, tap stride = dilation_s times that).  A row
 * with some i_s outside [0, extent_s) reads as zeros.  dim[0] is the outer dim when
 * n = 2.  Only the pipelined 16-bit kernels take it: both operands K-contiguous (16-byte
 * aligned, channel count a multiple of 64), tiles of 256 rows, 32-bit offsets, A's
 * span plus sum(pad_s * stride_s) below 2 GiB, at most 32 taps in all, extents and
 * output positions below 65536.  Otherwise the call returns ES_ERR_UNSUPPORTED and
 * launches nothing.
 * Replaces: F.pad followed by F.conv{1,2}d(padding=0) in einconv (conv.py:185-210),
 * for which einconv otherwise writes a padded copy of its input with es_gather. */
typedef struct {
  int32_t m_axis;   /* index in desc.m of the output position o_s */
  int32_t reserved;
  int64_t extent;   /* input extent along dim s */
  int64_t dilation; /* >= 1 */
  int64_t pad;      /* zeros before input position 0, >= 0 */
} es_halo_dim;

typedef struct {
  int32_t n; /* spatial dims: 1 or 2 */
  int32_t reserved;
  es_halo_dim dim[2];
} es_halo_desc;

int es_contract_halo(const es_contract_desc* desc, const es_halo_desc* halo, const void* a, const void* b,
                     const void* bias, void* c, void* stream);

/* ---- library --------------------------------------------------------------- */
int es_abi_version(void);
const char* es_version(void);
const char* es_last_error(void);
/* Name of the kernel variant the last successful launch on this thread used. */
const char* es_last_kernel(void);

#ifdef __cplusplus
}
#endif

#endif /* EINSHARD_HIP_H */
