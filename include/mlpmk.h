/*
 * mlpmk.h -- C ABI of the MI355X (gfx950) fused softplus-MLP megakernel library
 * (libmlpmk.so).  Plain pointers and sizes only: no C++ types, no exceptions,
 * no torch types cross this boundary.
 *
 * Network: out = softplus(... softplus(x @ W1) ... @ W_{L-1}) @ W_L, no bias,
 * softplus with beta = 1 and threshold = 20, fp16 operands, fp32 accumulation,
 * fp16 output.  Weights are [in, out] row-major fp16, as the reference indexes
 * them (/root/reference/kernel.py:105,109,113-114).
 *
 * Conventions (every entry point):
 *   - Returns an mlpmk_status (0 = success).  Arguments are validated on the
 *     host before anything touches the device; a failed validation launches
 *     nothing.  mlpmk_last_error() gives a per-thread message for the last
 *     failure.
 *   - dims[] has num_layers + 1 entries: dims[0] = D (input features),
 *     dims[1 .. num_layers-1] = hidden widths, dims[num_layers] = OUT.
 *   - All device memory is caller-owned; the library allocates nothing.
 *     Launches are asynchronous on `stream` (a hipStream_t, NULL = the legacy
 *     default stream); nothing synchronises the host.
 *   - Device pointers must be 16-byte aligned (128-bit loads and stores);
 *     every tensor is dense row-major.
 *   - M == 0 is a successful no-op.
 *   - Functions are reentrant; device properties are read lazily, per device.
 */
#ifndef MLPMK_H
#define MLPMK_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum mlpmk_status {
  MLPMK_OK = 0,
  MLPMK_ERR_INVALID_ARG = 1,       /* null pointer, negative size, bad dtype */
  MLPMK_ERR_UNSUPPORTED_SHAPE = 2, /* no kernel instantiated for these dims */
  MLPMK_ERR_MISALIGNED = 3,        /* a pointer is not 16-byte aligned */
  MLPMK_ERR_HIP = 4,               /* a HIP runtime call failed */
  MLPMK_ERR_NO_DEVICE = 5          /* no usable gfx950 device */
} mlpmk_status;

/* Element types.  The forward (mlpmk_fwd) takes fp16, bf16 or fp32 tensors
 * (x, w and out all of that type), and so does the backward (mlpmk_bwd_ws /
 * _noalloc: x, w, dout, dx).  Accumulation, the stash and the weight
 * gradients are fp32 either way.  fp32 tensors run with every MFMA operand
 * split into bf16 hi + lo (products hi*hi + hi*lo + lo*hi): fp32's exponent
 * range and a ~16-bit significand, where the reference's TF32 tl.dot
 * operands keep 10 bits; widths up to 128.  The weight-norm parameters may
 * be fp32, fp16 or bf16.  The reference's kernels take their element type as
 * the INPUT_DTYPE constexpr (/root/reference/mlp_fused.md:159-166). */
enum { MLPMK_DTYPE_F32 = 0, MLPMK_DTYPE_F16 = 1, MLPMK_DTYPE_BF16 = 2 };

/* dout_row_stride of the backward entry points for a dL/dout that is one
 * value everywhere (the gradient of loss = out.sum(), possibly scaled): dout
 * then points at that single element (2-byte aligned).  No counterpart in the
 * reference, whose launcher receives the expanded tensor; it spares callers
 * the copy that would materialise a broadcast row.  Since ABI version 201. */
enum { MLPMK_DOUT_SCALAR = -1 };

/* Flag OR-ed into the dtype argument of mlpmk_bwd / _ws / _noalloc: dw is
 * written (=) instead of accumulated into (+=), so its prior contents do not
 * matter and the caller needs no zero-fill launch before a fresh gradient.
 * The reference's backward produces dW fresh for each step (its autograd
 * function returns the gradients, /root/reference/mlp_fused.md:88-112); the
 * accumulating default is kept for callers that sum several backwards.
 * With M = 0 the written gradient is zero (one clearing launch).  Since ABI
 * version 203. */
enum { MLPMK_BWD_WRITE_DW = 0x100 };

/* Library ABI version (major * 100 + minor). */
int mlpmk_version(void);

/* Static description of a status code. */
const char* mlpmk_status_string(int status);

/* Message describing the last failure on the calling thread ("" if none). */
const char* mlpmk_last_error(void);

/*
 * 1 if a forward kernel exists for (num_layers, dims), else 0.  Host only.
 * Supported: the compiled shapes 3 x 128-wide, 5 x 128-wide and 32-64-64-16,
 * and any network of 2..5 layers whose input and hidden widths are multiples
 * of 16 in [16, 128] and whose output width is in [1, 128] (runtime-width
 * kernels, compiled at width 128 with the true widths as launch parameters;
 * the reference's kernel takes tile-multiple K1, N1, N2 and masks N3,
 * /root/reference/kernel.py:60-63,86-87), and -- for fp16 and bf16 tensors --
 * the same with widths up to 256 (input and hidden multiples of 16 in
 * [16, 256], output in [1, 256]; a streamed-weight kernel: the weights do
 * not fit one workgroup's LDS).
 */
int mlpmk_fwd_supported(int num_layers, const int* dims);

/* mlpmk_fwd_supported for tensors of `dtype` (MLPMK_DTYPE_*): fp32 tensors
 * take the shapes with every width at most 128 (bf16 hi/lo split operands);
 * wider fp32 networks run layer by layer through mlpmk_softplus_f32 and
 * library GEMMs (mlpmk.fallback).  Host only.  Since ABI version 204. */
int mlpmk_fwd_supported_dtype(int num_layers, const int* dims, int dtype);

/* 1 if a backward kernel exists for (num_layers, dims) with 16-bit tensors,
 * else 0.  Host only.  The shapes of mlpmk_fwd_supported with every width at
 * most 128, and those with widths up to 256 (input and hidden multiples of
 * 16) whose output width is a multiple of 8 (the two-pass backward; other
 * wide networks train through the library-GEMM fallback,
 * mlpmk_sigmoid_h_mul). */
int mlpmk_bwd_supported(int num_layers, const int* dims);

/* mlpmk_bwd_supported for tensors of `dtype` (MLPMK_DTYPE_*): fp32 tensors
 * take networks of 2..5 layers with every width at most 128 (input and
 * hidden multiples of 16, output a multiple of 8).  Host only.  Since ABI
 * version 202. */
int mlpmk_bwd_supported_dtype(int num_layers, const int* dims, int dtype);

/*
 * 1 if mlpmk_bwd / mlpmk_bwd_ws accept stash[num_layers-2] == NULL for
 * (num_layers, dims), else 0.  Host only.  The backward then recomputes the
 * last hidden activation h_{L-1} = softplus(h_{L-2} W_{L-2}) at the start of
 * each row block, from the stashed h_{L-2} and W_{L-2}, instead of reading it:
 * the training forward writes, and the backward reads, one fp32 activation
 * block less (M x 512 bytes for the 3-layer 128-wide network, half of its
 * stash) for one more layer of MFMA and softplus work.  The reference lists
 * this trade as future work ("skip saving H in forward, recompute from X +
 * weights in backward", /root/reference/mlp_fused.md:451-452).  Supported:
 * the 3-layer and 5-layer 128-wide networks, with or without dx (the
 * recomputing kernel reads W_{L-2}'s forward operands transposed out of the
 * dgrad copy it stages anyway; 5 layers: mlpmk_bwd_ws / _noalloc).
 */
int mlpmk_bwd_recompute_supported(int num_layers, const int* dims);

/*
 * Forward megakernel (one launch).
 *
 * Replaces the reference's inference launcher `_fused_mlp_fwd(x, w1, w2, w3)`
 * (/root/reference/kernel.py:130-156, kernel /root/reference/kernel.py:60-123)
 * and its training-forward variant that stores the hidden activations
 * (/root/reference/mlp_fused.md:52-61, fp32 storage README.md:30).
 *
 *   dtype  MLPMK_DTYPE_F16, MLPMK_DTYPE_BF16 or MLPMK_DTYPE_F32: element
 *          type of x, w and out (bf16: bf16 MFMA operands, hidden
 *          activations rounded to bf16 between layers, as the reference's
 *          casts to INPUT_DTYPE do; fp32: x, the weights and the hidden
 *          activations split into bf16 hi/lo operand pairs -- fp32's
 *          exponent range, a ~16-bit significand -- and out written in fp32
 *          from the accumulators; widths up to 128)
 *   x      [M, dims[0]]            dtype, device
 *   w[l]   [dims[l], dims[l+1]]    dtype, device, l = 0 .. num_layers-1
 *   out    [M, dims[num_layers]]   dtype, device (written)
 *   stash  NULL for inference, or an array of num_layers-1 device pointers,
 *          stash[l] = h_{l+1} [M, dims[l+1]] fp32 (post-activation, written);
 *          a NULL entry is not written (the recomputing backward below
 *          needs no h_{num_layers-1})
 */
int mlpmk_fwd(int num_layers, const int* dims, int dtype, const void* x, const void* const* w, void* out,
              float* const* stash, int64_t M, void* stream);

/* Forward kernels, as reported by mlpmk_fwd_launch_info. */
enum {
  MLPMK_KERNEL_NONE = -1,          /* M == 0: nothing is launched */
  MLPMK_KERNEL_PERSISTENT = 0,     /* persistent grid, one 32*k-row block per wave at a time */
  MLPMK_KERNEL_FEATURE_SPLIT = 1   /* small batches: the waves of a workgroup share each 32-row block */
};

/*
 * The launch mlpmk_fwd makes for (num_layers, dims, dtype, M, stash != 0) on
 * the current device, without launching: info[0] = kernel (MLPMK_KERNEL_*),
 * info[1] = rows per batch block, info[2] = 64-lane waves per workgroup,
 * info[3] = workgroups in the grid, info[4] = resident workgroups per CU.
 * Needs the device (CU count, occupancy); launches nothing.  The library
 * side of the reference's launch heuristic `_pick_config` (/root/reference/
 * kernel.py:25-53, grid kernel.py:139-142), whose Python mirror kernel.py
 * keeps; it answers from the same code path that mlpmk_fwd launches from.
 */
int mlpmk_fwd_launch_info(int num_layers, const int* dims, int dtype, int64_t M, int stash, int* info);

/*
 * Backward megakernel (one launch): data gradients with MFMA, weight gradients
 * as split-K partials reduced in LDS and then added with global fp32 atomics
 * by every workgroup.  mlpmk_bwd_ws below is the faster form, and the only
 * one for fp32 tensors and widths above 128 (their two-pass backward hands
 * dz between its passes through the workspace): here those return
 * MLPMK_ERR_INVALID_ARG without touching the device.
 *
 * Replaces the fused backward of the reference's `FusedMLPSoftplus` autograd
 * function (/root/reference/mlp_fused.md:88-112, README.md:32) -- the file that
 * held it (fused_mlp.py, README.md:18) is not in the reference snapshot.
 *
 *   dtype            MLPMK_DTYPE_F16, MLPMK_DTYPE_BF16 or MLPMK_DTYPE_F32
 *                    (mlpmk_bwd_ws / _noalloc only): element type of x, w,
 *                    dout and dx
 *   x                [M, dims[0]] dtype
 *   w[l]             as in mlpmk_fwd
 *   stash[l]         h_{l+1} [M, dims[l+1]] fp32, as written by mlpmk_fwd;
 *                    stash[num_layers-2] may be NULL where
 *                    mlpmk_bwd_recompute_supported says so: the kernel then
 *                    recomputes h_{num_layers-1} from h_{num_layers-2}
 *   dout             dL/dout, dtype, row l at dout + l * dout_row_stride
 *                    elements; dout_row_stride = 0 broadcasts one row,
 *                    MLPMK_DOUT_SCALAR one element to every row and column
 *                    (the expanded gradient of loss = out.sum(); aligned to
 *                    its element size), otherwise a multiple of 8 not below
 *                    the output width
 *   dx               NULL, or [M, dims[0]] dtype (written)
 *   dw[l]            [dims[l], dims[l+1]] fp32, ACCUMULATED into (+=); the
 *                    caller zeroes them for a fresh gradient, or passes
 *                    dtype | MLPMK_BWD_WRITE_DW to have them written (=)
 * Networks of 4 and 5 layers are supported through mlpmk_bwd_ws only (they
 * hand dz between two launches through the workspace); here they return
 * MLPMK_ERR_INVALID_ARG without touching the device.
 */
int mlpmk_bwd(int num_layers, const int* dims, int dtype, const void* x, const void* const* w,
              const float* const* stash, const void* dout, int64_t dout_row_stride, void* dx,
              float* const* dw, int64_t M, void* stream);

/*
 * mlpmk_bwd with a caller-provided device workspace (same arguments and
 * results; replaces the same reference interface).  Two forms run behind it:
 *   - the one-pass megakernel (16-bit tensors, widths up to 128, batches
 *     above 16,384 rows, and every recomputing call): each workgroup stores
 *     its weight-gradient partial sums in the workspace with plain stores,
 *     and a second kernel on the same stream sums them into dw (+=, one
 *     thread per element, in a fixed order) instead of every workgroup
 *     adding a whole dW with fp32 atomics (~45-65 us at M = 131072: 256
 *     workgroups x 49152 elements from few CUs each);
 *   - the two-pass backward (fp32 tensors, widths above 128, and 16-bit
 *     batches up to 16,384 rows): a data-gradient kernel over 32-row blocks
 *     of the whole chip writes every dz_l into the workspace, then a
 *     weight-gradient kernel whose workgroups own 64 x 64 blocks of one dW_l
 *     and a chunk of rows adds its tiles to dw with fp32 atomics (summation
 *     order not fixed).
 * Networks of 4 and 5 layers run as two launches (all their dgrad weights
 * and exchange tiles do not fit one workgroup's 160 KiB of LDS): layers
 * L-1..S, whose fp16 gradient of h_S goes through the first M * 256 bytes
 * of the workspace (rounded up to 256) to layers S-1..0; S = 3 for the
 * 5-layer 128-wide network, 2 otherwise.  Numerically the same as one
 * launch: the in-register chain also hands dz on as fp16.
 *   workspace        device memory, 16-byte aligned, at least the size that
 *                    mlpmk_bwd_workspace_size reports for the same
 *                    (num_layers, dims, dtype, M, dx != NULL) on the current
 *                    device;
 *                    free again once both launches have run (stream order)
 */
int mlpmk_bwd_ws(int num_layers, const int* dims, int dtype, const void* x, const void* const* w,
                 const float* const* stash, const void* dout, int64_t dout_row_stride, void* dx,
                 float* const* dw, void* workspace, int64_t workspace_bytes, int64_t M, void* stream);

/* Size of the library-owned scratch array of mlpmk_bwd_noalloc (64 MiB per device). */
#define MLPMK_NOALLOC_SCRATCH_BYTES (64ll << 20)

/*
 * mlpmk_bwd_ws without the workspace argument and without any allocation:
 * the same kernels, with a library-owned device array of
 * MLPMK_NOALLOC_SCRATCH_BYTES per device in place of the caller's workspace.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  It calls no hipMalloc / hipFree.
 *   - Shapes whose workspace (mlpmk_bwd_workspace_size) exceeds
 *     MLPMK_NOALLOC_SCRATCH_BYTES return MLPMK_ERR_UNSUPPORTED_SHAPE before
 *     anything is launched.  What fits: every 3-layer and 2-layer network with
 *     16-bit tensors and widths up to 128 at any M (the partials take at most
 *     48 MiB on MI355X); 4- and 5-layer ones up to the M whose dz hand-over
 *     (M x 256 bytes) still fits (M = 65,536 for the 5-layer 128-wide
 *     network); fp32 tensors and widths above 128 up to the M whose
 *     two-pass dz blocks (M x the hidden widths x the element size) fit
 *     (M = 65,536 for the 3-layer 128-wide network in fp32).
 *   - Every call on a device shares that device's array, and calls that
 *     overlap on one device (two streams) race; calls in one stream order are
 *     safe.  The array keeps the last call's contents; nothing needs to start
 *     at zero.
 *   - The array's device address is looked up once per device, on the first
 *     call on that device.
 */
int mlpmk_bwd_noalloc(int num_layers, const int* dims, int dtype, const void* x, const void* const* w,
                      const float* const* stash, const void* dout, int64_t dout_row_stride, void* dx,
                      float* const* dw, int64_t M, void* stream);

/*
 * Bytes of workspace mlpmk_bwd_ws needs on the current device: for the
 * one-pass megakernel one fp32 copy of all dW blocks per workgroup of the
 * backward grid, plus for 4- and 5-layer networks the dz block of the
 * hand-over between their two launches; for the two-pass backward the dz of
 * every hidden layer ([M, width], element size of dtype); the larger where
 * a call at this M may take either (0 when M == 0).
 */
int mlpmk_bwd_workspace_size(int num_layers, const int* dims, int dtype, int64_t M, int with_dx, int64_t* bytes);

/*
 * Weight-norm forward for all layers in ONE launch:
 *   W_l[:, j] = g_l[j] * v_l[:, j] / ||v_l[:, j]||,   inv_norm_l[j] = 1 / ||v_l[:, j]||
 * Replaces `_wn_fwd_kernel` (/root/reference/mlp_fused.md:473-477; code absent
 * from the snapshot).  v and g live in two contiguous blocks, layer after layer
 * (v_all / g_all, mlp_fused.md:478-480):
 *   param_dtype  MLPMK_DTYPE_F32, _F16 or _BF16: element type of v and g
 *   w_dtype      MLPMK_DTYPE_F16, _BF16 or _F32: element type of w_out
 *   v      sum_l dims[l]*dims[l+1] elements of param_dtype, layer l = [dims[l], dims[l+1]]
 *   g      sum_l dims[l+1] elements of param_dtype
 *   w_out  same element layout as v, w_dtype (written)
 *   inv_norm  sum_l dims[l+1] fp32 (written)
 */
int mlpmk_wn_fwd(int num_layers, const int* dims, int param_dtype, int w_dtype, const void* v, const void* g,
                 void* w_out, float* inv_norm, void* stream);

/*
 * Weight-norm backward for all layers in ONE launch, reading the fp32 weight
 * gradient in its [in, out] layout column-wise (no transposed copy):
 *   u = v * inv_norm,  dg[j] = <dW[:, j], u[:, j]>,
 *   dv[:, j] = g[j] * inv_norm[j] * (dW[:, j] - dg[j] * u[:, j])
 * Replaces `_wn_bwd_from_dw_T_kernel` (/root/reference/mlp_fused.md:474,481-483).
 *   dw        fp32, same element layout as v (one block, layer after layer)
 *   dv, dg    param_dtype, layouts of v and g (written)
 */
int mlpmk_wn_bwd(int num_layers, const int* dims, int param_dtype, const float* dw, const void* v,
                 const void* g, const float* inv_norm, void* dv, void* dg, void* stream);

/*
 * The elementwise step of the reference's large-M backward fallback, its fused
 * `sigmoid_h_mul` kernel (/root/reference/mlp_fused.md:114-146):
 *   dz[i] = dh[i] * (1 - exp(-h[i])),  i < n
 * h is the fp32 activation stash, dh the data gradient of the layer above
 * (dh_dtype fp32, fp16 or bf16).  dz32 receives dz in fp32 (for the fp32
 * weight-gradient GEMM); dz16, if not NULL, the same values rounded to
 * dz16_dtype (fp16 or bf16, for the next data-gradient GEMM).  The library
 * GEMMs around it (rocBLAS / hipBLASLt through torch) complete the fallback
 * backward in mlpmk.fallback; the fused backward megakernel (mlpmk_bwd_ws) is
 * the default path at every M.
 */
int mlpmk_sigmoid_h_mul(const float* h, const void* dh, int dh_dtype, float* dz32, void* dz16, int dz16_dtype,
                        int64_t n, void* stream);

/*
 * The softplus of the reference's eager forward (/root/reference/kernel.py:168-171,
 * torch's softplus: beta 1, threshold 20), elementwise in fp32:
 *   h[i] = z[i] > 20 ? z[i] : log(1 + exp(z[i])),  i < n   (h may be z)
 * evaluated as max(z, 0) + log1p(exp(-|z|)) to a few fp32 ulp.  The
 * per-layer step of the library-GEMM forward in mlpmk.fallback, which runs
 * fp32 tensors for networks the fused fp32 forward does not take (widths
 * above 128), as the reference's INPUT_DTYPE = fp32 kernels take any width
 * (mlp_fused.md:159-166).  z and h 16-byte aligned.  Since ABI version 204.
 */
int mlpmk_softplus_f32(const float* z, float* h, int64_t n, void* stream);

/*
 * Diagnostic: a streaming copy of `bytes` bytes (multiple of 16) with the same
 * 128-bit load/store width and cache policy as the forward megakernel's x and
 * out traffic (default loads, non-temporal stores).  Used to calibrate
 * hardware byte counters (FETCH_SIZE / WRITE_SIZE) against a known size and
 * as the benchmark's achievable-HBM reference.  No counterpart in the
 * reference.
 */
int mlpmk_copy(const void* src, void* dst, int64_t bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MLPMK_H */
