/*
 * libnova_winograd.so -- C-ABI of the MI355X-native NOVA F(6,3) Winograd
 * convolution (3x3, stride 1, fp16 activations, fp32 weights).
 *
 * Every symbol the reference's ctypes bridge binds
 * (/root/reference/nova_winograd/ops.py:66-114) is declared here with the
 * reference's exact C signature (/root/reference/csrc/nova_winograd.hip:679-758),
 * so the reference's Python package, or any ctypes/cffi/C caller written
 * against it, binds this library unchanged. Extensions follow, each marked.
 *
 * Conventions (same as the reference):
 *   - all data pointers are device pointers owned by the caller;
 *   - x is fp16 NCHW [B][C][H][W], contiguous; w is fp32 [K][C][3][3];
 *     y is fp16 NCHW [B][K][Ho][Wo] with Ho = H + 2*pad - 2;
 *   - functions return void; failures no longer exit the process (the
 *     reference calls exit(1)): they leave the output untouched, record a
 *     code and message, and nova_get_last_error() reports them.
 * Streams: work of a handle goes to the stream set with nova_set_stream()
 * (default: the null stream, as in the reference). Handle-less entry points
 * (nova_filter_transform, nova_input_transform, nova_output_transform) use
 * the null stream, as in the reference.
 */
#ifndef NOVA_WINOGRAD_H
#define NOVA_WINOGRAD_H

#if defined(__GNUC__)
#define NOVA_API __attribute__((visibility("default")))
#else
#define NOVA_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

typedef void* nova_handle_t;

/* ---- Reference C-ABI (12 symbols) ---------------------------------------- */

/* Replaces nova_create, /root/reference/csrc/nova_winograd.hip:686-690.
 * No device work: the transform tables are compiled into the kernels. */
NOVA_API nova_handle_t nova_create(void);

/* Replaces nova_destroy, /root/reference/csrc/nova_winograd.hip:692-694.
 * Frees the handle's filter transform and workspace; NULL is a no-op. */
NOVA_API void nova_destroy(nova_handle_t h);

/* Replaces nova_set_weights, /root/reference/csrc/nova_winograd.hip:696-698.
 * Transforms fp32 w[K][C][3][3] into the handle's Winograd-domain filter
 * (asynchronous on the handle's stream). */
NOVA_API void nova_set_weights(nova_handle_t h, const void* d_weight, int K, int C);

/* Replaces nova_forward, /root/reference/csrc/nova_winograd.hip:700-706.
 * Uses a handle-owned, grow-only workspace (the reference mallocs and frees
 * per call). */
NOVA_API void nova_forward(nova_handle_t h, const void* d_input, void* d_output, int batch, int H,
                  int W, int pad);

/* Replaces nova_forward_workspace, /root/reference/csrc/nova_winograd.hip:708-717.
 * d_V_gemm / d_M_gemm are caller workspaces of at least 64*C*BP and 64*K*BP
 * fp16 elements, BP = batch*nh*nw with (nh, nw) from nova_compute_tiling.
 * They are used when large enough for the internal layout, otherwise the
 * handle's own workspace is used; their contents afterwards are unspecified. */
NOVA_API void nova_forward_workspace(nova_handle_t h, const void* d_input, void* d_output,
                            void* d_V_gemm, void* d_M_gemm, int batch, int H, int W, int pad,
                            int nh, int nw);

/* Replaces nova_compute_tiling, /root/reference/csrc/nova_winograd.hip:719-721
 * (law :617-631): Ho = H+2p-2; nh = ceil((Ho-1)/6)+1. Host-only, no device. */
NOVA_API void nova_compute_tiling(int H, int W, int pad, int* nh, int* nw, int* H_out, int* W_out);

/* Replaces nova_filter_transform, /root/reference/csrc/nova_winograd.hip:724-728.
 * Writes U in the reference layout U[p*K*C + c*K + k] and synchronizes. */
NOVA_API void nova_filter_transform(const void* d_weight, void* d_U_gemm, int K, int C);

/* Replaces nova_input_transform, /root/reference/csrc/nova_winograd.hip:731-739.
 * Writes V in the reference layout V[p*C*BP + bp*C + c], bp = b*nh*nw + tile. */
NOVA_API void nova_input_transform(const void* d_input, void* d_V_gemm, int batch, int C, int H, int W,
                          int pad, int nh, int nw, int BP);

/* Replaces nova_output_transform, /root/reference/csrc/nova_winograd.hip:742-750.
 * Reads M in the reference layout M[p*K*BP + bp*K + k]. */
NOVA_API void nova_output_transform(const void* d_M_gemm, void* d_output, int batch, int K, int H_out,
                           int W_out, int nh, int nw, int BP);

/* Replace nova_get_K / nova_get_C / nova_get_U_gemm,
 * /root/reference/csrc/nova_winograd.hip:752-754. The U pointer refers to
 * this library's layout U[p][k][Cp] (Cp = C rounded up to 8, zero padded). */
NOVA_API int nova_get_K(nova_handle_t h);
NOVA_API int nova_get_C(nova_handle_t h);
NOVA_API void* nova_get_U_gemm(nova_handle_t h);

/* ---- Reference fused C-API (declared in the reference, never bound) ------ */
/* Replace nova_fused_create/destroy/set_weights/forward/compute_tiling,
 * /root/reference/csrc/nova_winograd_fused.hip:619-652. They are the same
 * handle as above; the fused/3-pass choice is made per call. */
NOVA_API nova_handle_t nova_fused_create(void);
NOVA_API void nova_fused_destroy(nova_handle_t h);
NOVA_API void nova_fused_set_weights(nova_handle_t h, const void* d_weight, int K, int C);
NOVA_API void nova_fused_forward(nova_handle_t h, const void* d_input, void* d_output, int batch, int H,
                        int W, int pad);
NOVA_API void nova_fused_compute_tiling(int H, int W, int pad, int* nh, int* nw, int* H_out, int* W_out);

/* ---- Extensions (no reference counterpart) ------------------------------- */

/* Last error of the calling thread: returns the code (0 = none) and clears it. */
NOVA_API int nova_get_last_error(void);
/* Message for the calling thread's most recent error ("" if none). */
NOVA_API const char* nova_get_last_error_message(void);

/* No counterpart in the reference: nova_set_weights for fp16 w[K][C][3][3],
 * so that a module converted with .half() passes its weights without an fp32
 * copy (the reference reads such weights as fp32 bits). Each weight widens to
 * fp32 exactly: the transform equals nova_set_weights on the fp32 copy, bit
 * for bit. */
NOVA_API void nova_set_weights_f16(nova_handle_t h, const void* d_weight_f16, int K, int C);

/* No counterpart in the reference's C-ABI: the weight gradient, which the
 * reference computes in fp32 PyTorch with a per-sample unfold loop
 * (/root/reference/nova_winograd/conv2d.py:121-147). d_grad_weight receives
 * fp32 dL/dw [K][C][3][3] (overwritten) for x fp16 [B][C][H][W] and
 * d_grad_output [B][K][Ho][Wo] (fp16, or fp32 when grad_f32 = 1), NCHW,
 * padding pad. Computed on the Winograd domain in fp32 (the products reduced
 * over the tiles, deterministic), on the handle's stream with the handle's
 * workspace; the handle needs no weights. batch = 0 writes zeros. */
NOVA_API void nova_weight_grad(nova_handle_t h, const void* d_input, const void* d_grad_output,
                               void* d_grad_weight, int batch, int C, int K, int H, int W,
                               int pad, int grad_f32);

/* Stream for the handle's subsequent work (a hipStream_t; NULL = null stream). */
NOVA_API void nova_set_stream(nova_handle_t h, void* stream);

/* Path selection: 0 = automatic (default), 1 = force 3-pass, 2 = force the
 * fused kernel split by position row (small batches), 3 = force the fused
 * tile-block kernel (few channels, batch > 1), 5 = force the small-problem
 * fused kernel (C, K <= 128: one launch of 2 tiles x 16 output channels per
 * workgroup; chosen automatically for C, K <= 64 while its grid is at most
 * two workgroups per CU, e.g. batch 1), 6 = force the two-pass path (the
 * input transform, then the 64 products and the output transform in one
 * launch of 16 tiles x 32 output channels per workgroup, M kept on chip;
 * bit-identical to 3-pass), 7 = force the input transform fused into the
 * products (few tiles: at most 64 per sub-batch, at most 512 input channels,
 * pads up to 4; each workgroup builds the row of the transformed input its
 * products need from x, M goes to memory and the output transform follows:
 * two launches instead of three, bit-identical to 3-pass; chosen
 * automatically for at most 32 tiles and 128 output channels, e.g. batch 1
 * at ResNet-50 conv3_x), 4 = windowed 3-pass: the batch
 * runs in windows of whole images whose V + M fit the window budget
 * (nova_set_window_bytes), each window's three kernels back to back -- the
 * BP-windowed pipeline of /root/reference/tests/test_bp_tiled.hip:482-571,
 * never chosen automatically. A forced fused path outside its envelope runs
 * 3-pass and reports an error. The fused kernels read a second, fragment-
 * ordered copy of the transformed filter (device memory the size of U); a
 * handle builds it in nova_set_weights when a fused kernel can run (C, K <= 64
 * on the automatic path, or 2 / 3 / 5 already forced), here when 2, 3 or 5 is
 * forced after the weights, and otherwise never. */
NOVA_API void nova_set_path(nova_handle_t h, int path);
/* V + M bytes per window of path 4 (0 = default, 4 MiB, the reference's
 * budget; at least one image per window). No counterpart in the reference,
 * whose window size is computed inline (test_bp_tiled.hip:613-614). */
NOVA_API void nova_set_window_bytes(nova_handle_t h, long long bytes);
/* Output epilogue of every subsequent forward on the handle: d_bias_f16 is a
 * device array of K fp16 values added per output channel (NULL: none), with
 * the rounding of the reference's separate `y + bias.half()`; relu = 1 clamps
 * negative outputs to zero. No counterpart in the reference, whose bias is a
 * separate elementwise op after the convolution
 * (/root/reference/nova_winograd/conv2d.py:240-241). */
NOVA_API void nova_set_epilogue(nova_handle_t h, const void* d_bias_f16, int relu);
/* Activation layout of every subsequent forward on the handle: 0 = NCHW
 * (default, the reference's), 1 = NHWC (channels last): x is [B][H][W][C]
 * and y (and a residual) [B][Ho][Wo][K]. NHWC runs the three-pass pipeline
 * with channels-last transform kernels or, where it fits (C % 8 == 0 and a
 * 16-byte aligned x), the tile-block fused kernel; the position-row fused
 * kernel is NCHW only (path 2 runs 3-pass). Results equal the NCHW path's of
 * the same kind, bit for bit, in the other layout. No counterpart in the
 * reference. */
NOVA_API void nova_set_layout(nova_handle_t h, int nhwc);
/* Residual of every subsequent forward on the handle: an fp16 tensor with the
 * output's shape and layout [B][K][Ho][Wo], added after the bias and before
 * the ReLU (each add rounded to fp16, as separate `y + bias.half()` and
 * `y + residual` ops); NULL: none. It is a per-call operand: set it before
 * each forward that uses it and clear it after. No counterpart in the
 * reference (a residual there is a separate elementwise op). */
NOVA_API void nova_set_residual(nova_handle_t h, const void* d_residual_f16);
/* Path the most recent forward on this handle took: 1 = 3-pass, 2 = fused
 * (position rows), 3 = fused (tile blocks), 4 = windowed 3-pass, 5 = fused
 * (small problems), 6 = two-pass (input transform + products with the output
 * transform). */
NOVA_API int nova_get_last_path(nova_handle_t h);

/* No counterpart in the reference. nova_forward for callers that cannot
 * allocate device memory: code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc. Nothing is allocated: the three-pass
 * workspace is a scratch array of NOVA_NOALLOC_SCRATCH_BYTES compiled into
 * the library (one copy per GPU, held until the process ends), batches are
 * split so every launch fits it, and a shape whose single image needs more
 * workspace than that is refused (error 4, output untouched). The result is
 * nova_forward's bit for bit when both run the same sub-batches; where the
 * scratch splits a batch that nova_forward runs whole, the GEMM's tile
 * follows the smaller launch and the outputs agree within fp32 accumulation
 * order (the same rounding points, M summed in another order). Every call on a GPU shares that
 * GPU's scratch: calls that overlap on one GPU (unordered streams, other host
 * threads) race. The position-row fused path needs allocated scratch and is
 * never taken here (a forced path 2 runs three-pass and reports it); the
 * fused and path-7 kernels run only once a forward with allocation has built
 * their copy of the transformed filter (else three-pass, the same bits for
 * path 7); and these calls are not timed by nova_profile_enable. */
#define NOVA_NOALLOC_SCRATCH_BYTES (64ll << 20)
NOVA_API void nova_forward_noalloc(nova_handle_t h, const void* d_input, void* d_output, int batch,
                                   int H, int W, int pad);

/* Internal workspace bytes a forward of this shape needs on this handle. */
NOVA_API long long nova_workspace_bytes(nova_handle_t h, int batch, int H, int W, int pad);

/* Per-kernel timing for measurement. enable != 0 times each kernel of every
 * forward on the handle with a pair of hipEvents that the kernel's own
 * dispatch packet records (hipExtLaunchKernelGGL start/stop events), so the
 * interval is the kernel's execution alone (at most 4096 three-kernel
 * forwards between reads); nova_profile_read() waits for them, writes the
 * total ms and launch count per kernel kind (0 input transform, 1 GEMM,
 * 2 output transform, 3 fused) and resets. Returns the number of timed
 * launches. */
NOVA_API void nova_profile_enable(nova_handle_t h, int enable);
NOVA_API int nova_profile_read(nova_handle_t h, double* total_ms, long long* count);
/* Re-launches the kernel of `kind` from the handle's most recent forward
 * (first sub-batch) `reps` times back to back on the handle's stream, timed by
 * one hipEvent pair around the loop; returns the mean ms per launch (< 0 on
 * error). The kernels are idempotent, so outputs are unchanged. Measurement
 * only: the buffers of that forward must still be alive. */
NOVA_API double nova_profile_replay(nova_handle_t h, int kind, int reps);
/* Name of the kernel last timed for a kind (e.g. "wgemm_kernel<2, 2, 2, 2>"). */
NOVA_API const char* nova_profile_kernel_name(nova_handle_t h, int kind);

/* Library version string. */
NOVA_API const char* nova_version(void);

#ifdef __cplusplus
}
#endif

#endif /* NOVA_WINOGRAD_H */
