/*
 * nt_mi355x.h — C ABI of the MI355X (gfx950) kernel library libnt_mi355x.so.
 *
 * This library stands where the reference's generated launchers stand: the
 * Triton launch_<name> (reference src/ninetoothed/backends/emitters/triton.py:683-693)
 * and the CUDA backend's `extern "C" int launch_<name>(ptrs..., int64 dims..., stream)`
 * (reference src/ninetoothed/backends/emitters/cuda.py:362-380), bound from Python
 * with ctypes exactly as reference src/ninetoothed/backends/materializers/cuda.py:96-130
 * binds its library.
 *
 * Conventions shared by every entry point:
 *   - device pointers are `const void*` (inputs) and `void*` (outputs);
 *   - sizes and strides are int64_t and counted in ELEMENTS, not bytes;
 *     4-D strides are passed as a host pointer to four int64_t values;
 *   - the stream is the last argument and every launch is asynchronous on it;
 *   - the return value is a hipError_t as int: 0 = success, a launch or runtime
 *     error otherwise, and NT_ERR_INVALID (= hipErrorInvalidValue) when the
 *     arguments are rejected before anything is launched (null pointers,
 *     negative sizes, unsupported dtype codes, index ranges beyond int32 where a
 *     kernel indexes in 32 bits);
 *   - an empty problem (any size 0) launches nothing and returns 0, as the
 *     reference's runtime does (reference src/ninetoothed/compiler/runtime.py:1411-1422);
 *   - the library never allocates device memory: callers own every buffer,
 *     including the optional conv2d workspace.
 */
#ifndef NT_MI355X_H
#define NT_MI355X_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NT_ABI_VERSION 1
#define NT_ERR_INVALID 1

/* Element type codes for arguments whose type differs from the entry point's. */
#define NT_DTYPE_NONE (-1)
#define NT_DTYPE_F32 0
#define NT_DTYPE_F16 1
#define NT_DTYPE_BF16 2
#define NT_DTYPE_E5M2 3 /* GEMM bias (c) only: OCP float8_e5m2 */
#define NT_DTYPE_E4M3 4 /* GEMM bias (c) only: OCP float8_e4m3fn */

/* Manifest check: returns NT_ABI_VERSION. Replaces the reference's ABI field of
 * its built manifest (reference src/ninetoothed/compiler/runtime.py:1485-1503). */
int nt_abi_version(void);

/* ---------------------------------------------------------------------------
 * Elementwise add: out[i] = lhs[i] + rhs[i] for i < n, each operand addressed as
 * base + i * stride.  Replaces the launcher of the `add_kernel` application
 * (reference tests/test_add.py:9-24; elementwise-grid program,
 * src/ninetoothed/backends/emitters/triton.py:518, 592-594).
 * ------------------------------------------------------------------------- */
int nt_add_f32(const void* lhs, int64_t lhs_stride, const void* rhs, int64_t rhs_stride,
               void* out, int64_t out_stride, int64_t n, hipStream_t stream);
int nt_add_f16(const void* lhs, int64_t lhs_stride, const void* rhs, int64_t rhs_stride,
               void* out, int64_t out_stride, int64_t n, hipStream_t stream);
int nt_add_bf16(const void* lhs, int64_t lhs_stride, const void* rhs, int64_t rhs_stride,
                void* out, int64_t out_stride, int64_t n, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Row softmax over segments: every row of the [rows, cols] input is cut into
 * segments of `block` columns (the application's BLOCK_SIZE constexpr) and each
 * segment is normalised on its own: y = exp(x - max) / sum(exp(x - max)), with
 * columns past the row end taking the value -inf.  block >= cols gives the usual
 * full-row softmax.  Math in fp32, result rounded to the element type.
 * Replaces the launcher of `softmax_kernel` (reference tests/test_softmax.py:10-27;
 * row-vector schedule, src/ninetoothed/materializers/triton.py:1299-1314).
 * Any strides: a column stride other than 1 takes an element-wise kernel.
 * ------------------------------------------------------------------------- */
int nt_softmax_f32(const void* x, int64_t x_row_stride, int64_t x_col_stride,
                   void* y, int64_t y_row_stride, int64_t y_col_stride,
                   int64_t rows, int64_t cols, int64_t block, hipStream_t stream);
int nt_softmax_f16(const void* x, int64_t x_row_stride, int64_t x_col_stride,
                   void* y, int64_t y_row_stride, int64_t y_col_stride,
                   int64_t rows, int64_t cols, int64_t block, hipStream_t stream);
int nt_softmax_bf16(const void* x, int64_t x_row_stride, int64_t x_col_stride,
                    void* y, int64_t y_row_stride, int64_t y_col_stride,
                    int64_t rows, int64_t cols, int64_t block, hipStream_t stream);

/* One kernel configuration of the softmax, for the auto-tuner: the arguments of
 * nt_softmax_* plus `config` (0 = as nt_softmax_* choose; 1, 2, 3 = the register path
 * with workgroups of four, eight, one wave, when the segment fits it; 4 = the two-sweep
 * kernel; 5 = a group of lanes per segment, up to four 16-byte vectors per lane of one
 * wave; 6 = the element-wise kernel for any strides).  A forced configuration that does
 * not fit returns NT_ERR_INVALID before launching.  Replaces the reference's tuning over num_warps 4, 8, 1
 * (reference src/ninetoothed/backends/triton.py:151-155). */
int nt_softmax_config_f32(const void* x, int64_t x_row_stride, int64_t x_col_stride,
                          void* y, int64_t y_row_stride, int64_t y_col_stride,
                          int64_t rows, int64_t cols, int64_t block, hipStream_t stream, int config);
int nt_softmax_config_f16(const void* x, int64_t x_row_stride, int64_t x_col_stride,
                          void* y, int64_t y_row_stride, int64_t y_col_stride,
                          int64_t rows, int64_t cols, int64_t block, hipStream_t stream, int config);
int nt_softmax_config_bf16(const void* x, int64_t x_row_stride, int64_t x_col_stride,
                           void* y, int64_t y_row_stride, int64_t y_col_stride,
                           int64_t rows, int64_t cols, int64_t block, hipStream_t stream, int config);

/* Softmax with input and output of any two element types (x_dtype, y_dtype: NT_DTYPE_F32,
 * F16 or BF16): the reference's kernel takes strides as arguments and its store casts the
 * fp32 quotient to the output's type (reference tests/test_softmax.py:13-21,
 * src/ninetoothed/frontend/types.py:319-324), so an fp16 input with an fp32 output is a
 * valid program.  Equal types behave as nt_softmax_*; others take the element-wise
 * kernel (any strides).  Other arguments as nt_softmax_*. */
int nt_softmax_cast(const void* x, int x_dtype, int64_t x_row_stride, int64_t x_col_stride,
                    void* y, int y_dtype, int64_t y_row_stride, int64_t y_col_stride,
                    int64_t rows, int64_t cols, int64_t block, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * 2-D max pooling on an N-C-H-W indexed input:
 *   y[n,c,p,q] = max over r < kh, s < kw of x[n, c, p*sh - ph + r*dh, q*sw - pw + s*dw],
 * where positions outside [0,H) x [0,W) read -inf (the arrangement's
 * `other=float("-inf")`).  Bit-exact: max involves no rounding.
 * Replaces the launcher of the max_pool2d application
 * (reference tests/test_max_pool2d.py:13-36; tile(..., floor_mode) semantics
 * src/ninetoothed/tensor.py:200-286).
 * ------------------------------------------------------------------------- */
int nt_max_pool2d_f32(const void* x, const int64_t* x_strides, void* y, const int64_t* y_strides,
                      int64_t N, int64_t C, int64_t H, int64_t W, int64_t P, int64_t Q,
                      int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
                      int64_t dh, int64_t dw, hipStream_t stream);
int nt_max_pool2d_f16(const void* x, const int64_t* x_strides, void* y, const int64_t* y_strides,
                      int64_t N, int64_t C, int64_t H, int64_t W, int64_t P, int64_t Q,
                      int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
                      int64_t dh, int64_t dw, hipStream_t stream);
int nt_max_pool2d_bf16(const void* x, const int64_t* x_strides, void* y, const int64_t* y_strides,
                       int64_t N, int64_t C, int64_t H, int64_t W, int64_t P, int64_t Q,
                       int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
                       int64_t dh, int64_t dw, hipStream_t stream);

/* One kernel configuration of max_pool2d, for the auto-tuner: the arguments of
 * nt_max_pool2d_* plus `config` (0 = as nt_max_pool2d_* choose; 1 = the vector kernels:
 * 16-bit, 2-wide windows of stride 2 inside the input, unit inner strides, 16-byte aligned
 * input rows; 2-high windows with Q a multiple of 4 take the pair-row kernel, others the
 * per-plane kernel with Q a multiple of 8; 2 = the element-wise kernel, any shape; 3 = the
 * flat kernel: 2-high windows, Q a multiple of 8; 4 = the LDS kernel: any window, stride,
 * padding and dilation whose (kh - 1) * dh + 1 input rows fit 16 KiB of LDS, the default for
 * the shapes the vector kernels do not take when x's rows are contiguous or whole 16-byte
 * vectors).  A forced kernel whose conditions do not hold returns NT_ERR_INVALID before
 * launching.  Replaces the
 * per-configuration launchers of the reference's auto-tuner for the max_pool2d
 * application (reference tests/test_max_pool2d.py:13-64). */
int nt_max_pool2d_config_f32(const void* x, const int64_t* x_strides, void* y, const int64_t* y_strides,
                             int64_t N, int64_t C, int64_t H, int64_t W, int64_t P, int64_t Q,
                             int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
                             int64_t dh, int64_t dw, hipStream_t stream, int config);
int nt_max_pool2d_config_f16(const void* x, const int64_t* x_strides, void* y, const int64_t* y_strides,
                             int64_t N, int64_t C, int64_t H, int64_t W, int64_t P, int64_t Q,
                             int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
                             int64_t dh, int64_t dw, hipStream_t stream, int config);
int nt_max_pool2d_config_bf16(const void* x, const int64_t* x_strides, void* y, const int64_t* y_strides,
                              int64_t N, int64_t C, int64_t H, int64_t W, int64_t P, int64_t Q,
                              int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
                              int64_t dh, int64_t dw, hipStream_t stream, int config);

/* max_pool2d with input and output of any two element types (x_dtype, y_dtype: NT_DTYPE_F32,
 * F16 or BF16; the reference's store casts the window max to the output's type,
 * tests/test_max_pool2d.py:33-36): equal types behave as nt_max_pool2d_*, others take the
 * element-wise kernel.  Still bit-exact: the max of the widened inputs, rounded once,
 * equals the rounded max.  Other arguments as nt_max_pool2d_*. */
int nt_max_pool2d_cast(const void* x, int x_dtype, const int64_t* x_strides, void* y, int y_dtype,
                       const int64_t* y_strides, int64_t N, int64_t C, int64_t H, int64_t W, int64_t P,
                       int64_t Q, int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
                       int64_t dh, int64_t dw, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * GEMM with the addmm epilogue, fp32 accumulation:
 *   acc[m,n]  = sum_k a[m,k] * b[k,n]
 *   out[m,n]  = cast_out(beta * c[m,n] + alpha * round(acc[m,n]))     (fp32 math)
 * `round` rounds acc to `round_dtype` first (NT_DTYPE_NONE = no rounding); it is
 * the application's `accumulator.to(ntl.float16)` (reference tests/test_matmul.py:47).
 * c may be NULL (then beta is ignored).  `out_dtype` packs two codes: bits 0-7 are
 * out's element type (NT_DTYPE_F32/F16/BF16); bits 8-15 are c's type + 1, or 0 when
 * c has out's type.  c may be fp8 (NT_DTYPE_E5M2/E4M3, widened exactly), as in the
 * reference's float8_e5m2 addmm case (tests/test_addmm.py:65-85: fp8 input, fp16 out).
 * Plain matmul is alpha = 1, c = NULL.  Replaces the launchers of the matmul and
 * addmm applications (reference tests/test_matmul.py:14-47, tests/test_addmm.py:13-38;
 * blocked-linalg schedule, src/ninetoothed/compiler/passes.py:1070-1084).
 * a is [M,K] with strides (sa_m, sa_k); b is [K,N] with (sb_k, sb_n); c and out are
 * [M,N] with (sc_m, sc_n) and (so_m, so_n).  Any strides are accepted; unit
 * stride along k for a and along n for b takes the vectorised path.
 * ------------------------------------------------------------------------- */
int nt_gemm_f16(const void* a, int64_t sa_m, int64_t sa_k, const void* b, int64_t sb_k, int64_t sb_n,
                const void* c, int64_t sc_m, int64_t sc_n, void* out, int64_t so_m, int64_t so_n,
                int out_dtype, int64_t M, int64_t N, int64_t K, float alpha, float beta,
                int round_dtype, hipStream_t stream);
int nt_gemm_bf16(const void* a, int64_t sa_m, int64_t sa_k, const void* b, int64_t sb_k, int64_t sb_n,
                 const void* c, int64_t sc_m, int64_t sc_n, void* out, int64_t so_m, int64_t so_n,
                 int out_dtype, int64_t M, int64_t N, int64_t K, float alpha, float beta,
                 int round_dtype, hipStream_t stream);
/* One kernel configuration of the 16-bit GEMM, for the auto-tuner: the arguments of
 * nt_gemm_f16/bf16 plus `config`:
 *   0 = the fastest kernel whose conditions hold, as nt_gemm_*;
 *   1 = the DMA kernel: a k-contiguous; b n-contiguous (N a multiple of 8) or
 *       k-contiguous; 16-byte aligned rows; any M; K a multiple of 8 and at least 96;
 *   2 = the register-staged eight-wave kernel: a k-contiguous, b n-contiguous, M and N
 *       multiples of 256, K of 64;
 *   3 = the element-wise loader kernel: anything;
 *   4 = the DMA kernel on 128 x 128 tiles (four waves, two workgroups per CU): the
 *       conditions of 1, and an out (and c) of the operands' 16-bit type with unit column
 *       stride and 16-byte aligned rows;
 *   5 = the few-rows kernel (the default where it fits with M <= 32, or N <= 4096): M <= 64,
 *       a and b k-contiguous (b^T rows, x @ w.t()) with 16-byte aligned rows, K a multiple
 *       of 8; any N, out.
 * A forced configuration whose conditions do not hold returns NT_ERR_INVALID before
 * launching.  Replaces the per-configuration launchers the reference's auto-tuner times
 * (src/ninetoothed/compiler/driver.py:975-1031, src/ninetoothed/auto_tuner.py:14-202). */
int nt_gemm_config_f16(const void* a, int64_t sa_m, int64_t sa_k, const void* b, int64_t sb_k, int64_t sb_n,
                       const void* c, int64_t sc_m, int64_t sc_n, void* out, int64_t so_m, int64_t so_n,
                       int out_dtype, int64_t M, int64_t N, int64_t K, float alpha, float beta,
                       int round_dtype, int config, hipStream_t stream);
int nt_gemm_config_bf16(const void* a, int64_t sa_m, int64_t sa_k, const void* b, int64_t sb_k, int64_t sb_n,
                        const void* c, int64_t sc_m, int64_t sc_n, void* out, int64_t so_m, int64_t so_n,
                        int out_dtype, int64_t M, int64_t N, int64_t K, float alpha, float beta,
                        int round_dtype, int config, hipStream_t stream);
int nt_gemm_f32(const void* a, int64_t sa_m, int64_t sa_k, const void* b, int64_t sb_k, int64_t sb_n,
                const void* c, int64_t sc_m, int64_t sc_n, void* out, int64_t so_m, int64_t so_n,
                int out_dtype, int64_t M, int64_t N, int64_t K, float alpha, float beta,
                int round_dtype, hipStream_t stream);
/* fp8 operands (OCP float8_e5m2 / float8_e4m3fn, one byte per element, any strides); c and
 * out are f32/f16/bf16 as above.  The reference's float8_e5m2 matmul case,
 * tests/test_matmul.py:64-88 (a row-major, b column-major, fp16 out), runs at the fp8
 * matrix rate when M and N are multiples of 256 and K a multiple of 64 (at least 192). */
int nt_gemm_e5m2(const void* a, int64_t sa_m, int64_t sa_k, const void* b, int64_t sb_k, int64_t sb_n,
                 const void* c, int64_t sc_m, int64_t sc_n, void* out, int64_t so_m, int64_t so_n,
                 int out_dtype, int64_t M, int64_t N, int64_t K, float alpha, float beta,
                 int round_dtype, hipStream_t stream);
int nt_gemm_e4m3(const void* a, int64_t sa_m, int64_t sa_k, const void* b, int64_t sb_k, int64_t sb_n,
                 const void* c, int64_t sc_m, int64_t sc_n, void* out, int64_t so_m, int64_t so_n,
                 int out_dtype, int64_t M, int64_t N, int64_t K, float alpha, float beta,
                 int round_dtype, hipStream_t stream);

/* The GEMM entry points above with all their arguments in one array of 22 int64 values:
 *   v[0]  entry: 0 nt_gemm_f16, 1 nt_gemm_bf16, 2 nt_gemm_f32, 3 nt_gemm_e5m2, 4 nt_gemm_e4m3;
 *   v[1..16]  a, sa_m, sa_k, b, sb_k, sb_n, c, sc_m, sc_n, out, so_m, so_n, out_dtype, M, N, K
 *             (pointers as their address);
 *   v[17], v[18]  alpha and beta, the bits of each float in the low 32 bits;
 *   v[19]  round_dtype;  v[20]  config (nonzero: nt_gemm_config_f16/bf16; entries 0 and 1
 *          only, else NT_ERR_INVALID);  v[21]  the stream.
 * Same results and status as the entry it selects.  No counterpart in the reference: it is
 * for bindings whose per-argument call cost is as long as a small GEMM (the Python binding
 * fills the array once per bound call and rewrites only the data pointers, alpha, beta and
 * the stream: one argument instead of 20). */
int nt_gemm_packed(const int64_t* v);

/* ---------------------------------------------------------------------------
 * 2-D convolution as an implicit GEMM (cross-correlation, as F.conv2d):
 *   y[n,k,p,q] = cast_y(round(sum_{c,r,s} x[n,c,p*sh - ph + r*dh, q*sw - pw + s*dw] * w[k,c,r,s]))
 * with zero outside the input.  The GEMM view is M = N*P*Q, N = K, K = C*R*S, as the
 * conv2d arrangement builds it (reference tests/test_conv2d.py:14-49, pad
 * src/ninetoothed/tensor.py:538-563); the body is the matmul application, so
 * `round_dtype` carries its fp16 cast.  `workspace` (may be NULL) lets the library
 * re-lay the input and filter for vector loads (channels zero-filled up to a multiple
 * of 32 or 64); nt_conv2d_workspace_size() gives the bytes it wants for a shape (0 =
 * not used).  With too small a workspace the direct path runs.
 * ------------------------------------------------------------------------- */
int64_t nt_conv2d_workspace_size(int64_t N, int64_t C, int64_t H, int64_t W, int64_t K,
                                 int64_t R, int64_t S, int64_t ph, int64_t pw, int dtype);
int nt_conv2d_f16(const void* x, const int64_t* x_strides, const void* w, const int64_t* w_strides,
                  void* y, const int64_t* y_strides, int y_dtype,
                  int64_t N, int64_t C, int64_t H, int64_t W, int64_t K, int64_t R, int64_t S,
                  int64_t P, int64_t Q, int64_t ph, int64_t pw, int64_t sh, int64_t sw,
                  int64_t dh, int64_t dw, int round_dtype, void* workspace,
                  int64_t workspace_bytes, hipStream_t stream);
int nt_conv2d_bf16(const void* x, const int64_t* x_strides, const void* w, const int64_t* w_strides,
                   void* y, const int64_t* y_strides, int y_dtype,
                   int64_t N, int64_t C, int64_t H, int64_t W, int64_t K, int64_t R, int64_t S,
                   int64_t P, int64_t Q, int64_t ph, int64_t pw, int64_t sh, int64_t sw,
                   int64_t dh, int64_t dw, int round_dtype, void* workspace,
                   int64_t workspace_bytes, hipStream_t stream);

/* One path of the 16-bit convolution, for the auto-tuner: the arguments of
 * nt_conv2d_f16/bf16 plus `config` (0 = the fastest path whose conditions hold, as
 * nt_conv2d_*; 1 = the re-laid input through the DMA kernel: a workspace of
 * nt_conv2d_workspace_size bytes (which also holds the fp32 partials when the kernel splits
 * the reduction of a small output), C*R*S >= 96 with C rounded up to 32, y of the input
 * type; 2 = the re-laid input through the N-H-W-C kernel:
 * the workspace; 3 = the direct kernel, no workspace; 4 = the re-laid input through the
 * DMA kernel of 224-position tiles, as 1 but never splitting the reduction; 5 = the input
 * read in place, N-C-H-W, by the 224-position strip kernel, only the filter re-laid into the
 * workspace: stride and dilation 1, C % 32 == 0, Q dividing 224 and 224 / Q dividing P,
 * unit w stride, W % 8 == 0, 16-byte aligned input rows, W + pw and Q + S - 1 at most
 * Q + 16, y of the input type; 6 = 1 x 1 filters at stride 1 without padding as a batch of
 * N products (filter [K, C] times image [C, H W]) on the 128 x 128-tile GEMM kernel, no
 * workspace: unit C stride of the filter, H W positions back to back in x and y with
 * 16-byte aligned rows, H W and C multiples of 8, C >= 96, a 16-bit y; H W no multiple of 8
 * through the workspace with rows padded to 8); 7 = the re-laid input through the DMA kernel
 * of 128 x 128 tiles (four waves, two workgroups per CU), as 1 otherwise; the default for
 * outputs of fewer than 136 tiles of 256 x 256).  A forced path whose
 * conditions do not hold returns NT_ERR_INVALID before launching.  Replaces the
 * per-configuration launchers the reference's auto-tuner times
 * (src/ninetoothed/compiler/driver.py:975-1031, tests/test_conv2d.py:109-113). */
int nt_conv2d_config_f16(const void* x, const int64_t* x_strides, const void* w, const int64_t* w_strides,
                         void* y, const int64_t* y_strides, int y_dtype,
                         int64_t N, int64_t C, int64_t H, int64_t W, int64_t K, int64_t R, int64_t S,
                         int64_t P, int64_t Q, int64_t ph, int64_t pw, int64_t sh, int64_t sw,
                         int64_t dh, int64_t dw, int round_dtype, void* workspace,
                         int64_t workspace_bytes, int config, hipStream_t stream);
int nt_conv2d_config_bf16(const void* x, const int64_t* x_strides, const void* w, const int64_t* w_strides,
                          void* y, const int64_t* y_strides, int y_dtype,
                          int64_t N, int64_t C, int64_t H, int64_t W, int64_t K, int64_t R, int64_t S,
                          int64_t P, int64_t Q, int64_t ph, int64_t pw, int64_t sh, int64_t sw,
                          int64_t dh, int64_t dw, int round_dtype, void* workspace,
                          int64_t workspace_bytes, int config, hipStream_t stream);
/* Allocation-free conv2d.  No counterpart in the reference: for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  The arguments of nt_conv2d_f16/bf16 without the workspace: the
 * re-layout workspace is a file-scope device array of NT_CONV2D_SCRATCH_BYTES per GPU
 * (held from the library's first such call on that GPU until the process ends).  A shape
 * whose re-layout needs more (nt_conv2d_workspace_size() > NT_CONV2D_SCRATCH_BYTES)
 * returns NT_ERR_SCRATCH before launching anything.  Nothing is allocated.  All calls on
 * one GPU share its array: calls that overlap on one GPU (different streams, or host
 * threads without ordering) race; calls ordered on one stream do not.  Each call writes
 * every scratch byte it reads, so nothing carries over between calls. */
#define NT_CONV2D_SCRATCH_BYTES (32LL << 20)
#define NT_ERR_SCRATCH 2 /* = hipErrorOutOfMemory: the shape needs more than the static scratch */
int nt_conv2d_noalloc_f16(const void* x, const int64_t* x_strides, const void* w, const int64_t* w_strides,
                          void* y, const int64_t* y_strides, int y_dtype,
                          int64_t N, int64_t C, int64_t H, int64_t W, int64_t K, int64_t R, int64_t S,
                          int64_t P, int64_t Q, int64_t ph, int64_t pw, int64_t sh, int64_t sw,
                          int64_t dh, int64_t dw, int round_dtype, hipStream_t stream);
int nt_conv2d_noalloc_bf16(const void* x, const int64_t* x_strides, const void* w, const int64_t* w_strides,
                           void* y, const int64_t* y_strides, int y_dtype,
                           int64_t N, int64_t C, int64_t H, int64_t W, int64_t K, int64_t R, int64_t S,
                           int64_t P, int64_t Q, int64_t ph, int64_t pw, int64_t sh, int64_t sw,
                           int64_t dh, int64_t dw, int round_dtype, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Fused attention forward (online softmax in base 2), per (b, h):
 *   qs    = round_in(q * q_scale)                 q_scale = log2(e) * softmax scale
 *   s_ij  = qs_i . k_j  (fp32),  -inf where j >= Sk or (causal and i < j)
 *   p_ij  = exp2(s_ij - m_i),  m_i = max_j s_ij,  l_i = sum_j p_ij
 *   o_i   = cast_o(sum_j round_in(p_ij) * v_j / l_i)
 * This is the attention application (reference tests/test_attention.py:45-70),
 * whose q pre-scale is the constant 1.44269504089 and whose causal mask is
 * q_pos >= k_pos.  Tensors are [B, H, S, D] with arbitrary strides; D <= 128.
 * With no keys (Sk == 0) every output is zero, as torch's scaled_dot_product_attention
 * gives; q, k and v are then not read and may be null.
 * ------------------------------------------------------------------------- */
int nt_attention_f16(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                     const void* v, const int64_t* v_strides, void* o, const int64_t* o_strides,
                     int o_dtype, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D,
                     float q_scale, int causal, hipStream_t stream);
int nt_attention_bf16(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                      const void* v, const int64_t* v_strides, void* o, const int64_t* o_strides,
                      int o_dtype, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D,
                      float q_scale, int causal, hipStream_t stream);
int nt_attention_f32(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                     const void* v, const int64_t* v_strides, void* o, const int64_t* o_strides,
                     int o_dtype, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D,
                     float q_scale, int causal, hipStream_t stream);

/* One kernel configuration of the 16-bit attention, for the auto-tuner: the arguments
 * of nt_attention_f16/bf16 plus `config` (0 = the fastest kernel whose conditions hold,
 * as nt_attention_f16/bf16 choose; 1 = the one-wave-per-SIMD pipelined kernel, head dim
 * 128 with unit d-stride and 16-byte aligned rows; 2 = the eight-wave kernel, same
 * conditions, any head dim up to 128 that is a multiple of 8 (padded with zeros to 64 or
 * 128); 3 = the four-wave kernels, any strides).  A forced
 * configuration whose conditions do not hold returns NT_ERR_INVALID before launching.
 * Replaces the per-configuration launchers the reference's auto-tuner times over
 * BLOCK_SIZE_M/N (reference tests/test_attention.py:10-11,
 * src/ninetoothed/compiler/driver.py:975-1031). */
int nt_attention_config_f16(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                            const void* v, const int64_t* v_strides, void* o, const int64_t* o_strides,
                            int o_dtype, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D,
                            float q_scale, int causal, hipStream_t stream, int config);
int nt_attention_config_bf16(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                             const void* v, const int64_t* v_strides, void* o, const int64_t* o_strides,
                             int o_dtype, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D,
                             float q_scale, int causal, hipStream_t stream, int config);

/* ---------------------------------------------------------------------------
 * Generic kernels for programs that match none of the families above.  They replace
 * the reference's run-time toolchain step for generated sources (nvcc + cuModule in
 * src/ninetoothed/backends/materializers/cuda.py:96-170, Triton's compile for the
 * default backend): ninetoothed_amd.generic emits HIP source, these entry points
 * compile it for gfx950 with hipRTC, load it and launch it.
 *   nt_rtc_compile: source -> code object (malloc'd; free with nt_rtc_free); on failure
 *                   NT_ERR_INVALID and the compiler log in `log`.  Needs no GPU.
 *   nt_rtc_load:    code object -> kernel handle; the module stays loaded for the
 *                   process.
 *   nt_rtc_launch:  1-D launch (grid x block threads) with hipModuleLaunchKernel's
 *                   kernel_params (one pointer per argument value) on `stream`.
 * ------------------------------------------------------------------------- */
int nt_rtc_compile(const char* source, const char* name, void** code, int64_t* size, char* log,
                   int64_t log_cap);
void nt_rtc_free(void* code);
int nt_rtc_load(const void* code, const char* kernel_name, void** function);
int nt_rtc_launch(void* function, uint32_t grid, uint32_t block, void** kernel_params, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* NT_MI355X_H */
