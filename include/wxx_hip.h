/* wxx_hip.h — C ABI of libwxx_hip.so, the MI355X (gfx950) backend of wxx.
 *
 * Each entry point replaces one WGSL dispatch (or one runtime service) of the
 * reference's WebGPU backend; the comment on each names the reference
 * interface it stands in for (paths under the reference's src/wxx/).
 *
 * Conventions:
 *  - all functions return 0 on success or a negative WXX_E_* code; the text
 *    of the last failure (per host thread) is wxx_last_error();
 *  - pointers are device addresses from wxx_alloc (already advanced to the
 *    first element of a view); sizes, shapes and strides are int64 element
 *    counts; f32 data is IEEE binary32, u32 indices are uint32, c64 is
 *    interleaved (re, im) binary32 pairs;
 *  - every call enqueues on the library's single in-order HIP stream (the
 *    reference's single shared compute pass); only wxx_d2h, wxx_sync and
 *    wxx_timer_elapsed wait for the device.
 */
#ifndef WXX_HIP_H
#define WXX_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  WXX_OK = 0,
  WXX_E_HIP = -1,
  WXX_E_ARG = -2,
  WXX_E_OOM = -3,
  WXX_E_INIT = -4,
  WXX_E_RANGE = -5,
  WXX_E_UNSUPPORTED = -6,
  WXX_E_CAPTURE = -7
};

/* ---- runtime: replaces WebGPUContext / GPUBufferPool / GPUCommandBuffer
 *      (backend/device.py:9-273) and Tensor storage I/O (Tensor.py:66-90,
 *      522-569) ---------------------------------------------------------- */
const char* wxx_last_error(void);
int wxx_device_count(int* count);
/* device.py:11-13 (adapter + device request) */
int wxx_init(int device);
int wxx_device_info(int* compute_units, char* name, int name_len, size_t* total_mem);
/* GPUBufferPool.create_buffer / release (device.py:53-61, 88-113) */
void* wxx_alloc(size_t bytes);
int wxx_free(void* ptr);
/* GPUBufferPool.clear_cache (device.py:135-141) */
int wxx_empty_cache(void);
/* GPUBufferPool.get_memory_snapshot (device.py:115-133) */
int wxx_mem_stats(size_t* live, size_t* cached, size_t* peak, size_t* n_malloc);
/* create_buffer_with_data upload (device.py:63-86) */
int wxx_h2d(void* dst, const void* src, size_t bytes);
/* Tensor.read_buffer readback (Tensor.py:552-569) */
int wxx_d2h(void* dst, const void* src, size_t bytes);
int wxx_d2d(void* dst, const void* src, size_t bytes);
/* Tensor(value=...) fill (Tensor.py:66-78) */
int wxx_fill_u32(void* dst, int64_t n, uint32_t bits);
/* GPUCommandBuffer.flush(wait=True) (device.py:208-224) */
int wxx_sync(void);
void* wxx_stream(void);
int wxx_timer_record(int slot);
int wxx_timer_elapsed(int start, int stop, float* ms);

/* ---- step graphs.  No reference counterpart: the reference re-encodes every
 *      dispatch of every step (backend/device.py:15-16 notes that this host
 *      cost dominates small models).  wxx_graph_begin starts recording the
 *      library's stream; every entry point called until wxx_graph_end is
 *      recorded, not run.  While recording: wxx_d2h, wxx_sync, the timers and
 *      wxx_empty_cache fail with WXX_E_CAPTURE; wxx_h2d records a copy of the
 *      bytes it is given (replays upload those same bytes); blocks allocated
 *      belong to the graph until wxx_graph_destroy.  wxx_graph_launch replays
 *      the whole recording with one launch, in stream order. */
int wxx_graph_begin(void);
int wxx_graph_end(void** graph, int64_t* nodes);
int wxx_graph_abort(void);
int wxx_graph_launch(void* graph);
int wxx_graph_destroy(void* graph);
int wxx_graph_capturing(int* on);

/* ---- A: GEMM — functional.matmul_add (functional/utils.py:378-499) +
 *      shaders/matmul.wgsl.  sA/sB = batch strides (0 = unbatched);
 *      bias_mode 0 none, 1 (N,), 2 (M,N), 3 (batch,M,N); tile 0 = auto, else a
 *      tile code (1-15) plus 256 x the number of K splits; tiles 11 / 12 /
 *      13 / 14 / 15 (128 x 128 / 128 x 192 / 128 x 64 / 128 x 64 with three
 *      LDS buffers / 64 x 64 with three buffers; operand tiles loaded straight
 *      into LDS) need M a multiple of the tile height, N of its width, K a
 *      multiple of 32 and 16-byte aligned operands, else the call fails. ---- */
int wxx_matmul_add(const float* A, const float* B, const float* bias, float* C, int64_t M,
                   int64_t N, int64_t K, int64_t batch, int64_t sA, int64_t sB, int64_t sBias,
                   int bias_mode, int transpose_A, int transpose_B, int tile);
/* No counterpart in the reference: wxx_matmul_add for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, kernels and results (bit
 * for bit); the split-K partials go to a fixed 64 MiB (16 Mi floats) device
 * array instead of the allocator, and a call needing more fails with
 * WXX_E_RANGE before enqueuing anything.  Calls share that array per GPU:
 * calls that overlap on one GPU race. */
int wxx_matmul_add_noalloc(const float* A, const float* B, const float* bias, float* C,
                           int64_t M, int64_t N, int64_t K, int64_t batch, int64_t sA,
                           int64_t sB, int64_t sBias, int bias_mode, int transpose_A,
                           int transpose_B, int tile);
/* No counterpart in the reference: the products of causal attention with
 * their exactly-zero triangles skipped (same results as wxx_matmul_add, no
 * bias).  tri 1: C square, tiles wholly above the diagonal set to 0 (Q K^T,
 * dO V^T); tri 2: op(A) square lower triangular (P V, dS K); tri 3: op(A)
 * square upper triangular (P^T dO, dS^T Q); tri 4: as 1 with the tiles above
 * the diagonal left unwritten.  Used by nn MultiHeadAttention under GPT-2's
 * causal mask (nn/module.py:447-495, nn/gpt.py:75-96). */
int wxx_matmul_tri(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K,
                   int64_t batch, int64_t sA, int64_t sB, int transpose_A, int transpose_B,
                   int tri);

/* ---- B: convolution and pooling (functional/convolution.py), NCHW f32.
 *      Output size Ho = (H + 2ph - dh(KH-1) - 1)/sh + 1 (conv), (H + 2ph - KH)/sh + 1 (pool). */
/* functional.conv2d (functional/convolution.py:658-729); bias may be null */
int wxx_conv2d(const float* X, const float* W, const float* bias, float* Y, int64_t B,
               int64_t Cin, int64_t H, int64_t Wd, int64_t Cout, int64_t KH, int64_t KW,
               int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw);
/* functional.conv2ddx (functional/convolution.py:732-793): dX from dY and W */
int wxx_conv2ddx(const float* dY, const float* W, float* dX, int64_t B, int64_t Cin, int64_t H,
                 int64_t Wd, int64_t Cout, int64_t KH, int64_t KW, int64_t sh, int64_t sw,
                 int64_t ph, int64_t pw, int64_t dh, int64_t dw);
/* functional.conv2ddw + conv2ddw_reduce (functional/convolution.py:796-908): dW from dY and X */
int wxx_conv2ddw(const float* dY, const float* X, float* dW, int64_t B, int64_t Cin, int64_t H,
                 int64_t Wd, int64_t Cout, int64_t KH, int64_t KW, int64_t sh, int64_t sw,
                 int64_t ph, int64_t pw, int64_t dh, int64_t dw);
/* functional.conv2dtranspose (functional/convolution.py:911-1000): X (B,Cin,H,Wd),
 * W (Cin,Cout,KH,KW), Y (B,Cout,Hout,Wout) with
 * Hout = (H-1)sh - 2ph + dh(KH-1) + output_padding_h + 1; bias may be null */
int wxx_conv2dtranspose(const float* X, const float* W, const float* bias, float* Y, int64_t B,
                        int64_t Cin, int64_t H, int64_t Wd, int64_t Cout, int64_t KH, int64_t KW,
                        int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw,
                        int64_t Hout, int64_t Wout);
/* functional.conv2dtranspose_dx (functional/convolution.py:1003-1064) */
int wxx_conv2dtranspose_dx(const float* dY, const float* W, float* dX, int64_t B, int64_t Cin,
                           int64_t H, int64_t Wd, int64_t Cout, int64_t KH, int64_t KW,
                           int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw,
                           int64_t Hout, int64_t Wout);
/* functional.conv2dtranspose_dw (functional/convolution.py:1067-1185) */
int wxx_conv2dtranspose_dw(const float* dY, const float* X, float* dW, int64_t B, int64_t Cin,
                           int64_t H, int64_t Wd, int64_t Cout, int64_t KH, int64_t KW,
                           int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw,
                           int64_t Hout, int64_t Wout);
/* functional.maxpool2d (avg 0) / avgpool2d (avg 1) (functional/convolution.py:60-192) and
 * maxpool1d / avgpool1d (:195-321, as H = 1); idx (u32 flat input index) may be null */
int wxx_pool2d(const float* x, float* y, uint32_t* idx, int64_t B, int64_t C, int64_t H,
               int64_t W, int64_t KH, int64_t KW, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
               int avg);
/* functional.maxpool2ddx (avg 0, idx required) / avgpool2ddx (avg 1)
 * (functional/convolution.py:425-476, 601-653) and the 1-D backwards (:324-422) */
int wxx_pool2d_backward(const float* dy, const uint32_t* idx, float* dx, int64_t B, int64_t C,
                        int64_t H, int64_t W, int64_t KH, int64_t KW, int64_t sh, int64_t sw,
                        int64_t ph, int64_t pw, int avg);
/* functional.adaptive_avgpool2d (functional/convolution.py:490-543) */
int wxx_adaptive_avgpool2d(const float* x, float* y, int64_t B, int64_t C, int64_t H, int64_t W,
                           int64_t Ho, int64_t Wo);
/* functional.adaptive_avgpool2ddx (functional/convolution.py:546-598) */
int wxx_adaptive_avgpool2ddx(const float* dy, float* dx, int64_t B, int64_t C, int64_t H,
                             int64_t W, int64_t Ho, int64_t Wo);
/* functional.causal_conv1d (functional/convolution.py:1188-1257); x is a strided
 * (B, D, L) view: base pointer, element offset and strides */
int wxx_causal_conv1d(const float* x, int64_t x_off, int64_t sb, int64_t sc, int64_t sl,
                      const float* w, const float* bias, float* y, int64_t B, int64_t D,
                      int64_t L, int64_t KS);
/* functional.causal_conv1d_backward (functional/convolution.py:1260-1351);
 * dw and db are both null when the weight gradient is not needed */
int wxx_causal_conv1d_backward(const float* dy, const float* x, int64_t x_off, int64_t sb,
                               int64_t sc, int64_t sl, const float* w, float* dx, float* dw,
                               float* db, int64_t B, int64_t D, int64_t L, int64_t KS);

/* ---- D: reductions over (outer, reduce, inner) ------------------------- */
/* functional.sum / mean / sumsq (functional/reductions.py:27-197); mode 0/1/2 */
int wxx_reduce(const float* x, float* out, int64_t outer, int64_t reduce, int64_t inner,
               int mode);
/* functional.max / min (functional/reductions.py:241-312); op 0 max, 1 min */
int wxx_reduce_minmax(const float* x, float* vals, uint32_t* idx, int64_t outer,
                      int64_t reduce, int64_t inner, int op);
/* functional.maxmin_backward (functional/reductions.py:200-237) */
int wxx_maxmin_backward(const float* g, const uint32_t* idx, float* out, int64_t outer,
                        int64_t reduce, int64_t inner);
/* functional.softmax (functional/activations.py:126-173) */
int wxx_softmax(const float* x, float* y, int64_t outer, int64_t C, int64_t inner);
/* Softmax backward dx = y * (g - sum(g * y)) along C: the multiply / sum /
 * subtract / multiply chain of autograd softmax (autograd/reductions.py:25-35) */
int wxx_softmax_backward(const float* y, const float* g, float* dx, int64_t outer, int64_t C,
                         int64_t inner);
/* No single reference counterpart: the score path of MultiHeadAttention
 * (nn/module.py:478-483: scores * 1/sqrt(d_head), + mask, softmax) fused into
 * one row pass; y = softmax(x * scale + mask[row % mask_rows]); mask may be null,
 * its rows mask_ld floats apart */
int wxx_softmax_scale_mask(const float* x, const float* mask, float* y, int64_t rows, int64_t C,
                           int64_t mask_rows, int64_t mask_ld, float scale);
/* Gradient of wxx_softmax_scale_mask: dx = scale * y * (g - sum(g y)) — the
 * softmax backward (autograd/reductions.py:25-35) times the scalar-multiply
 * backward (autograd/pointwise.py mulscaler) in one pass */
int wxx_softmax_backward_scale(const float* y, const float* g, float* dx, int64_t rows, int64_t C,
                               float scale);
/* No counterpart in the reference: softmax_scale_mask / its gradient under
 * GPT-2's causal mask (-1e9 above the diagonal, 0 on and below it): row
 * i = row % S reads columns j <= i only; the entries above the diagonal are
 * 0 (left unwritten when skip = 1). */
int wxx_softmax_causal(const float* x, float* y, int64_t rows, int64_t C, int64_t S, float scale,
                       int skip);
int wxx_softmax_backward_causal(const float* y, const float* g, float* dx, int64_t rows, int64_t C,
                                int64_t S, float scale, int skip);
/* functional.meanvarnorm (functional/normalization.py:82-145); row_cap 0 = all rows */
int wxx_meanvarnorm(const float* x, const float* gamma, const float* beta, float* y,
                    float* mean, float* inv_std, int64_t outer, int64_t reduce, int64_t inner,
                    float eps, int64_t row_cap);
/* functional.meanvarnormdx (functional/normalization.py:308-359) */
int wxx_meanvarnormdx(const float* dy, const float* x, const float* gamma, const float* mean,
                      const float* inv_std, float* dx, int64_t outer, int64_t reduce,
                      int64_t inner, int64_t row_cap);
/* functional.meanvarnormdg (functional/normalization.py:362-412) */
int wxx_meanvarnormdg(const float* dy, const float* x, const float* mean, const float* inv_std,
                      float* dgamma, float* dbeta, int64_t outer, int64_t reduce,
                      int64_t inner);
/* functional.rmsnorm (functional/normalization.py:24-79) */
int wxx_rmsnorm(const float* x, const float* gamma, float* y, float* inv_rms, int64_t outer,
                int64_t reduce, int64_t inner, float eps, int64_t row_cap);
/* functional.rmsnormdx (functional/normalization.py:415-463) */
int wxx_rmsnormdx(const float* dy, const float* x, const float* gamma, const float* inv_rms,
                  float* dx, int64_t outer, int64_t reduce, int64_t inner);
/* functional.rmsnormdg (functional/normalization.py:466-513) */
int wxx_rmsnormdg(const float* dy, const float* x, const float* inv_rms, float* dgamma,
                  int64_t outer, int64_t reduce, int64_t inner);
/* functional.batchnorm (functional/normalization.py:148-206); HW = H*W */
int wxx_batchnorm(const float* x, const float* gamma, const float* beta, float* running_mean,
                  float* running_var, float* y, float* saved_mean, float* inv_std, int64_t B,
                  int64_t C, int64_t HW, float eps, float momentum, int training);
/* functional.batchnormdg (functional/normalization.py:260-305) */
int wxx_batchnormdg(const float* dy, const float* x, const float* saved_mean,
                    const float* inv_std, float* dgamma, float* dbeta, int64_t B, int64_t C,
                    int64_t HW);
/* functional.batchnormdx (functional/normalization.py:209-257) */
int wxx_batchnormdx(const float* dy, const float* x, const float* gamma, const float* dgamma,
                    const float* dbeta, const float* saved_mean, const float* inv_std,
                    float* dx, int64_t B, int64_t C, int64_t HW);
/* functional.batchnormdg then functional.batchnormdx (functional/normalization.py:209-305),
 * as autograd's batchnorm backward calls them (autograd/normalization.py): dgamma, dbeta
 * and dx in one call (one launch while B*HW <= 8192, two above) */
int wxx_batchnorm_backward(const float* dy, const float* x, const float* gamma,
                           const float* saved_mean, const float* inv_std, float* dgamma,
                           float* dbeta, float* dx, int64_t B, int64_t C, int64_t HW);
/* functional.batchnorm in training (functional/normalization.py:148-206) followed by the
 * residual add and relu of ResNet's blocks (nn/resnet.py:31-37, 65-66): y = relu(bn(x) +
 * residual), residual null for none, relu 0/1 (one launch while B*HW <= 8192, two above);
 * the running statistics take `updates` (1 or 2) EMA updates, 2 being resnet.py:33's double
 * bn1 evaluation.  B*HW >= 1 and B*C*HW < 2^31, else WXX_E_UNSUPPORTED. */
int wxx_batchnorm_act(const float* x, const float* gamma, const float* beta,
                      const float* residual, float* running_mean, float* running_var, float* y,
                      float* saved_mean, float* inv_std, int64_t B, int64_t C, int64_t HW,
                      float eps, float momentum, int updates, int relu);
/* The backward of wxx_batchnorm_act (autograd/normalization.py batchnorm backward after the
 * relu's and the add's, autograd/pointwise.py): dgamma, dbeta, dx and, exactly when the
 * forward had a residual, dresidual; relu' is taken from the recomputed pre-activation. */
int wxx_batchnorm_act_backward(const float* dy, const float* x, const float* gamma,
                               const float* beta, const float* residual, const float* saved_mean,
                               const float* inv_std, float* dgamma, float* dbeta, float* dx,
                               float* dresidual, int64_t B, int64_t C, int64_t HW, int relu);

/* ---- E: elementwise / layout -------------------------------------------- */
/* functional.pointwise (functional/pointwise.py:29-98) and, with out == a,
 * functional._pointwise (pointwise.py:231-289); op 0 add 1 sub 2 mul 3 div */
int wxx_pointwise(float* out, const float* a, const float* b, int rank, const int64_t* shape,
                  const int64_t* s_out, const int64_t* s_a, const int64_t* s_b, int op);
/* functional.scalarpointwise (functional/pointwise.py:101-146) */
int wxx_scalarpointwise(const float* x, float* y, int64_t n, int op, float c, int reverse);
/* backend/dispatch.py:_unary_op (:59-89) for the activation and unary math
 * kernels of functional/activations.py:22-124 and pointwise.py:293-354 */
int wxx_unary(const float* x, float* y, int64_t n, int op);
/* f'(x) * g for the activation backwards of autograd/pointwise.py:291-388
 * (derivative kernel + pointwise multiply in one pass); op = derivative code */
int wxx_unary_backward(const float* x, const float* g, float* y, int64_t n, int op);
/* SwiGLU's gate h = silu(a) * b (nn/module.py:541-552, Tensor.silu = sigmoid(x) * x at
 * Tensor.py:724-727) in one pass, each operation rounded as the sigmoid and product kernels
 * it replaces round it */
int wxx_swiglu_gate(const float* a, const float* b, float* h, int64_t n);
/* its backward: da, db from dh, a, b in one pass (the mul, mul and sigmoid backwards of
 * autograd/pointwise.py and the gradient sum they replace, same roundings) */
int wxx_swiglu_gate_backward(const float* dh, const float* a, const float* b, float* da,
                             float* db, int64_t n);
/* dst (dense over shape) = src (strides s_src, 0 = broadcast) * scale: the
 * ones_like * grad products of sum/mean backward (autograd/reductions.py:38-95) */
int wxx_broadcast_scale(float* dst, const float* src, int rank, const int64_t* shape,
                        const int64_t* s_src, float scale);
/* functional.clamp / clampbackwards (pointwise.py:149-228), masked_fill
 * (functional/utils.py:558-597); mode 0/1/2 */
int wxx_clamp(const float* x, float* y, int64_t n, float lo, float hi, int mode);
/* functional.equal / equal_number (functional/utils.py:502-556) */
int wxx_equal(const void* a, const void* b, float* out, int64_t n, int mode, uint32_t number);
/* functional.mul_backward (functional/pointwise.py:460-502) */
int wxx_mul_backward(const float* g, const float* a, const float* b, float* da, float* db,
                     int64_t n);
/* functional.contiguous (functional/utils.py:316-369), complex_contiguous
 * (functional/fft.py:295-342), assign from a tensor (utils.py:29-101) */
int wxx_copy_strided(void* dst, const void* src, int itemsize, int rank, const int64_t* shape,
                     const int64_t* s_dst, const int64_t* s_src);
/* functional.assign with a scalar (functional/utils.py:29-101) */
int wxx_fill_strided(void* dst, int rank, const int64_t* shape, const int64_t* s_dst,
                     uint32_t bits);
/* functional.scatter_zeros (functional/utils.py:760-827) */
int wxx_scatter_zeros(float* out, const float* grad, int rank, const int64_t* shape,
                      const int64_t* s_grad, int dim, int64_t start, int64_t length);
/* functional.unfolddx (functional/utils.py:239-287) */
int wxx_unfolddx(const float* dy, float* dx, int64_t prefix, int64_t length, int64_t suffix,
                 int64_t windows, int64_t size, int64_t step);

/* ---- C: FFT and complex ops (functional/fft.py).  X/complex pointers are c64. */
/* functional.rfft (fft.py:484-563): rows x in_len -> rows x (n/2+1); n = 2^k <= 2^27
 * (n <= 32768 in one LDS-resident pass per row, longer as a four-step transform) */
int wxx_rfft(const float* x, void* X, int64_t rows, int64_t in_len, int64_t n);
/* functional.irfft (fft.py:566-645): rows x in_len -> rows x n; n = 2^k, 2 <= n <= 2^27 */
int wxx_irfft(const void* X, float* x, int64_t rows, int64_t in_len, int64_t n);
/* functional.irfft(..., length=L) and the Hyena crop irfft(...)[..., :L]
 * (nn/hyena.py:208-216): the first out_len samples of each row (row stride
 * out_len), times post_scale after the 1/n normalisation (the rfft backward's
 * factor n, autograd/utils.py:549-718). */
int wxx_irfft_crop(const void* X, float* x, int64_t rows, int64_t in_len, int64_t n,
                   int64_t out_len, float post_scale);
/* The Hyena long convolution irfft(rfft(x) * rfft(h))[..., :L] (nn/hyena.py:208-216)
 * and its backward (the rfft / irfft / complex_mul adjoints, autograd/utils.py:549-718)
 * with the spectrum products fused into the transforms; each equals, bit for bit, the
 * separate ops it fuses.  n = 2^k, 2 <= n <= 32768.
 * Bin weights w_k are real: w_edge at bins 0 and n/2, w_mid between (the adjoints'
 * weights), multiplied as the complex (w_k, 0).
 * wxx_rfft_mul: wxx_rfft, then bin k of every row times w_k.
 * wxx_irfft_mul: wxx_irfft_crop of X * h * w: row r of X times row r mod hrows of h
 *   (conjugated when conj_h; null h skips it, h rows have in_len bins) times w_k
 *   when weighted (in_len must then be n/2 + 1).
 * wxx_complex_mul_batch_sum: out[i] = sum_b a[b n + i] * c[b n + i] (conj when conj_c),
 *   the broadcast filter's gradient summed over the batch. */
int wxx_rfft_mul(const float* x, void* X, int64_t rows, int64_t in_len, int64_t n,
                 float w_edge, float w_mid);
int wxx_irfft_mul(const void* X, const void* h, float* x, int64_t rows, int64_t in_len,
                  int64_t hrows, int conj_h, int weighted, float w_edge, float w_mid, int64_t n,
                  int64_t out_len, float post_scale);
int wxx_complex_mul_batch_sum(void* out, const void* a, const void* c, int64_t batch, int64_t n,
                              int conj_c);
/* functional.complex_mul (fft.py:168-213, op 0) and complex_add_inplace
 * (fft.py:216-245, op 1); strides in complex elements, 0 = broadcast */
int wxx_complex_binary(void* out, const void* a, const void* b, int rank, const int64_t* shape,
                       const int64_t* s_out, const int64_t* s_a, const int64_t* s_b, int op,
                       int conj_a, int conj_b);
/* functional.complex_conj (fft.py:248-292) */
int wxx_complex_conj(void* dst, const void* src, int rank, const int64_t* shape,
                     const int64_t* s_dst, const int64_t* s_src);
/* functional.complex_pad (fft.py:345-383) */
int wxx_complex_pad(const void* src, void* dst, int64_t batch, int64_t in_len, int64_t out_len);

/* ---- D7: loss — functional.cceloss (functional/loss.py:20-101) +
 *      shaders/loss/cceloss.wgsl.  *bad (device int) is set to 1 when a
 *      target is >= K; the caller zeroes and reads it. ---- */
int wxx_cceloss(const float* z, const uint32_t* targets, float* loss, float* dz, int64_t B,
                int64_t K, int* bad);
/* No single reference counterpart: cceloss with dlogits deferred to the
 * backward (autograd/layers.py:6-20), already scaled by the upstream gradient
 * g[row * g_stride].  stats holds (max, exp-sum) per row; K <= 65536. */
int wxx_cceloss_stats(const float* z, const uint32_t* targets, float* loss, float* stats,
                      int64_t B, int64_t K, int* bad);
int wxx_cceloss_backward(const float* z, const uint32_t* targets, const float* stats,
                         const float* g, int64_t g_stride, float* dz, int64_t B, int64_t K);

/* ---- E8 / D8: optimizer and gradient norm ---------------------------------- */
/* functional.adamw (functional/layers.py:21-68) */
int wxx_adamw(float* p, const float* g, float* m, float* v, int64_t n, float lr, float beta1,
              float beta2, float eps, float weight_decay, float bc1, float bc2);
/* No reference counterpart: one launch for the whole parameter list of
 * AdamW.step (nn/optimizer.py:69-84); p/g/m/v/n are host arrays of length count */
int wxx_adamw_multi(void* const* p, void* const* g, void* const* m, void* const* v,
                    const int64_t* n, int count, float lr, float beta1, float beta2, float eps,
                    float weight_decay, float bc1, float bc2);
/* No reference counterpart: the per-gradient sumsq + accumulate loop of
 * clip_grad_norm_ (nn/utils.py:82-93) as one reduction into out[0] */
int wxx_sumsq_multi(void* const* x, const int64_t* n, int count, float* out);
/* No reference counterpart: the rescale loop of clip_grad_norm_ (nn/utils.py:97-101) */
int wxx_scale_multi(void* const* x, const int64_t* n, int count, float c);
/* No reference counterpart: wxx_adamw_multi reading its 7 hyperparameters
 * (lr, beta1, beta2, eps, weight_decay, bc1, bc2) from device memory `hyper`
 * when it runs, for recorded step graphs */
int wxx_adamw_multi_dev(void* const* p, void* const* g, void* const* m, void* const* v,
                        const int64_t* n, int count, const float* hyper);
/* clip_grad_norm_'s decision and rescale (nn/utils.py:89-101) taken on the
 * device from the sum of squares at `sumsq`: c = max_norm / (sqrt(s) + 1e-6)
 * in float64, applied when c < 1; `norm` (may be null) gets sqrt(s) */
int wxx_clip_scale_multi(void* const* x, const int64_t* n, int count, const float* sumsq,
                         double max_norm, float* norm);

/* ---- E6 / E7: embedding, dropout; C6: Hyena decay window ------------------ */
/* functional.embed (functional/layers.py:161-206) */
int wxx_embed(const uint32_t* ids, const float* W, float* out, int64_t ntok, int64_t D,
              int64_t V);
/* functional.embeddx (functional/layers.py:209-254), deterministic */
int wxx_embeddx(const float* g, const uint32_t* ids, float* grad, int64_t ntok, int64_t D,
                int64_t V);
/* functional.dropout / dropoutdx (functional/layers.py:73-158) */
int wxx_dropout(const float* x, float* y, int64_t n, uint32_t seed, float p, float scale);
/* No reference counterpart: wxx_dropout with the seed read from device memory
 * `seed` when it runs, for recorded step graphs */
int wxx_dropout_dev(const float* x, float* y, int64_t n, const uint32_t* seed, float p,
                    float scale);
/* ---- fused attention: MultiHeadAttention's score / softmax / dropout /
 *      value path (nn/module.py:460-495) for (B, S, H, d) projections, d in
 *      {32, 64, 128}, 16-byte aligned; causal 1 = GPT-2's causal mask, 0 = no
 *      mask; dropout keeps element (b*H+h, i, j) of the probabilities as
 *      functional.dropout does for that flat index under `seed` (or *seed_dev
 *      when seed_dev is set).  lse: B*H*S row log-sum-exps for the backward. */
int wxx_attention_fwd(const float* q, const float* k, const float* v, float* out, float* lse,
                      int64_t batch, int64_t seq, int64_t heads, int64_t head_dim, int causal,
                      float scale, float p_drop, float drop_scale, uint32_t seed,
                      const uint32_t* seed_dev);
int wxx_attention_bwd(const float* q, const float* k, const float* v, const float* out,
                      const float* dout, const float* lse, float* dq, float* dk, float* dv,
                      int64_t batch, int64_t seq, int64_t heads, int64_t head_dim, int causal,
                      float scale, float p_drop, float drop_scale, uint32_t seed,
                      const uint32_t* seed_dev);

/* functional.decay_window (functional/pointwise.py:357-404) */
int wxx_decay_window(const float* decay, float* w, int64_t rows, int64_t channels,
                     int64_t length, int64_t stage);
/* functional.decay_window_backward (functional/pointwise.py:407-457) */
int wxx_decay_window_backward(const float* g, const float* decay, float* out, int64_t rows,
                              int64_t channels, int64_t length, int64_t stage);

#ifdef __cplusplus
}
#endif

#endif /* WXX_HIP_H */
