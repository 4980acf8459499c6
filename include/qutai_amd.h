/* libqutai_amd — MI355X (gfx950) GEMM hot path of Qutai behind a C ABI.
 *
 * Every entry point takes plain device pointers, element counts and dtype
 * codes, enqueues its kernels on `stream` (NULL = the default stream, the
 * only stream the reference uses: src/qutai/backends/cuda_runtime.py:326)
 * and returns without synchronising.  Return value: QA_OK (0), a negative
 * QA_E* code for invalid arguments, or a positive hipError_t from the launch.
 *
 * Device memory is owned by the caller (the Python runtime in
 * qutai_amd/backends/amd_runtime.py allocates it through libamdhip64, as the
 * reference allocates through the CUDA driver: cuda_runtime.py:184-228).
 *
 * dtype codes are the positions in the reference storage table
 * (src/qutai/backends/cuda.py:17, `_TYPES`): float32 = 0, float64 = 1,
 * int64 = 4, bfloat16 = 5.  bfloat16 data is raw 16-bit words.
 */
#ifndef QUTAI_AMD_H
#define QUTAI_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QA_F32 0
#define QA_F64 1
#define QA_I64 4
#define QA_BF16 5

#define QA_OK 0
#define QA_EINVAL (-1)     /* shapes, strides, dtypes or pointers rejected */
#define QA_EWORKSPACE (-2) /* workspace missing or too small */
#define QA_ESCRATCH (-3)   /* needs more than the fixed scratch of qutai_amd_gemm_static */

/* The gcnArchName of HIP device `device` (e.g. "gfx950:sramecc+:xnack-"),
 * NUL-terminated into name[size].  Replaces the compute-capability query of
 * the reference runtime (src/qutai/backends/cuda_runtime.py:111-116, device
 * attributes 75/76) that gates its kernels (src/qutai/backends/cuda.py:340-341). */
int qutai_amd_device_arch(int device, char* name, size_t size);

/* Batched GEMM: for z in [0, batch)
 *   out[z][m][n] (+)= sum_k A_z(m,k) * B_z(k,n)
 *   A_z(m,k) = transpose_left  ? a[z*left_stride  + k*rows + m] : a[z*left_stride  + m*inner + k]
 *   B_z(k,n) = transpose_right ? b[z*right_stride + n*inner + k] : b[z*right_stride + k*cols + n]
 * out is [batch][rows][cols] contiguous.  A stride of 0 broadcasts one
 * operand over the batch.  fp32 x fp32 runs on v_mfma_f32_32x32x2_f32; any
 * bf16 operand, or bf16_compute != 0 (autocast), runs on
 * v_mfma_f32_32x32x16_bf16 with fp32 accumulation, an fp32 operand being
 * rounded to bf16 (nearest even) into `workspace` first (see
 * qutai_amd_gemm_workspace_size for when a workspace is needed and how
 * large); fp64 runs a SIMT
 * kernel.  accumulate != 0 adds the old output before the single rounding
 * to out_dtype.  inner == 0 writes zeros (or keeps out when accumulating).
 * Replaces: `cuda.gemm` (src/qutai/backends/cuda.py:305-362) and the kernels
 * gemm_tiled / gemm_register / gemm_bf16 / gemm_bf16_wide / gemm_bf16_long
 * (src/qutai/backends/cuda/gemm.cu:35-223), whose common signature
 * `(a, b, out, M, K, N, sa, sb, ta, tb, accumulate)` this mirrors. */
int qutai_amd_gemm(const void* a, const void* b, void* out, int64_t rows, int64_t inner, int64_t cols,
                   int64_t batch, int64_t left_stride, int64_t right_stride, int transpose_left,
                   int transpose_right, int a_dtype, int b_dtype, int out_dtype, int accumulate,
                   int bf16_compute, void* workspace, size_t workspace_bytes, void* stream);

/* qutai_amd_gemm without a workspace argument and without any allocation:
 * the workspace it needs (see qutai_amd_gemm_workspace_size) is a fixed
 * array in device memory of qutai_amd_gemm_static_capacity() bytes
 * (128 MiB) per GPU, held by the library until the process ends; the
 * caller still passes inputs and output.  Results are bit-identical to
 * qutai_amd_gemm (same kernels).  Returns QA_ESCRATCH when the operands need
 * more workspace than that (e.g. fp32 operands into the bf16 path of more
 * than 64 Mi elements together), before launching anything.  Every call on
 * one GPU shares that GPU's array, so calls that overlap on one GPU (two
 * streams, two host threads) race; calls in one stream are ordered.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc). */
int qutai_amd_gemm_static(const void* a, const void* b, void* out, int64_t rows, int64_t inner, int64_t cols,
                          int64_t batch, int64_t left_stride, int64_t right_stride, int transpose_left,
                          int transpose_right, int a_dtype, int b_dtype, int out_dtype, int accumulate,
                          int bf16_compute, void* stream);

/* Bytes of device scratch behind qutai_amd_gemm_static (per GPU). */
size_t qutai_amd_gemm_static_capacity(void);

/* Bytes of workspace qutai_amd_gemm needs for these arguments with
 * 256-byte-aligned operands (0 when both operands are used in place).  An
 * operand is re-laid out into the workspace when its dtype differs from the
 * MFMA input type (fp32 into the bf16 path) or when its rows are not 16-byte
 * aligned (e.g. a 4097-wide row-major matrix): it then gets a zero-padded
 * pitch so every kernel load is a 16-byte vector load.  Helper of
 * qutai_amd_gemm with no reference counterpart (the reference narrows inside
 * its kernels, gemm.cu:21-24, and uses scalar loads). */
size_t qutai_amd_gemm_workspace_size(int64_t rows, int64_t inner, int64_t cols, int64_t batch,
                                     int64_t left_stride, int64_t right_stride, int transpose_left,
                                     int transpose_right, int a_dtype, int b_dtype, int bf16_compute);

/* Grouped GEMM for MoE experts: group g owns rows [offsets[g], offsets[g+1])
 * of a (row-major, `inner` columns) and of out (row-major, `cols` columns);
 *   out_g = a_g @ B_g   with B_g = b + g*expert_stride, stored [cols][inner]
 *   when transpose_right (the lm weight layout (out, in)) else [inner][cols].
 * `offsets` ([groups+1] int64) lives in device memory and is read by the
 * kernel, so the host never waits for the per-expert counts; max_rows is an
 * upper bound of offsets[groups] (rows * top_k).  dtype is QA_BF16 or QA_F32
 * for both operands.  Replaces the per-expert loop of 3 `cuda_lm.gemm`
 * launches per expert in SparseMoE (src/qutai/lm/layers.py:395-397,
 * src/qutai/backends/cuda_lm.py:31-55) and the count download that sizes
 * them (cuda_lm.py:432-434).
 * With `gather` (device, >= offsets[groups] int64 row indices, may be null)
 * row i of the grouped block is row gather[i] of a, which then holds
 * source_rows rows of `inner` values (source_rows * inner * element size
 * below 2^31): the routed token gather (`route_gather`, cuda_lm.py:471-485)
 * happens inside the operand copy.  An index outside [0, source_rows) reads
 * zeros. */
int qutai_amd_gemm_grouped(const void* a, const void* b, void* out, const int64_t* offsets, int groups,
                           int64_t max_rows, int64_t inner, int64_t cols, int64_t expert_stride,
                           int transpose_right, int dtype, int out_dtype, int accumulate, const int64_t* gather,
                           int64_t source_rows, void* stream);

/* Two grouped products summed in one accumulator:
 *   out_g (+)= a_g @ B_g + a_tail_g @ Btail_g
 * with a / a_tail [offsets[groups]][inner] and b / b_tail laid out as in
 * qutai_amd_gemm_grouped (same expert_stride and orientation), i.e. one
 * grouped product over K = 2 * inner whose first half reads (a, b) and
 * second half (a_tail, b_tail); inner a multiple of 64.  Replaces the two
 * input-gradient products of a SwiGLU expert, dX = dGate W_gate + dUp W_up
 * (src/qutai/lm/layers.py:291-314 under the SparseMoE expert loop 395-397,
 * each a `cuda_lm.gemm`, cuda_lm.py:31-55), which otherwise write and re-read
 * an fp32 [rows][cols] partial between the two. */
int qutai_amd_gemm_grouped_pair(const void* a, const void* a_tail, const void* b, const void* b_tail, void* out,
                                const int64_t* offsets, int groups, int64_t max_rows, int64_t inner, int64_t cols,
                                int64_t expert_stride, int transpose_right, int dtype, int out_dtype, int accumulate,
                                void* stream);

/* SwiGLU feed-forward input side in one GEMM (bf16 only):
 *   out = silu(a @ w_gate^T) * (a @ w_up^T)      [rows][hidden] bf16
 * with the roundings of the unfused form: both products rounded to bf16,
 * silu(gate) rounded to bf16, the product rounded once.  a is [rows][inner]
 * (row-major), w_gate / w_up are [hidden][inner] (the lm weight layout).
 * gate_out / up_out (optional, may be null) receive the two bf16 products
 * for the backward pass.  With offsets (device, [groups+1] int64) the rows
 * are grouped by expert as in qutai_amd_gemm_grouped (rows = an upper bound
 * of offsets[groups]; expert g uses w + g*expert_stride); without, one
 * plain product.  Rows of a and the weights need 16-byte alignment (inner a
 * multiple of 8).  Replaces `silu(self.gate(x)) * self.up(x)` of the SwiGLU
 * block (src/qutai/lm/layers.py:310-311: two projections, lm_silu of
 * cuda/lm.cu:54 and the elementwise multiply), run per expert by SparseMoE
 * (lm/layers.py:395-397).  `gather` / source_rows (grouped calls only) read
 * the rows through an index table as in qutai_amd_gemm_grouped. */
int qutai_amd_gemm_swiglu(const void* a, const void* w_gate, const void* w_up, void* out, void* gate_out,
                          void* up_out, const int64_t* offsets, int groups, int64_t rows, int64_t inner,
                          int64_t hidden, int64_t expert_stride, int dtype, const int64_t* gather,
                          int64_t source_rows, void* stream);

/* Element-wise dtype conversion of n values (fp32/fp64/bf16 among each
 * other; narrowing to bf16 rounds to nearest even).
 * Replaces: `cast` (src/qutai/backends/cuda/tensor.cu:21-29) as driven by
 * `cuda.from_storage` (src/qutai/backends/cuda.py:125-133). */
int qutai_amd_cast(const void* src, void* dst, int64_t n, int src_dtype, int dst_dtype, void* stream);

/* dst[0..n) = value (rounded to dtype; int64 takes the integer part).
 * Replaces: `fill` / `fill_int` (src/qutai/backends/cuda/tensor.cu:11),
 * driven by `cuda.full` (src/qutai/backends/cuda.py:116-122). */
int qutai_amd_fill(void* dst, int64_t n, double value, int dtype, void* stream);

/* out = left + right element-wise (fp32/fp64/bf16; computed in fp32 or fp64,
 * one rounding).  Replaces the `binary` add of tensor.cu used by
 * `cuda.add` for gradient accumulation (src/qutai/core/grad.py:60). */
int qutai_amd_add(const void* left, const void* right, void* out, int64_t n, int dtype, void* stream);

/* out = left + right with fp32 left / out and bf16 right (widened exactly):
 * the residual update `x + update.to(x.dtype)` of the lm blocks
 * (src/qutai/lm/layers.py:31-32), a cast and an add in the reference, in one
 * pass with the same result. */
int qutai_amd_add_widen(const float* left, const void* right, float* out, int64_t n, void* stream);

/* out = x * factor (element-wise, fp32 math for bf16).  Replaces `cuda.scale`
 * (src/qutai/backends/cuda.py:198), used by the lm loss head
 * (src/qutai/lm/layers.py:212). */
int qutai_amd_scale(const void* x, void* out, int64_t n, double factor, int dtype, void* stream);

/* dst[z][r][c] = src[z][r][c] for r < src_rows, c < src_cols, else 0: a
 * stack of `batches` matrices re-pitched from src_rows x src_cols to
 * dst_rows x dst_cols (zero padding or cropping; fp32 or bf16, bits copied).
 * Pads expert weights and routed rows to multiples of 8 columns so that the
 * grouped expert GEMMs serve any d_model / d_expert, as the reference's
 * per-expert `cuda.gemm` calls do (src/qutai/lm/layers.py:395-397; its tiny
 * test models use d_model 8, d_expert 6, tests/test_lm_decoder.py:18-31). */
int qutai_amd_repitch(const void* src, void* dst, int64_t batches, int64_t src_rows, int64_t src_cols,
                      int64_t dst_rows, int64_t dst_cols, int dtype, void* stream);

/* Softmax backward along rows: out = scale * p * (g - rowsum(g * p)), p the
 * softmax of (scale * x) (fp32 math; fp32/fp64/bf16 storage).  Replaces
 * `_softmax_backward` (src/qutai/core/operations/normalization.py:18-25), the
 * rule behind nn.Attention.weights (src/qutai/nn/layers.py:298-303, 334-343). */
int qutai_amd_softmax_backward(const void* probs, const void* grad, void* out, int64_t rows, int64_t width,
                               double scale, int dtype, void* stream);

/* Causal mask of attention scores [rows][width]: row r (query r % length of
 * its batch/head block) keeps keys c <= offset + r % length, the rest become
 * -inf.  Replaces the host-built mask that nn.MultiHeadAttention adds to its
 * scores (src/qutai/nn/layers.py:337-341). */
int qutai_amd_causal_mask(const void* x, void* out, int64_t rows, int64_t width, int64_t length, int64_t offset,
                          int dtype, void* stream);

/* out[r][c] = x[r][c] + bias[c] (rows x cols; one rounding).  The bias add
 * of nn.Linear (src/qutai/nn/layers.py:145-148, a broadcast `add`) and the
 * broadcast of a scalar gradient (cols = 1). */
int qutai_amd_add_rows(const void* x, const void* bias, void* out, int64_t rows, int64_t cols, int dtype,
                       void* stream);

/* out[g] = reduce over the middle axis of x viewed as [outer][count][inner]
 * (sum).  Used to sum gradients over broadcast batch axes; replaces
 * `cuda.unbroadcast` as called by src/qutai/core/operations/linalg.py:51,55. */
int qutai_amd_sum_middle(const void* x, void* out, int64_t outer, int64_t count, int64_t inner, int dtype,
                         void* stream);

/* Two adjacent axes swapped: x is (outer, m, n, inner), out is
 * (outer, n, m, inner) (inner = 1: a transpose of the last two axes).
 * Replaces the general axis permutation of `cuda.transpose`
 * (src/qutai/backends/cuda.py:255) for the head split and merge of
 * nn.MultiHeadAttention (src/qutai/nn/layers.py:322-325, 354). */
int qutai_amd_swap_axes(const void* x, void* out, int64_t outer, int64_t m, int64_t n, int64_t inner, int dtype,
                        void* stream);

/* Swap the last two axes: out[z][c][r] = x[z][r][c].  Replaces the
 * `broadcast`-kernel transpose of src/qutai/backends/cuda.py:255-262 on the
 * non-gemm branch of the matmul gradient (linalg.py:48-55). */
int qutai_amd_transpose_last2(const void* x, void* out, int64_t batch, int64_t rows, int64_t cols, int dtype,
                              void* stream);

/* Row softmax of (scale * x): rows x width, fp32 math, max subtracted.
 * dtype QA_F32 or QA_BF16 (in and out); QA_F64 is computed in fp64.
 * Replaces: `softmax_rows` / `softmax_forward`
 * (src/qutai/backends/cuda/nn.cu:28-37, 67-76) driven by `cuda.softmax`
 * (src/qutai/backends/cuda.py:464-472); scale folds the 1/sqrt(D) of
 * src/qutai/nn/layers.py:336 into the same pass. */
int qutai_amd_softmax_rows(const void* x, void* out, int64_t rows, int64_t width, double scale, int dtype,
                           void* stream);

/* Softmax of (scale * x) along the middle axis of x viewed as
 * [outer][width][inner] (any axis of a row-major tensor).  inner == 1 is
 * qutai_amd_softmax_rows; otherwise one lane per (outer, inner) column with
 * coalesced passes (max, sum of exp, write).  fp32 math for fp32/bf16,
 * fp64 for fp64.  Replaces `cuda.softmax` on any axis
 * (src/qutai/backends/cuda.py:464-472) and its kernels `softmax_rows` /
 * `softmax_forward` (src/qutai/backends/cuda/nn.cu:28-37, 67-76). */
int qutai_amd_softmax(const void* x, void* out, int64_t outer, int64_t width, int64_t inner, double scale,
                      int dtype, void* stream);

/* Strided copy: for every coordinate c of the row-major index space dims[rank]
 *   dst[sum_d c_d * dst_strides[d]] = src[sum_d c_d * src_strides[d]]
 * (strides in elements of element_bytes = 2, 4 or 8; a source stride of 0
 * broadcasts; rank <= 8).  dims and strides are host arrays.  Unit axes are
 * dropped and axes contiguous on both sides merged before the launch; runs
 * of the innermost axis move 16 bytes per lane when both sides allow it.
 * One kernel for `cuda.broadcast` (src/qutai/backends/cuda.py:245-252),
 * `cuda.transpose` (:255-262, any permutation), `cuda.concatenate`
 * (:383-394) and `cuda.gather_slice` / `cuda.scatter_slice` (:229-242), all
 * of which drive the reference's `broadcast` / `slice_copy` /
 * `concatenate` kernels (src/qutai/backends/cuda/tensor.cu:49-54, 56-58,
 * 67-69) with int64 metadata uploaded per call; here the metadata travels in
 * the kernel arguments. */
int qutai_amd_strided_copy(const void* src, void* dst, int rank, const int64_t* dims, const int64_t* src_strides,
                           const int64_t* dst_strides, int element_bytes, void* stream);

/* out = left (op) right element-wise, op 0 add, 1 subtract, 2 multiply,
 * 3 divide; fp32 math for fp32/bf16 (one rounding), fp64 for fp64.  With
 * zero_flag (device int32) the call first sets *zero_flag = 0 and a divide
 * sets it to 1 when any divisor is zero (the caller reads it to raise
 * ZeroDivisionError).  out may be left or right (in place).  Replaces
 * `cuda.add/subtract/multiply/divide` and `add_into`
 * (src/qutai/backends/cuda.py:171-189, 141-147) over the `binary` kernel
 * (src/qutai/backends/cuda/tensor.cu:30). */
int qutai_amd_binary(const void* left, const void* right, void* out, int64_t n, int op, int dtype, int* zero_flag,
                     void* stream);

/* out = f(x) element-wise (gradient = NULL) or g * f'(x) (gradient given):
 * op 0 negate, 1 square, 2 x * factor, 3 relu, 4 relu backward, 5 gelu,
 * 6 gelu backward, 7 exp, 8 log (sets *flag = 1 when some x <= 0), 9 tanh,
 * 10 atan, 11 tanh backward, 12 atan backward, 13 x / factor.  fp32 math
 * for fp32/bf16, fp64 for fp64; with flag the call first clears it.  out
 * may be x (in place).  Replaces `cuda.divide_scalar`, `negate` ...
 * `atan_backward` and `scale_into` (src/qutai/backends/cuda.py:157-168,
 * 192-208, 150-154) over the `unary` kernel
 * (src/qutai/backends/cuda/tensor.cu:31-46). */
int qutai_amd_unary(const void* x, const void* gradient, void* out, int64_t n, int op, double factor, int dtype,
                    int* flag, void* stream);

/* out[o][j] = sum_c x[o][c][j] for x viewed as [outer][width][inner]
 * (inner = 1: row sums; outer = inner = 1: the sum of everything), in fp32
 * (fp64 for fp64) with one rounding.  Long sums are split into parts whose
 * partial sums land in `workspace` and are added in part order, so results
 * repeat bit for bit.  Replaces `cuda.sum` / `cuda.mean` / `cuda.unbroadcast`
 * (src/qutai/backends/cuda.py:265-289) and the `reduce_sum` kernel
 * (src/qutai/backends/cuda/tensor.cu:59-61), which sums each output in one
 * thread. */
int qutai_amd_reduce_sum(const void* x, void* out, int64_t outer, int64_t width, int64_t inner, int dtype,
                         void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of workspace qutai_amd_reduce_sum needs (0 when one pass does). */
size_t qutai_amd_reduce_sum_workspace_size(int64_t outer, int64_t width, int64_t inner, int dtype);

/* out[i] = x[positions[i]] for n elements of element_bytes (positions:
 * device int64).  Replaces `cuda.gather` (src/qutai/backends/cuda.py:211-215,
 * kernel src/qutai/backends/cuda/tensor.cu:48). */
int qutai_amd_gather(const void* x, const int64_t* positions, void* out, int64_t n, int element_bytes, void* stream);

/* out[t] = sum of x[order[k]] for k in [start[t], start[t+1]), in k order, for
 * t < size (start: size+1 device int64, order: device int64; the host groups
 * every source index under its target position).  Deterministic form of
 * `cuda.scatter` (src/qutai/backends/cuda.py:218-226, an atomicAdd kernel
 * src/qutai/backends/cuda/tensor.cu:55). */
int qutai_amd_scatter(const void* x, const int64_t* start, const int64_t* order, void* out, int64_t size, int dtype,
                      void* stream);

/* out = silu(gate) * up element-wise (fp32 math, one rounding to dtype).
 * Replaces `lm_silu` (src/qutai/backends/cuda/lm.cu:54) followed by the
 * elementwise multiply of SwiGLU (src/qutai/lm/layers.py:310-311). */
int qutai_amd_silu_mul(const void* gate, const void* up, void* out, int64_t n, int dtype, void* stream);

/* Gradients of out = silu(gate) * up: dgate = dy * up * s * (1 + gate (1 - s))
 * and dup = dy * silu(gate), s = sigmoid(gate).  Replaces the backward of
 * `lm_silu` (src/qutai/backends/cuda/lm.cu:54, backward branch) and of the
 * elementwise multiply in SwiGLU (src/qutai/lm/layers.py:310-311). */
int qutai_amd_silu_mul_backward(const void* dy, const void* gate, const void* up, void* dgate, void* dup, int64_t n,
                                int dtype, void* stream);

/* MoE routing, forward.  scores: [rows][experts] fp32 router logits.
 * Writes probs [rows][experts] (fp32 softmax), weights [rows][top_k] (fp32,
 * renormalised over the selected experts), indices [rows][top_k] (int64;
 * descending probability, lowest expert index first on ties), counts
 * [experts], ids / slots [experts][capacity] (stable token-major lists per
 * expert), locations [rows][top_k] (position inside the expert list),
 * offsets [experts+1] (exclusive prefix sum of counts), order [rows*top_k]
 * (ids concatenated expert-major: order[offsets[e]+i] = ids[e][i]),
 * utilization [experts] (count / (rows*top_k)) and aux [1]
 * (experts * sum_{r,e} probs*utilization / rows).  capacity = rows * top_k
 * (below 2^31, else QA_EINVAL).
 * Replaces `cuda_lm.routing` (src/qutai/backends/cuda_lm.py:368-449) and its
 * kernels lm_route, lm_route_pack, lm_route_util, lm_route_aux
 * (src/qutai/backends/cuda/lm.cu:345-387); selection follows the CPU
 * oracle `cpu_lm.routing` (src/qutai/backends/cpu_lm.py:204-242). */
int qutai_amd_route(const float* scores, float* probs, float* weights, int64_t* indices, int64_t* counts,
                    int64_t* ids, int64_t* slots, int64_t* locations, int64_t* offsets, int64_t* order,
                    float* utilization, float* aux, int64_t rows, int64_t experts, int64_t top_k, void* workspace,
                    size_t workspace_bytes, void* stream);

/* Device workspace bytes for qutai_amd_route's chunked path (up to 32
 * experts and top-8: three launches over chunks of 256 tokens, no per-expert
 * pass over all assignments); 0 when that path does not apply.  With a smaller
 * or NULL workspace qutai_amd_route runs its one-workgroup-per-expert pack.
 * Same outputs either way (the aux loss up to fp32 summation order). */
size_t qutai_amd_route_workspace_size(int64_t rows, int64_t experts, int64_t top_k);

/* out[r] = x[order[r]] for r in [0, count): gathers the token rows of all
 * experts into one expert-major block (width values per row).  backward != 0
 * scatters instead: out[order[r]] = x[r] (each token appears once per
 * expert, so no accumulation is needed within one expert).
 * Replaces `lm_route_gather` (src/qutai/backends/cuda/lm.cu:394-396) driven
 * per expert by `cuda_lm.route_gather` (src/qutai/backends/cuda_lm.py:471-502). */
int qutai_amd_route_gather(const void* x, const int64_t* order, void* out, int64_t count, int64_t width,
                           int backward, int dtype, void* stream);

/* Weighted combine: y[row] = sum_slot weights[row][slot] *
 *   expert_out[offsets[indices[row][slot]] + locations[row][slot]]
 * summed in fp32 in slot order with one rounding to dtype.
 * Replaces `lm_pointer_table` + `lm_combine_all`
 * (src/qutai/backends/cuda/lm.cu:400-416, src/qutai/backends/cuda_lm.py:505-541).
 * weights may be NULL: unit weights, i.e. the sum over a token's slots (the
 * backward of the one-launch gather).  out_dtype is dtype, or QA_BF16 for
 * fp32 expert rows (the token gradient rounded once from the fp32 sum). */
int qutai_amd_combine(const void* expert_out, const float* weights, const int64_t* indices,
                      const int64_t* locations, const int64_t* offsets, void* y, int64_t rows, int64_t width,
                      int64_t top_k, int dtype, int out_dtype, void* stream);

/* Attention forward, fp32 math:
 *   out = softmax(scale * Q K^T [+ causal mask]) V  per (batch, head),
 * without materialising the time x time scores.  dtype QA_BF16 or QA_F32 for
 * q, k, v and out; head dimension `dim` <= 256.  bf16 with dim = 64 runs the
 * fused MFMA kernel (16-byte aligned pointers required); every other case the
 * one-wave-per-row kernel of the reference's general path.  layout 0: q/k/v/out
 * are [batch][heads][time][dim] (the nn layout); layout 1:
 * [batch][time][heads][dim] (the lm layout, head-interleaved).  kv_heads divides heads (grouped-query
 * attention: head h reads kv head h / (heads / kv_heads)).  lse (optional,
 * fp32) receives the natural-log sum of exponentials, laid out like q without
 * the last axis: [batch][heads][time] (layout 0), [batch][time][heads]
 * (layout 1, the reference's lse layout).  The normaliser sums fp32
 * probabilities; the value product takes them rounded to bf16, as in the
 * reference kernel.  Replaces `lm_attention_bf16_d64` and the general
 * `lm_attention` (src/qutai/backends/cuda/lm.cu:91-157, :65-87, driven by
 * `cuda_lm.attention`, src/qutai/backends/cuda_lm.py:229-252) and the
 * S = Q K^T / softmax / P V sequence of nn attention
 * (src/qutai/nn/layers.py:334-354). */
int qutai_amd_attention_fwd(const void* q, const void* k, const void* v, void* out, float* lse, int64_t batch,
                            int64_t heads, int64_t kv_heads, int64_t time, int64_t dim, int dtype, int layout,
                            double scale, int causal, void* stream);

/* Grouped-K GEMM for the MoE weight gradients: for every group g,
 *   out[g] (rows x cols) (+)= A_g^T B_g,
 * where A_g / B_g are the K rows [offsets[g], offsets[g+1]) of a ([K][rows])
 * and b ([K][cols]) -- the expert-major routed rows.  E.g. dW_down[e] =
 * dY_e^T act_e.  An empty group writes zeros (or keeps out with accumulate).
 * dtype QA_BF16 / QA_F32 for a and b, out_dtype QA_F32 / QA_BF16; rows and
 * cols multiples of 8 (bf16) / 4 (fp32), 16-byte aligned operands.  total_k
 * = offsets[groups] (only used for tile choice).  With gather (the route's
 * order, total_k entries), K row k of b is row gather[k] of b, a
 * [source_rows][cols] token matrix below 2 GiB: the weight gradients
 * dW_gate / dW_up = dY_e^T X_e read the routed token rows in place instead
 * of a gathered copy (src/qutai/backends/cuda_lm.py:471-502 copies them,
 * lm.cu:394-396); an index outside [0, source_rows) reads a zero row.
 * Replaces the per-expert weight-gradient GEMMs of the expert SwiGLU
 * backward (`linear` backward, src/qutai/lm/layers.py:57-66, run once per
 * expert by SparseMoE, lm/layers.py:395-397). */
int qutai_amd_gemm_grouped_k(const void* a, const void* b, void* out, const int64_t* offsets, int groups, int64_t rows,
                             int64_t cols, int64_t total_k, int dtype, int out_dtype, int accumulate,
                             const int64_t* gather, int64_t source_rows, void* stream);

/* Backward of qutai_amd_combine for every routed (token, slot) pair: the
 * pair's expert-major row of d_expert_out = dy[token] * weight, and
 * d_weights[pair] = dy[token] . expert_out[row] (fp32).  Same routing arrays
 * as qutai_amd_combine.  Replaces `cuda_lm.combine_backward`
 * (src/qutai/backends/cuda_lm.py:544-581; cpu_lm.py:306-320). */
int qutai_amd_combine_backward(const void* dy, const void* expert_out, const float* weights, const int64_t* indices,
                               const int64_t* locations, const int64_t* offsets, void* d_expert_out,
                               float* d_weights, int64_t rows, int64_t width, int64_t top_k, int dtype,
                               void* stream);

/* Gradient of the router logits from the gradient of the routing weights
 * (auxiliary = 0: gradient [rows*top_k]) or of the auxiliary loss
 * (auxiliary = 1: gradient [1]); out [rows*experts] fp32 is overwritten.
 * Replaces `cuda_lm.routing_backward` (src/qutai/backends/cuda_lm.py:452-467;
 * cpu_lm.py:245-276). */
int qutai_amd_route_backward(const float* gradient, const float* probs, const float* weights,
                             const int64_t* indices, const float* utilization, float* out, int64_t rows,
                             int64_t experts, int64_t top_k, int auxiliary, void* stream);

/* Fused attention backward for the forward above (same layouts, scale and
 * causal flag): from dO (grad), q, k, v, the forward's bf16 output `out` and
 * its fp32 `lse`, writes dq, dk, dv (bf16) and delta = rowsum(dO * out)
 * (fp32, lse's layout; a caller-provided buffer of batch*heads*time floats):
 *   P = exp(scale q k^T - lse), dS = P (dO v^T - delta) scale,
 *   dq = dS k, dk = dS^T q (summed over the heads sharing a kv head),
 *   dv = P^T dO.
 * Same dtype / dim / path rules as the forward.  Deterministic (no atomics).
 * Replaces `cuda_lm.attention_backward`
 * (src/qutai/backends/cuda_lm.py:278-365) with its kernels
 * lm_attention_delta / lm_attention_bf16_dq / lm_attention_bf16_dkv /
 * lm_attention_backward_q / _kv (src/qutai/backends/cuda/lm.cu:159-343);
 * semantics of
 * cpu_lm.attention_backward (src/qutai/backends/cpu_lm.py:176-201).
 * `workspace` (optional, 16-byte aligned) of
 * qutai_amd_attention_bwd_workspace_size bytes lets grouped-query attention
 * (heads > kv_heads) on small batches split each kv head's dK/dV work over
 * its query heads and sum the fp32 partials in order; without it (or when
 * that size is 0) one workgroup covers all query heads of a kv head. */
int qutai_amd_attention_bwd(const void* grad, const void* q, const void* k, const void* v, const void* out,
                            const float* lse, void* dq, void* dk, void* dv, float* delta, void* workspace,
                            size_t workspace_bytes, int64_t batch, int64_t heads, int64_t kv_heads, int64_t time,
                            int64_t dim, int dtype, int layout, double scale, int causal, void* stream);

/* Bytes of the optional qutai_amd_attention_bwd workspace for these
 * arguments (0 when the split does not apply).  No reference counterpart:
 * the reference's dK/dV kernel always loops over the query heads of a kv
 * head in one block (src/qutai/backends/cuda/lm.cu:217-288). */
size_t qutai_amd_attention_bwd_workspace_size(int64_t batch, int64_t heads, int64_t kv_heads, int64_t time,
                                              int64_t dim, int dtype);

/* ---- decoder glue around the contractions (a full Decoder.loss step) ----
 * Activation dtype QA_BF16 or QA_F32; embedding / RMSNorm weights, RMSNorm
 * outputs and statistics, embedding gradients and head losses are fp32 (the
 * reference's accumulation type for both activation types). */

/* out[r] = weight[ids[r]] (count rows of width) in out_dtype.  Replaces
 * `cuda_lm.embedding` / `lm_embedding` (src/qutai/backends/cuda_lm.py:77-93,
 * cuda/lm.cu:30). */
int qutai_amd_embedding(const float* weight, const int64_t* ids, void* out, int64_t count, int64_t width,
                        int out_dtype, void* stream);

/* out[tokens[g]] = sum of gradient rows rows[offsets[g] .. offsets[g+1]) (input
 * order) for each of `groups` distinct tokens, added to the old row when
 * `accumulate` (a tied table's gradient that already holds the head's part);
 * other rows of out untouched.  Replaces `cuda_lm.embedding_backward` /
 * `lm_embedding_backward` (cuda_lm.py:96-123, cuda/lm.cu:32-38). */
int qutai_amd_embedding_backward(const void* gradient, const int64_t* tokens, const int64_t* offsets,
                                 const int64_t* rows, float* out, int64_t groups, int64_t width, int dtype,
                                 int accumulate, void* stream);

/* inverse[r] = 1/sqrt(mean(x[r]^2) + eps), out = x * inverse * weight.
 * Replaces `cuda_lm.rms_norm` / `lm_rms` (cuda_lm.py:126-145, cuda/lm.cu:39-45). */
int qutai_amd_rms_norm(const void* x, const float* weight, float* out, float* inverse, int64_t rows, int64_t width,
                       double eps, int dtype, void* stream);

/* qutai_amd_rms_norm that also stores out rounded to bf16 (RNE, the cast
 * kernel's rounding) into out_bf16 when it is not null: the copy the
 * bf16-path products of the normalised activation take under autocast
 * (the reference rounds the fp32 norm output when its Linear runs in bf16,
 * lm/layers.py:20-28 with 88-96), written by the norm instead of a separate
 * cast pass.  Same fp32 outputs as qutai_amd_rms_norm. */
int qutai_amd_rms_norm_bf16(const void* x, const float* weight, float* out, void* out_bf16, float* inverse,
                            int64_t rows, int64_t width, double eps, int dtype, void* stream);

/* Floats of the `partial` workspace qutai_amd_rms_norm_backward needs. */
int64_t qutai_amd_rms_norm_workspace(int64_t rows, int64_t width);

/* dx = inverse * (g w - x inverse^2 mean(g w x)) (dx in the activation dtype),
 * dweight[j] = sum_r g x inverse (fp32, fixed-order chunked sum through
 * `partial`).  Replaces `cuda_lm.rms_norm_backward` / `lm_rms_dx` / `lm_rms_dw`
 * (cuda_lm.py:148-177, cuda/lm.cu:46-52).  `residual` (NULL, or fp32 rows x
 * width, not dx itself; QA_F32 only) is added to dx as it is stored:
 * dx = residual + dx with one fp32 rounding, the value of a separate add (the
 * residual stream's gradient summed with the norm's; no counterpart in the
 * reference, whose autograd adds the two). */
int qutai_amd_rms_norm_backward(const float* gradient, const void* x, const float* weight, const float* inverse,
                                const float* residual, void* dx, float* dweight, float* partial, int64_t rows,
                                int64_t width, int dtype, void* stream);

/* out = x sigmoid(x), or with backward = 1 out = g s (1 + x (1 - s)).
 * Replaces `cuda_lm.silu` / `silu_backward` (cuda_lm.py:180-207, cuda/lm.cu:54). */
int qutai_amd_silu(const void* x, const void* gradient, void* out, int64_t n, int backward, int dtype,
                   void* stream);

/* Rotary embedding of [batch][time][heads][dim] pairs (2i, 2i+1) by the angle
 * (offset + t) theta^(-d/dim), d = 2 (i mod dim/2); inverse rotates back.
 * Replaces `cuda_lm.rope` / `lm_rope` (cuda_lm.py:210-226, cuda/lm.cu:55-59). */
int qutai_amd_rope(const void* x, void* out, int64_t batch, int64_t time, int64_t heads, int64_t dim, double theta,
                   int64_t offset, int inverse, int dtype, void* stream);

/* The same rotation where a position's heads*dim values sit x_row (out_row)
 * elements after the previous position's (>= heads*dim): RoPE read from, or
 * written into, a column slice of a wider row-major matrix -- the q and k
 * columns of the stacked q/k/v projection output [rows][dq + 2 dkv], which
 * replaces the three `Projection` calls ahead of `rope` in the reference's
 * GQA block (src/qutai/lm/layers.py:317-350, cuda_lm.py:210-226). */
int qutai_amd_rope_rows(const void* x, void* out, int64_t batch, int64_t time, int64_t heads, int64_t dim,
                        double theta, int64_t offset, int inverse, int64_t x_row, int64_t out_row, int dtype,
                        void* stream);

/* The rows start .. start+count of the (time-1) prediction positions of every
 * sequence of a [.][time][width] block (backward = 1: add them back into it).
 * Replaces `cuda_lm.head_rows` / `head_rows_backward` / `lm_head_rows`
 * (cuda_lm.py:584-613, cuda/lm.cu:425-427). */
int qutai_amd_head_rows(const void* x, void* out, int64_t count, int64_t start, int64_t width, int64_t time,
                        int backward, int dtype, void* stream);

/* out[r] = log sum exp(logits[r] - max) - (logits[r][label] - max), 0 for label
 * -100.  Replaces `lm_head_loss` (cuda_lm.py:629-643, cuda/lm.cu:428-433). */
int qutai_amd_head_loss(const void* logits, const int64_t* labels, float* out, int64_t rows, int64_t vocab,
                        int dtype, void* stream);

/* In place: logits = gradient[0] * factor * (softmax(logits) - onehot(label)),
 * 0 for label -100.  Replaces `lm_head_gradient` (cuda_lm.py:646-660,
 * cuda/lm.cu:434-440). */
int qutai_amd_head_gradient(void* logits, const int64_t* labels, const float* gradient, int64_t rows, int64_t vocab,
                            double factor, int dtype, void* stream);

/* Vocabulary-blocked loss head.  `logits` is one block [rows][cols] of the
 * [rows][vocab] logits, holding vocabulary columns col0 .. col0+cols.
 * head_block_stats folds each row's (max, sum exp(v - max)) over the block
 * into stats[row] = {max, sum} (overwritten when `first`) and stores the
 * label's logit in picked[row] when the label lies in the block; rows with
 * label -100 are skipped.  head_block_loss writes out[r] = log(sum) + max -
 * picked (0 for label -100).  head_block_gradient turns a block in place into
 * gradient[0] * factor * (exp(v - max) / sum - onehot(label)) (0 for label
 * -100).  Together they compute what `lm_head_loss` / `lm_head_gradient` do
 * per row chunk (cuda_lm.py:629-660, cuda/lm.cu:428-440, driven by the
 * chunked head of src/qutai/lm/layers.py:194-257), with the chunks cut along
 * the vocabulary instead of the rows. */
int qutai_amd_head_block_stats(const void* logits, const int64_t* labels, float* stats, float* picked, int64_t rows,
                               int64_t cols, int64_t col0, int first, int dtype, void* stream);
int qutai_amd_head_block_loss(const float* stats, const float* picked, const int64_t* labels, float* out,
                              int64_t rows, void* stream);
int qutai_amd_head_block_gradient(void* logits, const int64_t* labels, const float* stats, const float* gradient,
                                  int64_t rows, int64_t cols, int64_t col0, double factor, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QUTAI_AMD_H */
