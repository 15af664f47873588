/* foidfinder_rocm: MI355X (gfx950) kernels for foidfinder's int8 ViT hot path, behind a plain C ABI.
 *
 * Every entry point takes raw device pointers, sizes and a hipStream_t passed as void* (NULL = the null stream),
 * launches asynchronously on that stream, allocates nothing and never synchronizes, so a caller may capture it in a
 * HIP graph. Buffers are owned by the caller. fp16 tensors are IEEE binary16 passed as void*.
 *
 * Return value: FF_OK (0), or a nonzero FF_E* code with a message retrievable through ff_last_error() (thread-local).
 * Shape and argument preconditions are checked on the host before any HIP call, so they can be exercised without a
 * GPU. The reference raises RuntimeError through TORCH_CHECK for the same preconditions.
 */
#ifndef FOIDFINDER_ROCM_H
#define FOIDFINDER_ROCM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FF_OK 0
#define FF_EINVAL 1  /* bad shape / argument */
#define FF_ELAUNCH 2 /* the HIP runtime rejected a launch */

/* Epilogue codes of ff_gemm_s8. 0-2 keep the reference's values (foidfinder/backends/cuda/csrc/gemm.cuh:8-12). */
#define FF_EPI_QKV_ROPE 0 /* fp16 out [M,N], N = 3C: RoPE on q and k column pairs (table row m % rope_len), q x q_scale */
#define FF_EPI_RESIDUAL 1 /* out [M,N] fp16 is the residual stream: out = fp16(fp16(y) + out) */
#define FF_EPI_GELU_F16 2 /* fp16 out = gelu_tanh(y) */
#define FF_EPI_SWIGLU 3   /* columns are (gate j, value j) pairs: fp16 out [M, N/2], out[m,j] = silu(y[m,2j]) * y[m,2j+1] */
#define FF_EPI_BIAS_F16 4 /* fp16 out = y */
#define FF_EPI_I32 5      /* int32 out [M,N] = the raw accumulators (no scale, no bias) */

/* Version of this ABI; bumps on any signature change. */
int ff_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* ff_last_error(void);

/* Walsh-Hadamard rotation of fp16 rows of 1024 fused with per-token symmetric int8 quantization.
 * x fp16 [T,1024] -> out int8 [T,1024], row_scale fp32 [T], value = code * row_scale.
 * If gamma != NULL, LayerNorm (fp32 gamma/beta [1024], epsilon eps) is applied first.
 * Replaces op `rot_q8_1024(x, gamma?, beta?, out!, row_scale!)`, foidfinder/backends/cuda/csrc/kernels.cu:220-235
 * (which fixes eps = 1e-5, kernels.cu:80). */
int ff_rot_q8_1024(const void* x, const float* gamma, const float* beta, float eps, int64_t T, int8_t* out,
                   float* row_scale, void* stream);

/* Block-diagonal 128-point Walsh-Hadamard rotation + per-token int8 over rows of C (C % 128 == 0, C <= 6144).
 * x fp16 [T,C] -> out int8 [T,C], row_scale fp32 [T]. If gamma != NULL, LayerNorm over the first c_real columns
 * (epsilon eps) is applied first and columns >= c_real are treated as zero padding; gamma/beta are fp32 [C] with
 * zeros in columns >= c_real.
 * Replaces op `rot_q8_h128(x, out!, row_scale!)`, foidfinder/backends/cuda/csrc/kernels.cu:238-251; the fused norm
 * is new (EVA02's SwiGLU LayerNorm, foidfinder/backends/mlx/kernels.py:31-72). */
int ff_rot_q8_h128(const void* x, int64_t T, int64_t C, int64_t c_real, const float* gamma, const float* beta,
                   float eps, int8_t* out, float* row_scale, void* stream);

/* W8A8 GEMM, exact int32 accumulation, fused epilogue:
 * y[m,n] = ((float)(sum_k A[m,k] W[n,k]) * row_scale[m]) * col_scale[n] + bias[n], then the epilogue `epi`.
 * A int8 [M,K], W int8 [N,K] (K contiguous); K % 64 == 0, N % 16 == 0, K <= 2^22, N <= 2^21. rope_cos/rope_sin
 * fp32 [rope_len, 32], 0 < rope_len < 2^24, are needed by FF_EPI_QKV_ROPE only. `variant` selects the tile shape:
 * 1 = 128x128 register-staged, 2 = 256x128 buffer->LDS ring (two workgroups per CU), 3 = 256x256 with 8 waves,
 * 4 = variant 3 on a persistent grid (the rows past the last whole 256-row tile as split-K blocks in the same
 * launch), 5 = variant 3 on 256x128 tiles (narrow products at small M), 6 = 64x64 blocks with K split over
 * 4 waves (small M); 0 = a default by M (6 below 4096 rows, 3 below 16384, else 4). All give identical
 * results.
 * Replaces op `gemm_s8(A, W, row_scale, col_scale, bias, out!, epi, stages, rope_cos?, rope_sin?, q_scale)`,
 * foidfinder/backends/cuda/csrc/kernels.cu:187-217, whose `stages` is the same kind of autotuned knob. */
int ff_gemm_s8(const int8_t* A, const int8_t* W, int64_t M, int64_t N, int64_t K, const float* row_scale,
               const float* col_scale, const float* bias, void* out, int epi, int variant, const float* rope_cos,
               const float* rope_sin, int64_t rope_len, float q_scale, void* stream);

/* Number of tile variants ff_gemm_s8 accepts (1 .. n); variant 0 picks the default. */
int ff_gemm_s8_variants(void);

/* Non-causal flash attention, head_dim 64, over packed qkv rows.
 * qkv fp16 [T, 3*heads*64] (q already rotated and scaled by softmax_scale*log2(e), k rotated) -> out fp16
 * [T, heads*64]; T = num_seqs * seq_len; any seq_len >= 1 (tails are masked).
 * Replaces op `attention(qkv, out!, seq_len)`, foidfinder/backends/cuda/csrc/kernels.cu:255-265 (16 heads and
 * seq_len % 96 == 0 there). */
int ff_attention(const void* qkv, void* out, int64_t T, int64_t heads, int64_t seq_len, void* stream);

/* One pass of Pillow's separable 8-bit resampling (libImaging/Resample.c) over uint8 RGB images [rows, cols, 3].
 * Output out [out_h, out_w, 3]: inside the region rows top .. top+h-1, columns left .. left+w-1, byte (y, x, c) is
 * clip((2^21 + sum_t src[...] * kk[o, t]) >> 22, 0, 255) with o = x - left along the width (axis 0: source row
 * row0 + y - top, columns bounds[o, 0] + t) or o = y - top along the height (axis 1: source rows row0 + bounds[o, 0]
 * + t, column x - left), t < bounds[o, 1]; every other byte is 255 (white). kk int32 [n, ksize] and bounds int32
 * [n, 2] with n >= w (axis 0) or n >= h (axis 1); taps whose source index falls outside src are skipped.
 * Replaces the Haruka letterbox resize pass of the reference's MLX backend, foidfinder/backends/mlx/kernels.py:75-96
 * (the reference's CUDA backend has no Haruka path). */
int ff_resample_u8(const uint8_t* src, int64_t src_h, int64_t src_w, int axis, const int32_t* kk,
                   const int32_t* bounds, int64_t ksize, int64_t row0, uint8_t* out, int64_t out_h, int64_t out_w,
                   int64_t top, int64_t left, int64_t h, int64_t w, void* stream);

/* Two LayerNorms in a row over fp16 rows of C (C % 64 == 0, C <= 2048): y = LN(x; g1, b1) rounded to fp16, then
 * out = LN(y; g2, b2) in fp16; fp16 gamma/beta [C], epsilon eps for both. Haruka's final backbone norm followed by its
 * pool's norm (foidfinder/backends/mlx/haruka.py:101, :122); no counterpart in the reference's CUDA backend. */
int ff_layer_norm2(const void* x, int64_t T, int64_t C, const void* g1, const void* b1, const void* g2,
                   const void* b2, float eps, void* out, void* stream);

/* Token blocks of ff_slot_weights for N tokens (the second dimension of its `partial` output). */
int64_t ff_slot_weights_blocks(int64_t N);

/* Slot-sigmoid pooling weights of Haruka's tree pool (foidfinder/backends/mlx/haruka.py:116-119, masses :133):
 * per batch b, token n and pool head h, with l[m] = logits[b, n, h*M + m] + c[b*c_stride + h*M + m] (c_stride 0: c shared by the
 * batch), w[m] = softmax_m(l)[m] * sigmoid(l[m] + bias[m]) over the M queries (M = 6 or 18). Writes a_t fp16
 * [B, G*M, N] (a_t[b, h*M + m, n] = w[m], query-major rows over the tokens) and partial fp32
 * [B, ff_slot_weights_blocks(N), G*M] (each row the sums of w over one block of tokens; summing over the blocks
 * gives each query's mass). logits fp16 [B, N, G*M], c fp32, bias fp32 [M]. */
int ff_slot_weights(const void* logits, const float* c, int64_t c_stride, const float* bias, int64_t B, int64_t N,
                    int64_t G, int64_t M, void* a_t, float* partial, void* stream);

#ifdef __cplusplus
}
#endif

#endif
