/*
 * molla_mi.h -- C ABI of the MI355X (gfx950) decode hot path for molla.
 *
 * A drop-in for molla's device matvec / decoder-layer entry points.  molla's
 * Mojo host reaches these through `external_call` (pointers cross as Int,
 * as in /root/reference/src/molla/sys/thread.mojo:104-161).  Every pointer
 * argument that names tensor data is a DEVICE pointer unless stated; shapes
 * are int32 as in the reference kernels (src/molla/nn/gpu.mojo:1558-1559),
 * byte strides int64.
 *
 * Conventions shared by every entry point:
 *  - Weights are raw GGUF blocks (ggml `block_q*` byte layout), rows back to
 *    back with no padding: row r of a (rows x cols) tensor starts at
 *    w + r * row_bytes, row_bytes = cols / block_elements * block_bytes.
 *    The reference device path repacks into its own "planar" layout first
 *    (src/molla/nn/repack.mojo:692); this library reads file bytes directly.
 *  - Everything is queued on the caller's stream and NOT synchronized, as in
 *    the reference (gpu.mojo:2178-2180).  mi_sync() waits.
 *  - Nothing allocates device memory per call.  Scratch comes from the
 *    caller as a workspace (size from the matching *_workspace call), the
 *    way the reference sizes its DeviceScratch once per session
 *    (src/molla/nn/gpu_block.mojo:495-622).  A workspace may not be shared by
 *    two calls in flight on different streams.
 *  - Return value: MI_OK (0) or a negative MI_ERR_* code.  A refused call
 *    launches nothing (the reference's pre-launch refusals,
 *    gpu.mojo:2070-2111); mi_last_error() then describes why (thread-local).
 *    There is no CPU fallback anywhere.
 */
#ifndef MOLLA_MI_H
#define MOLLA_MI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* mi_stream; /* a hipStream_t; NULL is the default stream */

enum {
  MI_OK = 0,
  MI_ERR_ARG = -1,       /* null pointer, negative size, bad flag */
  MI_ERR_KIND = -2,      /* ggml type without a device kernel */
  MI_ERR_SHAPE = -3,     /* cols not a whole number of blocks, row_bytes mismatch, too large */
  MI_ERR_WORKSPACE = -4, /* workspace missing or too small */
  MI_ERR_DEVICE = -5,    /* HIP runtime error (launch, sync) */
  MI_ERR_ALIGN = -6      /* pointer alignment the kernels require is not met */
};

/* ggml type numbers (src/molla/nn/quant.mojo:47-57).  Device dequant and
 * matvec kernels exist for the eight block-quantized kinds; F32 is accepted
 * by the embedding lookup only. */
enum {
  MI_F32 = 0,
  MI_F16 = 1,
  MI_Q4_0 = 2,
  MI_Q4_1 = 3,
  MI_Q5_0 = 6,
  MI_Q5_1 = 7,
  MI_Q8_0 = 8,
  MI_Q4_K = 12,
  MI_Q5_K = 13,
  MI_Q6_K = 14
};

/* Matvec epilogues, same integers and meaning as src/molla/nn/gpu.mojo:781-803:
 *   NONE: y = dot          BIAS: y = dot + aux[r]
 *   ADD:  y = y + dot      GLU:  y = act(dot) * aux[t*rows + r]  (act = silu,
 *                                or gelu-tanh with MI_ACT_GELU)
 * BIAS or GLU may be combined with ADD, as in the reference. */
enum { MI_EPI_NONE = 0, MI_EPI_BIAS = 1, MI_EPI_ADD = 2, MI_EPI_GLU = 4, MI_ACT_GELU = 8 };

/* ---- library ------------------------------------------------------------- */

int mi_version(void);                 /* (major << 16) | minor */
const char* mi_last_error(void);      /* last refusal / HIP error on this thread */
int mi_sync(mi_stream stream);        /* hipStreamSynchronize; ctx.synchronize() in the reference */
int mi_block_elements(int kind);      /* quant.mojo:78 */
int mi_block_bytes(int kind);         /* quant.mojo:97 */
int64_t mi_row_bytes(int kind, int32_t cols); /* tensor.mojo:204-229 row geometry, -1 if invalid */

/* ---- bit-exact dequant ----------------------------------------------------
 * out[i] = value i of the run of `count` values at w (count a whole number
 * of blocks).  Bit-identical to src/molla/nn/quant.mojo:412 dequant_run. */
int mi_dequant(mi_stream stream, int kind, const void* w, int64_t count, float* out);

/* ---- matvec (src/molla/nn/gpu.mojo:2148 device_matvec_into and
 *      :2945 device_matmul_into) -------------------------------------------
 * For t < tokens, r < rows:  dot = row r of W . x[t*cols : (t+1)*cols]
 * and y[t*rows + r] is written through the epilogue.  `y` is already offset
 * by the caller (the reference's `at`, gpu.mojo:201-223).  aux may be NULL
 * unless epi has BIAS or GLU.  tokens 1..8 (batch-1 decode up to the batch-8
 * head of the configs).  Activations are carried as 23-bit block fixed point
 * per 32 values (three int8 limbs), so every product is an exact integer dot;
 * the result agrees with the fp32 host path to ~1e-7 relative.
 * Workspace: mi_matvec_workspace(cols, tokens) bytes, 256-byte aligned (at
 * 2..8 tokens the activations twice over: the int8-limb form and, for the
 * f16 matrix-core tile, the same integers as pairs of halves).
 *
 * tokens 9..65536 is the prefill matmul (device_matmul_into at a prompt
 * chunk, gpu.mojo:1695 PREFILL_CHUNK; the tile of gpu.mojo:2665): matrix
 * cores on half-precision operands, the activations split into two halves
 * (22 bits) and the weights as the exact integer codes of their blocks, so
 * the result stays within ~1e-6 relative of the fp32 host dot.  It needs
 * mi_matvec_workspace(cols, tokens) bytes; given mi_matmul_workspace(rows,
 * cols, tokens) it may also split long reductions across more blocks, and so
 * may a batch of 2..8 tokens of a Q4_K matrix with few rows for its long K
 * (the down projection, 4096 x 14336). */
size_t mi_matvec_workspace(int32_t cols, int32_t tokens);
size_t mi_matmul_workspace(int32_t rows, int32_t cols, int32_t tokens);
int mi_matvec(mi_stream stream, int kind, const void* w, int64_t row_bytes,
              int32_t rows, int32_t cols, const float* x, int32_t tokens,
              float* y, int32_t epi, const float* aux, void* work, size_t work_bytes);

/* No counterpart in the reference: mi_matvec without a workspace argument,
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops that forbid hipMalloc).  The workspace is a static
 * per-device scratch array of MI_MATVEC_NOALLOC_BYTES, whose address is
 * resolved once per device on first use; the call itself allocates nothing.
 * Shapes whose mi_matvec_workspace(cols, tokens) is larger are refused
 * (MI_ERR_WORKSPACE).  Every call on one GPU shares that array: calls that
 * overlap on one GPU race.  The array is reserved on every GPU the library is
 * loaded on, 32 MiB each, whether or not this entry point is called.  The
 * first call on a device resolves the array's address (hipGetSymbolAddress,
 * which may load the code object): make that first call outside graph
 * capture; later calls may be captured. */
#define MI_MATVEC_NOALLOC_BYTES (32u << 20)
int mi_matvec_noalloc(mi_stream stream, int kind, const void* w, int64_t row_bytes,
                      int32_t rows, int32_t cols, const float* x, int32_t tokens,
                      float* y, int32_t epi, const float* aux);

/* The two halves of mi_matvec, for callers that reuse one quantized
 * activation across several matrices (q/k/v share the normed input; gate and
 * up share it too).  xq holds mi_matvec_workspace(cols, tokens) bytes. */
int mi_quantize(mi_stream stream, const float* x, int32_t cols, int32_t tokens, void* xq);
int mi_matvec_xq(mi_stream stream, int kind, const void* w, int64_t row_bytes,
                 int32_t rows, int32_t cols, const void* xq, int32_t tokens,
                 float* y, int32_t epi, const float* aux);

/* ---- block ops (src/molla/nn/gpu_ops.mojo) --------------------------------
 * rms_norm: out[t] = x[t] * rsqrt(mean(x[t]^2) + eps) * gain, sum of squares in
 * float64 as the host does (kernel.mojo:432-467).  If xq is non-NULL the
 * normalised row is also quantized for a following mi_matvec_xq (xq holds
 * mi_matvec_workspace(n, tokens) bytes). */
int mi_rms_norm(mi_stream stream, const float* x, const float* gain, int32_t n,
                int32_t tokens, float eps, float* out, void* xq);

/* Host-side helper (no device work): the rope frequency step per pair,
 * f32(exp(f64(-2p/dim) * log(base))) -- src/molla/nn/rope.mojo:230 step_table.
 * steps_host has dim/2 floats. */
void mi_rope_steps(float* steps_host, int32_t dim, float base);

/* Rotate `heads` heads of head_dim laid end to end in x (rows of row_stride
 * floats, one per token) at positions pos[t] (device int32), adjacent pairs
 * when neox == 0 (Llama).  cos/sin are taken in float64 of the float32 angle
 * pos*step, as rope.mojo:253-285 does.  steps: device f32[dim/2]. */
int mi_rope(mi_stream stream, float* x, int32_t heads, int32_t head_dim, int32_t dim,
            int32_t neox, const float* steps, const int32_t* pos, int32_t tokens,
            int64_t row_stride);

/* f32 k/v rows -> f16 cache rows at slot: cache[slot*kv_width + i] = half(src[i]).
 * gpu_ops.mojo:1491 store_kv_kernel. */
int mi_store_kv(mi_stream stream, const float* k, const float* v, int32_t kv_width,
                uint16_t* k_cache, uint16_t* v_cache, int32_t slot);

/* One query (heads*head_dim f32) against `count` cached positions (f16,
 * [pos][kv_heads][head_dim]); GQA with group = heads/kv_heads; scores scaled,
 * softmax with the maximum subtracted, weighted sum of values.
 * attention.mojo:144 attend; split over key slices with a flash-style merge
 * like gpu_ops.mojo:929/1104.  Workspace: mi_attend_workspace(heads, head_dim, count). */
size_t mi_attend_workspace(int32_t heads, int32_t head_dim, int32_t count);
int mi_attend(mi_stream stream, const float* q, const uint16_t* k_cache,
              const uint16_t* v_cache, int32_t heads, int32_t kv_heads,
              int32_t head_dim, float scale, int32_t count, float* out,
              void* work, size_t work_bytes);

/* KV cache forms (src/molla/nn/repack.mojo:174-218).  F16: a position is
 * kv_width halves.  Q8: kv_width signed bytes (q8_0 quants), then kv_width/32
 * float16 block factors, the row rounded up to a multiple of 8 halves; a
 * value reads back as float(q) * float(factor).  Rows are counted in halves
 * at either form: a cache of n positions is n * mi_cache_row(form, kv_width)
 * halves. */
enum { MI_CACHE_F16 = 0, MI_CACHE_Q8 = 1 };

/* Halves one position occupies (repack.mojo:221 cache_row), or -1 for an
 * unknown form or a q8_0 width that is not whole 32-value blocks. */
int32_t mi_cache_row(int32_t form, int32_t kv_width);

/* mi_store_kv into a cache of either form at position slot (a q8_0 row is
 * encoded by gpu_ops.mojo:1531 store_kv_q8_kernel's rule: factor amax/127
 * stored as a half, quants rounded half away from zero). */
int mi_store_kv_form(mi_stream stream, int32_t form, const float* k, const float* v, int32_t kv_width,
                     uint16_t* k_cache, uint16_t* v_cache, int32_t slot);

/* mi_attend over a cache of either form (gpu_ops.mojo:678 attend_kernel's
 * `form`); same workspace. */
int mi_attend_form(mi_stream stream, int32_t form, const float* q, const uint16_t* k_cache,
                   const uint16_t* v_cache, int32_t heads, int32_t kv_heads, int32_t head_dim, float scale,
                   int32_t count, float* out, void* work, size_t work_bytes);

/* Index of the maximum of x[t*n : (t+1)*n] for each t, ties to the lower
 * index (kernel.mojo:571 argmax, gpu_ops.mojo:408). out: device int32[tokens]. */
int mi_argmax(mi_stream stream, const float* x, int32_t n, int32_t tokens, int32_t* out);

/* The same argmax spread over the chip: each row in 64 parts, the parts'
 * winners left in `work` (mi_argmax_workspace(n, tokens) bytes, 8-byte
 * aligned) and folded in part order, ties to the lower index as above.
 * The single-block form (the reference's, gpu_ops.mojo:408) is bound by one
 * compute unit's bandwidth on a vocabulary-sized row.  Optionally the
 * decode loop's bookkeeping in the same launch (engine/device.mojo:917 pick
 * and the advance after it): next_ids[t] = out[t] and next_pos[t] += 1 when
 * those pointers are not NULL. */
size_t mi_argmax_workspace(int32_t n, int32_t tokens);
int mi_argmax_ws(mi_stream stream, const float* x, int32_t n, int32_t tokens, int32_t* out, void* work,
                 size_t work_bytes, int32_t* next_ids, int32_t* next_pos);

/* out[t] = row ids[t] of an f32 embedding (model.mojo:102 embed). */
int mi_embed(mi_stream stream, const float* embedding, int32_t vocab, int32_t width,
             const int32_t* ids, int32_t tokens, float* out);

/* Which kernel mi_matvec runs for a shape (no reference counterpart: an
 * introspection hook for tests and tools).  Assumes the weight rows are
 * cols / block_elements whole blocks at a 256-byte aligned address and a
 * workspace of work_bytes.  Returns one of MI_ROUTE_*, with
 * MI_ROUTE_SPLIT_BIT set when the matrix is split over K (the parts added
 * by a second launch), or a negative MI_ERR_* code; *part_cols (may be NULL)
 * gets the columns of one part (cols when not split). */
enum {
  MI_ROUTE_ROWS = 1,      /* batch-1 row kernel, Q4_K Q4_0 Q4_1 Q5_0 Q5_1 Q5_K Q8_0 */
  MI_ROUTE_Q6K_ROWS = 2,  /* batch-1 Q6_K row kernel */
  MI_ROUTE_HTILE = 3,     /* 2..8 tokens, f16 matrix-core tile, Q4_K / Q6_K */
  MI_ROUTE_Q4K_TILE = 4,  /* 2..8 tokens, int8 matrix-core tile, Q4_K */
  MI_ROUTE_B32_TILE = 5,  /* 2..8 tokens, int8 matrix-core tile, Q4_0 / Q8_0 */
  MI_ROUTE_Q6K_TILE = 6,  /* 2..8 tokens, int8 matrix-core tile, Q6_K */
  MI_ROUTE_GENERAL = 7,   /* the general kernel, any kind */
  MI_ROUTE_PREFILL = 8,   /* above 8 tokens, the prefill matmul */
  MI_ROUTE_SPLIT_BIT = 16
};
int mi_matvec_route(int kind, int32_t rows, int32_t cols, int32_t tokens, size_t work_bytes, int32_t* part_cols);

/* ---- decoder layer (src/molla/nn/gpu_block.mojo:899 device_layer) -------- */

typedef struct {
  const void* data; /* device pointer to GGUF blocks */
  int32_t kind;
  int32_t rows;
  int32_t cols;
  int64_t row_bytes;
} mi_weight;

typedef struct {
  int32_t width;    /* residual stream, 4096 for an 8B */
  int32_t hidden;   /* MLP inner width, 14336 */
  int32_t heads, kv_heads, head_dim; /* 32, 8, 128 */
  int32_t rope_dim; /* rotated elements per head, usually head_dim */
  int32_t neox;     /* 0 = adjacent pairs (Llama), 1 = half-split pairs */
  float eps;        /* RMSNorm epsilon */
  float attn_scale; /* usually 1/sqrt(head_dim) */
  const float* attn_norm; /* device f32[width] */
  const float* ffn_norm;  /* device f32[width] */
  const float* rope_steps; /* device f32[rope_dim/2] from mi_rope_steps */
  mi_weight wq, wk, wv, wo, gate, up, down;
  const float* rope_factors; /* device f32[rope_dim/2]: rope_freqs.weight of a
                                Llama 3.1 file (each pair's angle is divided by
                                its factor, rope.mojo:253), or NULL for none */
  int32_t cache_form;        /* MI_CACHE_F16 (0, the default) or MI_CACHE_Q8; the
                                caches' cache_stride counts halves either way */
  /* The optional parts of other families (block.mojo:61 BlockSpec, :116
   * LayerWeights; on the device gpu_block.mojo:678-896).  NULL / 0 in every
   * one of them is the Llama layer above. */
  const float* q_bias;         /* device f32[heads*head_dim], with k_bias and v_bias
                                  (f32[kv_heads*head_dim]): Qwen 2's projection biases */
  const float* k_bias;
  const float* v_bias;
  const float* q_norm;         /* device f32[head_dim], with k_norm: each head of q and
                                  k RMS-normed before rope (Qwen 3) */
  const float* k_norm;
  const float* attn_post_norm; /* device f32[width]: wo's output normed before the
                                  residual add (Gemma 2); likewise ffn_post_norm on down's */
  const float* ffn_post_norm;
  int32_t ungated;             /* 1: the MLP is down(act(up(x))), gate unused */
  int32_t act;                 /* 0 silu, MI_ACT_GELU gelu (tanh form, kernel.mojo:499) */
  /* Chaining layers at 2..8 tokens (no counterpart in the reference, which
   * norms each layer's input in that layer): with next_norm set (device
   * f32[width], the next layer's attn_norm), the layer also leaves that
   * RMSNorm of its output in the workspace, in the forms its first matvec
   * reads; a call with prenormed = 1 on the same workspace, tokens and
   * shapes then starts from it instead of norming resid itself.  Where the
   * down projection runs split over K on the f16 tile, the residual add and
   * that norm are one launch.  Both are ignored at 1 token and above 8. */
  const float* next_norm;
  int32_t prenormed;
} mi_layer_desc;

/* One Llama layer for `tokens` independent sequences (batch decode, one token
 * each), in place on resid[t*width ...].  Above 8 tokens (up to 65536; a
 * prompt chunk when cache_stride is 0, gpu_block.mojo:1654 forward over a
 * chunk) the same layer runs on f32 activations through the prefill matmul
 * (see mi_matvec) with rope, the cache store and attention per token;
 * mi_layer_workspace(desc, max_count, tokens) sizes it for that count.  Sequence t owns k_cache/v_cache at
 * t * cache_stride halves, laid out [slot][kv_heads*head_dim].  Its token sits
 * at position pos[t] (device int32[tokens], read by the kernels so a captured
 * graph can be replayed for the next token), which is also its cache slot (a
 * contiguous cache, where the reference's `slot` equals `pos`): the rotated key
 * and the value are written at slot pos[t] and attention runs over slots
 * 0..pos[t].  max_count bounds pos[t] + 1 and sizes the attention grid.
 * Order as block.mojo:466 layer: norm, q/k/v, rope q/k, store, attend,
 * wo (+residual), norm, up, gate (+silu gate), down (+residual). */
size_t mi_layer_workspace(const mi_layer_desc* desc, int32_t max_count, int32_t tokens);
int mi_decoder_layer(mi_stream stream, const mi_layer_desc* desc, float* resid,
                     uint16_t* k_cache, uint16_t* v_cache, int64_t cache_stride,
                     const int32_t* pos, int32_t max_count, int32_t tokens,
                     void* work, size_t work_bytes);

/* The same layer over a paged pool (gpu_ops.mojo:662 _row_of, gpu.mojo:571
 * DevicePaging): k_pool / v_pool hold cells of mi_cache_row(form, kv_width)
 * halves each, shared by every sequence; kv_index[t * index_stride + j] is
 * the cell holding position j of sequence t, or negative for a position the
 * sequence does not hold (masked out of attention).  The caller sets the
 * cell of the new position, kv_index[t * index_stride + pos[t]], before the
 * call; the rotated key and the value are written there.  index_stride 0
 * makes the tokens one sequence's chunk (the reference's `bases` all zero):
 * they share one list, sit at distinct positions pos[t], and each attends
 * over the positions up to its own, the chunk's earlier tokens included.
 * cache_stride 0 does the same for mi_decoder_layer. */
int mi_decoder_layer_paged(mi_stream stream, const mi_layer_desc* desc, float* resid, uint16_t* k_pool,
                           uint16_t* v_pool, const int32_t* kv_index, int64_t index_stride, const int32_t* pos,
                           int32_t max_count, int32_t tokens, void* work, size_t work_bytes);

#ifdef __cplusplus
}
#endif
#endif /* MOLLA_MI_H */
