/*
 * molla_oracle.h -- CPU restatement of molla's host decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the HIP kernels are
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and never as the thing measured or shipped.
 *
 * Every function follows one reference function operation for operation
 * (citations are to /root/reference, tamnd/molla v0.5.7).  Compile with
 * -ffp-contract=off and without -ffast-math so every float multiply and add is
 * rounded where the Mojo source rounds it.
 */
#ifndef MOLLA_ORACLE_H
#define MOLLA_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type numbers, src/molla/nn/quant.mojo:47-57 */
enum {
  OR_F32 = 0, OR_F16 = 1, OR_Q4_0 = 2, OR_Q4_1 = 3, OR_Q5_0 = 6, OR_Q5_1 = 7,
  OR_Q8_0 = 8, OR_Q4_K = 12, OR_Q5_K = 13, OR_Q6_K = 14, OR_BF16 = 30
};

int or_block_elements(int kind);                 /* quant.mojo:78  */
int or_block_bytes(int kind);                    /* quant.mojo:97  */
float or_f16(uint16_t bits);                     /* quant.mojo:135 */
uint16_t or_f32_to_f16(float v);                 /* RNE narrowing, device store_kv semantics */

/* Decode `count` values starting at p; 0 ok, -1 bad kind, -2 not whole blocks.
 * quant.mojo:412 dequant_run (per block: dequant_block :184). */
int or_dequant_run(int kind, const uint8_t* p, int64_t count, float* out);

/* Fused dot of one packed row with x (n values); kernel.mojo:75 row_dot. */
int or_row_dot(int kind, const uint8_t* p, const float* x, int64_t n, float* out);

/* y[r] = row_dot(row r, x); kernel.mojo:316 matvec.  threads>1 splits rows
 * over OpenMP threads (the courtesy upper bound; the reference is serial). */
int or_matvec(int kind, const uint8_t* w, int64_t row_bytes, int32_t rows,
              int32_t cols, const float* x, float* y, int32_t threads);

void or_rms_norm(float* out, const float* x, const float* gain, int32_t n, float eps); /* kernel.mojo:400 */
void or_softmax(float* x, int32_t n);            /* kernel.mojo:470 */
float or_silu(float v);                          /* kernel.mojo:494 */
float or_gelu(float v);                          /* kernel.mojo:499 */
void or_swiglu(float* gate, const float* up, int32_t n); /* kernel.mojo:512 */
int32_t or_argmax(const float* x, int32_t n);    /* kernel.mojo:571 */

/* rope.mojo:230 step_table; rope.mojo:253 angle; rope.mojo:294 rotate_scaled.
 * Plain rope (scale 1, no YaRN, attn_factor 1, no frequency factors). */
void or_rope_steps(float* steps, int32_t dim, float base);
void or_rope_angle(int32_t dim, float base, int32_t pos, int32_t pair, float* c, float* s);
void or_rotate_run(float* x, int32_t heads, int32_t head_dim, int32_t dim,
                   float base, int32_t neox, int32_t pos);
void or_rope_angle_scaled(int32_t dim, float base, int32_t pos, int32_t pair, float freq, float* c, float* s);
void or_rotate_run_scaled(float* x, int32_t heads, int32_t head_dim, int32_t dim,
                          float base, int32_t neox, int32_t pos, const float* factors);

/* attention.mojo:144 attend, contiguous run of `count` positions, no window,
 * no sinks, no softcap.  scores: scratch of `count` floats. */
void or_attend(int32_t heads, int32_t kv_heads, int32_t head_dim, float scale,
               const float* q, const float* keys, const float* values,
               int32_t count, float* out, float* scores);

typedef struct {
  const void* data;
  int32_t kind;
  int32_t rows;
  int32_t cols;
  int64_t row_bytes;
} or_weight;

typedef struct {
  int32_t width, hidden, heads, kv_heads, head_dim, rope_dim, neox;
  float eps, rope_base, attn_scale;
  const float* attn_norm;
  const float* ffn_norm;
  or_weight wq, wk, wv, wo, gate, up, down;
  const float* rope_factors; /* rope_dim/2 per-pair factors (rope_freqs.weight) or NULL */
  /* Optional parts of other families (block.mojo:61 BlockSpec, :116
   * LayerWeights); NULL / 0 is the Llama layer. */
  const float* q_bias;          /* q_width values (Qwen 2) */
  const float* k_bias;          /* kv_width */
  const float* v_bias;          /* kv_width */
  const float* q_norm;          /* head_dim gains, every query head (Qwen 3) */
  const float* k_norm;          /* head_dim gains, every key head */
  const float* attn_post_norm;  /* width gains on wo's output (Gemma 2) */
  const float* ffn_post_norm;   /* width gains on down's output */
  int32_t ungated;              /* 1: act(up(x)) instead of act(gate(x)) * up(x) */
  int32_t act;                  /* 0 silu, 1 gelu (tanh form, kernel.mojo:499) */
} or_layer;

/* block.mojo:466 layer (attention_layer :319 + mlp_layer :429), in place on x.
 * keys/values: f32 cache, one row of kv_heads*head_dim per slot.  When
 * f16_store is 1 the freshly rotated key and the value are rounded through
 * float16 before attending, which is what a device cache of halves holds.
 * threads as for or_matvec.  Returns 0 or a negative error. */
/* The values a q8_0 KV cache row reads back (float(q) * f16 factor per
 * 32-value block), in place; or_layer_step does this to the new key and value
 * when f16_store is 2. */
void or_q8_cache_round(float* v, int32_t n);
int or_layer_step(const or_layer* L, float* x, float* keys, float* values,
                  int32_t slot, int32_t pos, int32_t f16_store, int32_t threads);
/* One sublayer of it: parts 1 = attention_layer (block.mojo:319), 2 =
 * mlp_layer (:429), 3 = both (the same as or_layer_step). */
int or_layer_part(const or_layer* L, float* x, float* keys, float* values,
                  int32_t slot, int32_t pos, int32_t f16_store, int32_t threads, int32_t parts);

/* model.mojo:178 forward for a Llama stack with an f32 embedding:
 * embed (:102) -> layers -> head (:136).  keys[i]/values[i] per layer. */
int or_forward(const or_layer* layers, int32_t n_layers, const float* embedding,
               int32_t vocab, const float* output_norm, const or_weight* output,
               int32_t token, int32_t pos, int32_t slot, float** keys,
               float** values, int32_t f16_store, float* logits, int32_t threads);

/* tests/test_kernel.mojo:69-126: xorshift64 Rng and _blocks, so fixtures are
 * byte-identical to the inputs the reference's own tests build. */
uint64_t or_xorshift_next(uint64_t* state);
void or_test_blocks(int kind, int32_t count, uint64_t seed, uint8_t* out);
void or_test_units(uint64_t seed, int32_t n, float* out);

#ifdef __cplusplus
}
#endif
#endif
