// layer.cpp -- one Llama decoder layer on the device, as a sequence of
// launches on the caller's stream (src/molla/nn/gpu_block.mojo:899
// device_layer, whose host twin is src/molla/nn/block.mojo:466 layer):
//
//   rms_norm(attn_norm) -> xq                       (norm writes the matvec input form)
//   q | k | v = W{q,k,v} . xq                        (three projections, one fused row)
//   rope q, k; k, v -> f16 cache at slot pos[t]
//   attend over slots 0..pos[t] -> xq                (split-K + merge; merge writes xq)
//   resid += Wo . xq                                 (EPI_ADD)
//   rms_norm(ffn_norm) -> xq
//   up = Wup . xq;  gate = silu(Wgate . xq) * up     (EPI_GLU)
//   gate -> xq;  resid += Wdown . xq                 (EPI_ADD)
//
// Workspace (mi_layer_workspace), every piece 256-byte aligned:
//   xq     4 * max(width, q_width, hidden) * tokens   activation in matvec form
//   qkv    (q_width + 2 * kv_width) * tokens floats
//   up     hidden * tokens floats
//   gate   hidden * tokens floats
//   attn   attention slices (attend_workspace)
//   trig   rope (cos, sin) of this position
//   xq2    4 * hidden * tokens: the down projection's input, when the gate/up
//          launch writes it (it cannot share xq, which that launch reads)
// Above 8 tokens (prefill_layer) the activations stay f32 and the pieces are
// xn, qkv, attention output, up, act(gate)*up, attention slices and the
// prefill matmul's own workspace (prefill_carve).
#include <algorithm>

#include "mi_internal.h"
#include "matvec_rows.h"

namespace mi {
int check_weight(const char* name, int kind, const void* w, int64_t row_bytes, int32_t rows, int32_t cols);
}

using namespace mi;

namespace {

size_t up256(size_t v) { return (v + 255) & ~(size_t)255; }

struct Carve {
  size_t xq, qkv, up, gate, attn, trig, xq2, part, total;
};

Carve carve(const mi_layer_desc* d, int32_t max_count, int32_t tokens) {
  const int64_t qw = (int64_t)d->heads * d->head_dim, kvw = (int64_t)d->kv_heads * d->head_dim;
  const int64_t widest = std::max<int64_t>({d->width, qw, d->hidden});
  Carve c;
  size_t at = 0;
  c.xq = at;  // at 2..8 tokens followed by the hx form (for wo's f16 matrix-core tile)
  at += up256((size_t)xq_token_bytes((int32_t)widest) * tokens * (tokens > 1 ? 2 : 1));
  c.qkv = at;
  at += up256(sizeof(float) * (size_t)(qw + 2 * kvw) * tokens);
  c.up = at;
  at += up256(sizeof(float) * (size_t)d->hidden * tokens);
  c.gate = at;
  at += up256(sizeof(float) * (size_t)d->hidden * tokens);
  c.attn = at;
  at += up256(attend_workspace(d->heads, d->head_dim, max_count, tokens));
  c.trig = at;
  at += up256(sizeof(float) * (size_t)d->rope_dim);
  c.xq2 = at;  // down's input; at 2..8 tokens followed by its hx form
  at += up256((size_t)xq_token_bytes(d->hidden) * tokens * (tokens > 1 ? 2 : 1));
  c.part = at;  // split-K partial sums of the down projection (batch 2..8)
  at += tokens > 1 ? up256(std::max({q4k_tile_split_bytes(d->width, tokens),
                                     htile_split_bytes(d->width, d->hidden, tokens),
                                     htile_split_bytes(d->width, d->heads * d->head_dim, tokens, 2)}))
                   : 0;
  c.total = at;
  return c;
}

// A prefill chunk (tokens > 8): f32 activations for the prefill matmul.
struct PrefillCarve {
  size_t xn, qkv, attn_out, up, h, attn, mm, total;
};

PrefillCarve prefill_carve(const mi_layer_desc* d, int32_t max_count, int32_t tokens) {
  const int64_t qw = (int64_t)d->heads * d->head_dim, kvw = (int64_t)d->kv_heads * d->head_dim;
  PrefillCarve c;
  size_t at = 0;
  c.xn = at;
  at += up256(sizeof(float) * (size_t)d->width * tokens);
  c.qkv = at;
  at += up256(sizeof(float) * (size_t)(qw + 2 * kvw) * tokens);
  c.attn_out = at;
  at += up256(sizeof(float) * (size_t)qw * tokens);
  c.up = at;
  at += up256(sizeof(float) * (size_t)d->hidden * tokens);
  c.h = at;
  at += up256(sizeof(float) * (size_t)d->hidden * tokens);
  c.attn = at;
  at += up256(attend_workspace(d->heads, d->head_dim, max_count, tokens));
  c.mm = at;
  size_t mm = 0;
  const int32_t shapes[5][2] = {{(int32_t)(qw + 2 * kvw), d->width}, {(int32_t)qw, d->width},
                                {d->width, (int32_t)qw}, {d->hidden, d->width}, {d->width, d->hidden}};
  for (auto& sh : shapes) mm = std::max(mm, prefill_workspace(sh[0], sh[1], tokens));
  at += up256(mm);
  c.total = at;
  return c;
}

int check_desc(const mi_layer_desc* d) {
  if (!d) return fail(MI_ERR_ARG, "layer: null descriptor");
  if (d->width <= 0 || d->hidden <= 0 || d->width % 256 || d->hidden % 256)
    return fail(MI_ERR_SHAPE, "layer: width %d / hidden %d must be positive multiples of 256", d->width,
                d->hidden);
  if (d->heads <= 0 || d->kv_heads <= 0 || d->heads % d->kv_heads)
    return fail(MI_ERR_SHAPE, "layer: %d query heads over %d key heads", d->heads, d->kv_heads);
  const int group = d->heads / d->kv_heads;
  if (group != 1 && group != 2 && group != 4 && group != 8)
    return fail(MI_ERR_SHAPE, "layer: %d query heads per key head is not 1, 2, 4 or 8", group);
  if (d->head_dim <= 0 || d->head_dim % 32 || d->head_dim > 512)
    return fail(MI_ERR_SHAPE, "layer: head_dim %d", d->head_dim);
  if (cache_row(d->cache_form, d->kv_heads * d->head_dim) < 0)
    return fail(MI_ERR_SHAPE, "layer: cache form %d has no row for %d key heads of %d", d->cache_form, d->kv_heads,
                d->head_dim);
  if (d->rope_dim <= 0 || d->rope_dim % 2 || d->rope_dim > d->head_dim)
    return fail(MI_ERR_SHAPE, "layer: rope_dim %d in heads of %d", d->rope_dim, d->head_dim);
  if (!(d->eps > 0.0f)) return fail(MI_ERR_ARG, "layer: a norm epsilon has to be positive");
  if (!d->attn_norm || !d->ffn_norm || !d->rope_steps) return fail(MI_ERR_ARG, "layer: null norm or rope table");
  const int32_t qw = d->heads * d->head_dim, kvw = d->kv_heads * d->head_dim;
  // block.mojo:116 LayerWeights.check: the optional parts come whole or not at all
  const int biases = !!d->q_bias + !!d->k_bias + !!d->v_bias;
  if (biases != 0 && biases != 3) return fail(MI_ERR_ARG, "layer: q, k and v biases come together (%d of 3)", biases);
  if (!d->q_norm != !d->k_norm) return fail(MI_ERR_ARG, "layer: q and k norms come together");
  if (d->ungated != 0 && d->ungated != 1) return fail(MI_ERR_ARG, "layer: ungated is 0 or 1, not %d", d->ungated);
  if (d->act != 0 && d->act != MI_ACT_GELU) return fail(MI_ERR_ARG, "layer: act %d is neither silu (0) nor gelu", d->act);
  struct {
    const char* name;
    const mi_weight& w;
    int32_t rows, cols;
  } want[] = {{"wq", d->wq, qw, d->width},       {"wk", d->wk, kvw, d->width},
              {"wv", d->wv, kvw, d->width},      {"wo", d->wo, d->width, qw},
              {"gate", d->gate, d->hidden, d->width}, {"up", d->up, d->hidden, d->width},
              {"down", d->down, d->width, d->hidden}};
  for (auto& e : want) {
    if (d->ungated && &e.w == &d->gate) continue;  // act(up(x)): no gate
    // block.mojo:230-247 _shape: a projection of the wrong size is refused.
    if (e.w.rows != e.rows || e.w.cols != e.cols)
      return fail(MI_ERR_SHAPE, "layer: %s is %d x %d where the layer wants %d x %d", e.name, e.w.rows,
                  e.w.cols, e.rows, e.cols);
    int rc = check_weight(e.name, e.w.kind, e.w.data, e.w.row_bytes, e.w.rows, e.w.cols);
    if (rc) return rc;
  }
  return MI_OK;
}

// Whether the layer uses any part beyond the Llama layer (q|k|v biases,
// q/k norms, post norms, a non-gated or gelu MLP).
bool extended(const mi_layer_desc* d) {
  return d->q_bias || d->q_norm || d->attn_post_norm || d->ffn_post_norm || d->ungated || d->act;
}

}  // namespace

// The layer with the optional parts of other families at 1..8 tokens, as
// gpu_block.mojo:678 device_attention and :846 device_mlp run it: norm,
// q/k/v (bias epilogue), per-head q/k norms, rope and the cache store,
// attention, wo (then the post norm and the residual add, or the add
// epilogue), norm, up and gate (GLU epilogue, silu or gelu) or up and the
// activation, down (likewise).  Each part is its own launch; the fused
// Llama kernels stay for the Llama layer.
static int extended_layer(hipStream_t s, const mi_layer_desc* d, float* resid, uint16_t* k_cache,
                          uint16_t* v_cache, int64_t cache_stride, const int32_t* kv_index, int64_t index_stride,
                          const int32_t* pos, int32_t max_count, int32_t tokens, char* base, const Carve& c,
                          bool pre) {
  void* xq = base + c.xq;
  void* xq2 = base + c.xq2;
  float* qkv = (float*)(base + c.qkv);
  float* up = (float*)(base + c.up);
  float* gate = (float*)(base + c.gate);
  void* attn = base + c.attn;
  const int32_t qw = d->heads * d->head_dim, kvw = d->kv_heads * d->head_dim;
  const int64_t qkv_stride = qw + 2 * (int64_t)kvw;
  const int32_t bias = d->q_bias ? MI_EPI_BIAS : MI_EPI_NONE;
  int rc;
  // attention_layer (block.mojo:319)
  if (!pre && (rc = launch_rms_norm(s, resid, d->attn_norm, d->width, tokens, d->eps, nullptr, xq))) return rc;
  if ((rc = launch_matvec(s, d->wq.kind, d->wq.data, d->wq.row_bytes, qw, d->width, xq, tokens, qkv, qkv_stride,
                          bias, d->q_bias)))
    return rc;
  if ((rc = launch_matvec(s, d->wk.kind, d->wk.data, d->wk.row_bytes, kvw, d->width, xq, tokens, qkv + qw,
                          qkv_stride, bias, d->k_bias)))
    return rc;
  if ((rc = launch_matvec(s, d->wv.kind, d->wv.data, d->wv.row_bytes, kvw, d->width, xq, tokens, qkv + qw + kvw,
                          qkv_stride, bias, d->v_bias)))
    return rc;
  if (d->q_norm) {
    if ((rc = launch_head_norm(s, qkv, d->heads, d->head_dim, tokens, qkv_stride, d->q_norm, d->eps))) return rc;
    if ((rc = launch_head_norm(s, qkv + qw, d->kv_heads, d->head_dim, tokens, qkv_stride, d->k_norm, d->eps)))
      return rc;
  }
  if ((rc = launch_rope_store(s, qkv, d->heads, d->kv_heads, d->head_dim, d->rope_dim, d->neox, d->rope_steps, pos,
                              tokens, qkv_stride, k_cache, v_cache, cache_stride, d->rope_factors, d->cache_form,
                              kv_index, index_stride)))
    return rc;
  if ((rc = launch_attend(s, qkv, qkv_stride, k_cache, v_cache, cache_stride, d->heads, d->kv_heads, d->head_dim,
                          d->attn_scale, pos, -1, max_count, tokens, nullptr, xq, attn, d->cache_form, kv_index,
                          index_stride)))
    return rc;
  if (d->attn_post_norm) {
    // wo into a scratch row (the up buffer is free until the MLP), normed into the stream
    if ((rc = launch_matvec(s, d->wo.kind, d->wo.data, d->wo.row_bytes, d->width, qw, xq, tokens, up, d->width,
                            MI_EPI_NONE, nullptr)))
      return rc;
    if ((rc = launch_norm_add(s, resid, up, d->width, tokens, d->attn_post_norm, d->eps))) return rc;
  } else if ((rc = launch_matvec(s, d->wo.kind, d->wo.data, d->wo.row_bytes, d->width, qw, xq, tokens, resid,
                                 d->width, MI_EPI_ADD, nullptr))) {
    return rc;
  }
  // mlp_layer (block.mojo:429)
  if ((rc = launch_rms_norm(s, resid, d->ffn_norm, d->width, tokens, d->eps, nullptr, xq))) return rc;
  if ((rc = launch_matvec(s, d->up.kind, d->up.data, d->up.row_bytes, d->hidden, d->width, xq, tokens, up,
                          d->hidden, MI_EPI_NONE, nullptr)))
    return rc;
  float* h = up;
  if (d->ungated) {
    if ((rc = launch_act(s, up, (int64_t)d->hidden * tokens, d->act))) return rc;
  } else {
    if ((rc = launch_matvec(s, d->gate.kind, d->gate.data, d->gate.row_bytes, d->hidden, d->width, xq, tokens, gate,
                            d->hidden, MI_EPI_GLU | d->act, up)))
      return rc;
    h = gate;
  }
  if ((rc = launch_quantize(s, h, d->hidden, tokens, xq2))) return rc;
  if (d->ffn_post_norm) {
    float* tmp = h == up ? gate : up;  // whichever of the two the activation is not in
    if ((rc = launch_matvec(s, d->down.kind, d->down.data, d->down.row_bytes, d->width, d->hidden, xq2, tokens, tmp,
                            d->width, MI_EPI_NONE, nullptr)))
      return rc;
    return launch_norm_add(s, resid, tmp, d->width, tokens, d->ffn_post_norm, d->eps);
  }
  return launch_matvec(s, d->down.kind, d->down.data, d->down.row_bytes, d->width, d->hidden, xq2, tokens, resid,
                       d->width, MI_EPI_ADD, nullptr);
}

// The layer over a chunk of more than 8 tokens (a prompt chunk, cache stride
// or index stride 0, or that many sequences): the same chain on f32
// activations through the prefill matmul (prefill.hip), the norms writing f32
// rows, rope and the cache store per token, attention per token over the
// positions up to its own (the chunk's earlier tokens included).  The gate
// projection's GLU epilogue reads the up projection's output.
static int prefill_layer(hipStream_t s, const mi_layer_desc* d, float* resid, uint16_t* k_cache, uint16_t* v_cache,
                         int64_t cache_stride, const int32_t* kv_index, int64_t index_stride, const int32_t* pos,
                         int32_t max_count, int32_t tokens, void* work, size_t work_bytes) {
  const PrefillCarve c = prefill_carve(d, max_count, tokens);
  if (work_bytes < c.total)
    return fail(MI_ERR_WORKSPACE, "layer: workspace of %zu bytes (256-aligned), %zu needed", work_bytes, c.total);
  char* base = (char*)work;
  float* xn = (float*)(base + c.xn);
  float* qkv = (float*)(base + c.qkv);
  float* attn_out = (float*)(base + c.attn_out);
  float* up = (float*)(base + c.up);
  float* h = (float*)(base + c.h);
  void* attn = base + c.attn;
  void* mm = base + c.mm;
  const size_t mm_bytes = c.total - c.mm;
  const int32_t qw = d->heads * d->head_dim, kvw = d->kv_heads * d->head_dim;
  const int64_t qkv_stride = qw + 2 * (int64_t)kvw;
  int rc;
  auto mat = [&](const mi_weight& w, int32_t rows, int32_t cols, const float* x, float* y, int64_t ldy, int32_t epi,
                 const float* aux) {
    return matmul_tokens(s, w.kind, w.data, w.row_bytes, rows, cols, x, tokens, y, ldy, epi, aux, mm, mm_bytes);
  };
  // attention_layer (block.mojo:319)
  auto tile = [&](const mi_weight& w) { return prefill_fits(w.kind, w.cols, w.row_bytes, w.data); };
  if ((rc = launch_rms_norm(s, resid, d->attn_norm, d->width, tokens, d->eps, xn, nullptr))) return rc;
  if (d->q_bias) {
    // each projection with its bias in the epilogue (block.mojo:363-366)
    if ((rc = mat(d->wq, qw, d->width, xn, qkv, qkv_stride, MI_EPI_BIAS, d->q_bias))) return rc;
    if ((rc = mat(d->wk, kvw, d->width, xn, qkv + qw, qkv_stride, MI_EPI_BIAS, d->k_bias))) return rc;
    if ((rc = mat(d->wv, kvw, d->width, xn, qkv + qw + kvw, qkv_stride, MI_EPI_BIAS, d->v_bias))) return rc;
  } else if (tile(d->wq) && tile(d->wk) && tile(d->wv)) {
    // one activation prep for q, k and v; consecutive projections of one
    // kind as one launch over their rows end to end (q|k|v, or q|k and v
    // when v is of another kind, as in Q4_K_M files)
    if ((rc = prefill_prepare(s, xn, d->width, tokens, mm))) return rc;
    const mi_weight* ws[3] = {&d->wq, &d->wk, &d->wv};
    const int32_t ends[3] = {qw, qw + kvw, qw + 2 * kvw};
    for (int i = 0; i < 3;) {
      int j = i + 1;
      while (j < 3 && ws[j]->kind == ws[i]->kind) j++;
      RowSegs sg{};
      const int32_t base_row = i == 0 ? 0 : ends[i - 1];
      for (int k = i; k < j; k++) {
        sg.w[k - i] = (const uint8_t*)ws[k]->data;
        sg.rb[k - i] = ws[k]->row_bytes;
        sg.end[k - i] = ends[k] - base_row;
      }
      sg.nseg = j - i;
      if ((rc = launch_prefill_segs(s, ws[i]->kind, sg, d->width, tokens, qkv + base_row, qkv_stride, MI_EPI_NONE,
                                    nullptr, mm, mm_bytes)))
        return rc;
      i = j;
    }
  } else {
    if ((rc = mat(d->wq, qw, d->width, xn, qkv, qkv_stride, MI_EPI_NONE, nullptr))) return rc;
    if ((rc = mat(d->wk, kvw, d->width, xn, qkv + qw, qkv_stride, MI_EPI_NONE, nullptr))) return rc;
    if ((rc = mat(d->wv, kvw, d->width, xn, qkv + qw + kvw, qkv_stride, MI_EPI_NONE, nullptr))) return rc;
  }
  if (d->q_norm) {  // each head of q and k normed before rope (block.mojo:367-384)
    if ((rc = launch_head_norm(s, qkv, d->heads, d->head_dim, tokens, qkv_stride, d->q_norm, d->eps))) return rc;
    if ((rc = launch_head_norm(s, qkv + qw, d->kv_heads, d->head_dim, tokens, qkv_stride, d->k_norm, d->eps)))
      return rc;
  }
  if ((rc = launch_rope_store(s, qkv, d->heads, d->kv_heads, d->head_dim, d->rope_dim, d->neox, d->rope_steps, pos,
                              tokens, qkv_stride, k_cache, v_cache, cache_stride, d->rope_factors, d->cache_form,
                              kv_index, index_stride)))
    return rc;
  if ((rc = launch_attend(s, qkv, qkv_stride, k_cache, v_cache, cache_stride, d->heads, d->kv_heads, d->head_dim,
                          d->attn_scale, pos, -1, max_count, tokens, attn_out, nullptr, attn, d->cache_form,
                          kv_index, index_stride)))
    return rc;
  if (d->attn_post_norm) {  // wo into xn (free once q, k, v are made), normed into the stream
    if ((rc = mat(d->wo, d->width, qw, attn_out, xn, d->width, MI_EPI_NONE, nullptr))) return rc;
    if ((rc = launch_norm_add(s, resid, xn, d->width, tokens, d->attn_post_norm, d->eps))) return rc;
  } else if ((rc = mat(d->wo, d->width, qw, attn_out, resid, d->width, MI_EPI_ADD, nullptr))) {
    return rc;
  }
  // mlp_layer (block.mojo:429)
  if ((rc = launch_rms_norm(s, resid, d->ffn_norm, d->width, tokens, d->eps, xn, nullptr))) return rc;
  if (d->ungated || d->act || d->ffn_post_norm) {
    if ((rc = mat(d->up, d->hidden, d->width, xn, up, d->hidden, MI_EPI_NONE, nullptr))) return rc;
    float* act = up;
    if (d->ungated) {
      if ((rc = launch_act(s, up, (int64_t)d->hidden * tokens, d->act))) return rc;
    } else {
      if ((rc = mat(d->gate, d->hidden, d->width, xn, h, d->hidden, MI_EPI_GLU | d->act, up))) return rc;
      act = h;
    }
    if (!d->ffn_post_norm) return mat(d->down, d->width, d->hidden, act, resid, d->width, MI_EPI_ADD, nullptr);
    if ((rc = mat(d->down, d->width, d->hidden, act, xn, d->width, MI_EPI_NONE, nullptr))) return rc;
    return launch_norm_add(s, resid, xn, d->width, tokens, d->ffn_post_norm, d->eps);
  }
  if (tile(d->up) && tile(d->gate)) {  // one activation prep for both
    if ((rc = prefill_prepare(s, xn, d->width, tokens, mm))) return rc;
    if ((rc = launch_prefill_segs(s, d->up.kind, rows::one_matrix(d->up.data, d->up.row_bytes, d->hidden),
                                  d->width, tokens, up, d->hidden, MI_EPI_NONE, nullptr, mm, mm_bytes)))
      return rc;
    if ((rc = launch_prefill_segs(s, d->gate.kind, rows::one_matrix(d->gate.data, d->gate.row_bytes, d->hidden),
                                  d->width, tokens, h, d->hidden, MI_EPI_GLU, up, mm, mm_bytes)))
      return rc;
  } else {
    if ((rc = mat(d->up, d->hidden, d->width, xn, up, d->hidden, MI_EPI_NONE, nullptr))) return rc;
    if ((rc = mat(d->gate, d->hidden, d->width, xn, h, d->hidden, MI_EPI_GLU, up))) return rc;
  }
  return mat(d->down, d->width, d->hidden, h, resid, d->width, MI_EPI_ADD, nullptr);
}

// The next layer's attention norm, when the caller asks for it (gain set):
// done once a launch of this layer has written it.
struct NextNorm {
  const float* gain;
  bool done;
};

// The down projection at 2..8 tokens from a GLU tile's output xq2: at 4 or
// more tokens on the f16 tile split over K (the GLU tile then also writes
// the hx form, down_htile), else the int8 tile split in two, or the
// general matvec.  4096 x 14336 cold: 19.4 against 21.8 us at 4 tokens,
// 21.4 against 32.5 us at 8.
static bool down_htile(const mi_layer_desc* d, int32_t tokens) {
  const int k = d->down.kind;
  return tokens >= 4 && (k == MI_Q4_K || k == MI_Q6_K) && htile_split_fits(k, d->width, d->hidden, tokens) &&
         d->down.row_bytes == (int64_t)(d->hidden / 256) * (k == MI_Q6_K ? 210 : 144) &&
         !((uintptr_t)d->down.data & (k == MI_Q6_K ? 3 : 7));
}

// wo at 4..8 tokens split over K in two (its 4096 columns otherwise fill
// 128 tiles of one launch), the residual add and the ffn norm (with the hx
// form for the GLU tile) in the reduce launch after the parts.
static bool wo_split_norm(const mi_layer_desc* d, int32_t qw, int32_t tokens) {
  const int k = d->wo.kind;
  return tokens >= 4 && (k == MI_Q4_K || k == MI_Q6_K) &&
         htile_split_norm_fits(k, d->width, qw, tokens, 2) &&
         d->wo.row_bytes == (int64_t)(qw / 256) * (k == MI_Q6_K ? 210 : 144) &&
         !((uintptr_t)d->wo.data & (k == MI_Q6_K ? 3 : 7));
}

static int down_batch(hipStream_t s, const mi_layer_desc* d, const void* xq2, int32_t tokens, float* resid,
                      void* part, NextNorm* nn, void* xq) {
  const void* hx2 = (const uint8_t*)xq2 + (size_t)xq_token_bytes(d->hidden) * tokens;
  if (down_htile(d, tokens) && nn->gain && htile_split_norm_fits(d->down.kind, d->width, d->hidden, tokens)) {
    // the residual add and the next layer's norm in one launch after the parts
    nn->done = true;
    return launch_htile_split_norm(s, d->down.kind, d->down.data, d->down.row_bytes, d->width, d->hidden, xq2, hx2, tokens, resid,
                                   nn->gain, d->eps, (float*)part, xq,
                                   (uint8_t*)xq + (size_t)xq_token_bytes(d->width) * tokens);
  }
  if (down_htile(d, tokens))
    return launch_htile_split(s, d->down.kind, d->down.data, d->down.row_bytes, d->width, d->hidden, xq2, hx2,
                              tokens, resid,
                              d->width, MI_EPI_ADD, nullptr, (float*)part);
  if (d->down.kind == MI_Q4_K && q4k_tile_split_fits(d->width, d->hidden, tokens))
    // 128 tiles over a 14336-value K: two blocks per tile and an ordered reduce
    return launch_q4k_tile_split(s, d->down.data, d->down.row_bytes, d->width, d->hidden, xq2, tokens, resid,
                                 d->width, MI_EPI_ADD, nullptr, (float*)part);
  return launch_matvec(s, d->down.kind, d->down.data, d->down.row_bytes, d->width, d->hidden, xq2, tokens, resid,
                       d->width, MI_EPI_ADD, nullptr);
}

static int llama_layer(hipStream_t s, const mi_layer_desc* d, float* resid, uint16_t* k_cache, uint16_t* v_cache,
                       int64_t cache_stride, const int32_t* kv_index, int64_t index_stride, const int32_t* pos,
                       int32_t max_count, int32_t tokens, char* base, const Carve& c, bool pre, NextNorm* nn);

static int decoder_layer(mi_stream stream, const mi_layer_desc* d, float* resid, uint16_t* k_cache,
                         uint16_t* v_cache, int64_t cache_stride, const int32_t* kv_index, int64_t index_stride,
                         const int32_t* pos, int32_t max_count, int32_t tokens, void* work, size_t work_bytes) {
  int rc = check_desc(d);
  if (rc) return rc;
  if (!resid || !k_cache || !v_cache || !pos) return fail(MI_ERR_ARG, "layer: null pointer");
  if (((uintptr_t)k_cache | (uintptr_t)v_cache) & 15 || cache_stride % 8)
    return fail(MI_ERR_ALIGN, "layer: caches must be 16-byte aligned with a stride of a multiple of 8 halves");
  if (tokens < 1 || tokens > kMaxPrefill) return fail(MI_ERR_ARG, "layer: tokens %d outside 1..%d", tokens, kMaxPrefill);
  if (max_count <= 0) return fail(MI_ERR_SHAPE, "layer: max_count must be positive");
  const int64_t kvw = (int64_t)d->kv_heads * d->head_dim;
  const int64_t crow = cache_row(d->cache_form, (int32_t)kvw);  // halves per position
  // A stride of 0 makes the tokens one sequence's chunk at distinct positions
  // (every token reads and writes the same cache or index list).
  if (cache_stride < 0 || index_stride < 0) return fail(MI_ERR_SHAPE, "layer: negative stride");
  if (!kv_index && tokens > 1 && cache_stride != 0 && cache_stride < (int64_t)max_count * crow)
    return fail(MI_ERR_SHAPE, "layer: cache stride %lld holds fewer than %d slots", (long long)cache_stride,
                max_count);
  if (kv_index && tokens > 1 && index_stride != 0 && index_stride < max_count)
    return fail(MI_ERR_SHAPE, "layer: index stride %lld holds fewer than %d positions", (long long)index_stride,
                max_count);
  if (tokens > kMaxTokens) {
    if (!work || ((uintptr_t)work & 255)) return fail(MI_ERR_ALIGN, "layer: workspace must be 256-byte aligned");
    return prefill_layer((hipStream_t)stream, d, resid, k_cache, v_cache, cache_stride, kv_index, index_stride, pos,
                         max_count, tokens, work, work_bytes);
  }
  const Carve c = carve(d, max_count, tokens);
  if (!work || ((uintptr_t)work & 255) || work_bytes < c.total)
    return fail(MI_ERR_WORKSPACE, "layer: workspace of %zu bytes (256-aligned), %zu needed", work_bytes, c.total);

  hipStream_t s = (hipStream_t)stream;
  char* base = (char*)work;
  // 2..8 tokens: the input's norm may already be in the workspace, and the
  // next layer's may be asked for (mi_layer_desc next_norm / prenormed)
  const bool pre = tokens > 1 && d->prenormed;
  NextNorm nn{tokens > 1 ? d->next_norm : nullptr, false};
  rc = extended(d) ? extended_layer(s, d, resid, k_cache, v_cache, cache_stride, kv_index, index_stride, pos,
                                    max_count, tokens, base, c, pre)
                   : llama_layer(s, d, resid, k_cache, v_cache, cache_stride, kv_index, index_stride, pos, max_count,
                                 tokens, base, c, pre, &nn);
  if (rc || !nn.gain || nn.done) return rc;
  return launch_rms_norm(s, resid, nn.gain, d->width, tokens, d->eps, nullptr, base + c.xq,
                         (uint8_t*)(base + c.xq) + (size_t)xq_token_bytes(d->width) * tokens);
}

// The Llama layer at 1..8 tokens on the fused kernels (pre: the attention
// norm's xq and hx forms are in the workspace already, 2..8 tokens).
static int llama_layer(hipStream_t s, const mi_layer_desc* d, float* resid, uint16_t* k_cache, uint16_t* v_cache,
                       int64_t cache_stride, const int32_t* kv_index, int64_t index_stride, const int32_t* pos,
                       int32_t max_count, int32_t tokens, char* base, const Carve& c, bool pre, NextNorm* nn) {
  int rc;
  const int64_t kvw = (int64_t)d->kv_heads * d->head_dim;
  void* xq = base + c.xq;
  float* qkv = (float*)(base + c.qkv);
  float* up = (float*)(base + c.up);
  float* gate = (float*)(base + c.gate);
  void* attn = base + c.attn;
  const int32_t qw = d->heads * d->head_dim;
  const int64_t qkv_stride = qw + 2 * kvw;
  // a batch's attention output also in the hx form, right after its xq form
  void* hx = tokens > 1 ? (uint8_t*)xq + (size_t)xq_token_bytes(qw) * tokens : nullptr;

  // attention_layer (block.mojo:319)
  const bool fused_qkv = tokens == 1 && d->wq.kind == MI_Q4_K && d->wk.kind == MI_Q4_K &&
                         d->wv.kind == MI_Q4_K && q4k_rows_fits(d->width);
  RowSegs sg{};
  if (fused_qkv) {
    sg.w[0] = (const uint8_t*)d->wq.data;
    sg.w[1] = (const uint8_t*)d->wk.data;
    sg.w[2] = (const uint8_t*)d->wv.data;
    sg.rb[0] = d->wq.row_bytes;
    sg.rb[1] = d->wk.row_bytes;
    sg.rb[2] = d->wv.row_bytes;
    sg.end[0] = qw;
    sg.end[1] = qw + (int32_t)kvw;
    sg.end[2] = qw + 2 * (int32_t)kvw;
    sg.nseg = 3;
  }
  const bool q8 = d->cache_form == MI_CACHE_Q8;
  // a q8_0 cache takes the folded-norm kernel's q8 form (32-value blocks)
  const bool q8_fold = q8 && qw % 32 == 0 && kvw % 32 == 0 &&
                       q4k_qkv_norm_fits(d->width, d->head_dim, d->rope_dim, resid, d->attn_norm);
  if (fused_qkv && !d->neox && (!q8 || q8_fold) && q4k_qkv_rope_fits(d->width, d->head_dim, d->rope_dim)) {
    // norm (plus this position's rope table), then q|k|v with the rope and
    // the cache store in its epilogue: no separate rope launch
    float* trig = (float*)(base + c.trig);
    QkvRope rp{};
    rp.qw = qw;
    rp.kvw = (int)kvw;
    rp.head_dim = d->head_dim;
    rp.rope_dim = d->rope_dim;
    rp.trig = (const float2*)trig;
    rp.pos = pos;
    rp.k_cache = (__half*)k_cache;
    rp.v_cache = (__half*)v_cache;
    rp.kv_index = kv_index;
    rp.steps = d->rope_steps;
    rp.factors = d->rope_factors;
    if (q4k_qkv_norm_fits(d->width, d->head_dim, d->rope_dim, resid, d->attn_norm)) {
      // the norm and the rope angles inside the q|k|v launch
      if ((rc = launch_q4k_qkv_norm(s, sg, d->width, resid, d->attn_norm, d->eps, qkv, rp, q8))) return rc;
    } else {
      if ((rc = launch_rms_norm_trig(s, resid, d->attn_norm, d->width, d->eps, xq, pos, d->rope_steps,
                                     d->rope_factors, d->rope_dim / 2, trig)))
        return rc;
      if ((rc = launch_q4k_qkv_rope(s, sg, d->width, xq, qkv, rp))) return rc;
    }
  } else if (tokens == 1 && !kv_index && !d->neox && !q8 && d->wq.kind == MI_Q4_K && d->wk.kind == MI_Q4_K &&
             d->wv.kind == MI_Q6_K && q4k_rows_fits(d->width) &&
             q4k_qkv_rope_fits(d->width, d->head_dim, d->rope_dim)) {
    // a Q4_K_M file's layer at one token (Q6_K v): the norm with this
    // position's rope table, q|k with the rope and k's cache store in the
    // row kernel's epilogue, then v and its store
    float* trig = (float*)(base + c.trig);
    RowSegs qk{};
    qk.w[0] = (const uint8_t*)d->wq.data;
    qk.w[1] = qk.w[2] = (const uint8_t*)d->wk.data;
    qk.rb[0] = d->wq.row_bytes;
    qk.rb[1] = qk.rb[2] = d->wk.row_bytes;
    qk.end[0] = qw;
    qk.end[1] = qk.end[2] = qw + (int32_t)kvw;
    qk.nseg = 2;
    QkvRope rp{};
    rp.qw = qw;
    rp.kvw = (int)kvw;
    rp.head_dim = d->head_dim;
    rp.rope_dim = d->rope_dim;
    rp.trig = (const float2*)trig;
    rp.pos = pos;
    rp.k_cache = (__half*)k_cache;
    rp.v_cache = (__half*)v_cache;
    rp.steps = d->rope_steps;
    rp.factors = d->rope_factors;
    if ((rc = launch_rms_norm_trig(s, resid, d->attn_norm, d->width, d->eps, xq, pos, d->rope_steps,
                                   d->rope_factors, d->rope_dim / 2, trig)))
      return rc;
    if ((rc = launch_q4k_qkv_rope(s, qk, d->width, xq, qkv, rp))) return rc;
    float* vrow = qkv + qw + kvw;
    if ((rc = launch_matvec(s, d->wv.kind, d->wv.data, d->wv.row_bytes, (int32_t)kvw, d->width, xq, 1, vrow,
                            (int32_t)kvw, MI_EPI_NONE, nullptr)))
      return rc;
    if ((rc = launch_store_kv(s, nullptr, vrow, (int32_t)kvw, k_cache, v_cache, pos, 0, 1, qkv_stride, 0)))
      return rc;
  } else {
    // at 2..8 tokens the norm also writes the hx form (the f16 tile's input)
    void* hxn = tokens > 1 ? (uint8_t*)xq + (size_t)xq_token_bytes(d->width) * tokens : nullptr;
    if (!pre && (rc = launch_rms_norm(s, resid, d->attn_norm, d->width, tokens, d->eps, nullptr, xq, hxn)))
      return rc;
    bool roped = false;
    const bool tile_qkv = tokens > 1 && d->wq.kind == MI_Q4_K && d->wk.kind == MI_Q4_K &&
                          d->wv.kind == MI_Q4_K && q4k_tile_fits(d->width, tokens);
    // a Q4_K_M file's layer: Q4_K q and k, Q6_K v
    RowSegs qk{}, vs{};
    bool mixed_qkv = tokens > 1 && !d->neox && !q8 && d->wq.kind == MI_Q4_K && d->wk.kind == MI_Q4_K &&
                     d->wv.kind == MI_Q6_K;
    if (mixed_qkv) {
      qk.w[0] = (const uint8_t*)d->wq.data;
      qk.w[1] = qk.w[2] = (const uint8_t*)d->wk.data;
      qk.rb[0] = d->wq.row_bytes;
      qk.rb[1] = qk.rb[2] = d->wk.row_bytes;
      qk.end[0] = qw;
      qk.end[1] = qk.end[2] = qw + (int32_t)kvw;
      qk.nseg = 2;
      vs = rows::one_matrix(d->wv.data, d->wv.row_bytes, (int32_t)kvw);
      mixed_qkv = htile_qkv_rope_fits(qk, d->width, tokens, d->head_dim, d->rope_dim) &&
                  htile_qkv_rope_fits(vs, d->width, tokens, d->head_dim, d->rope_dim, MI_Q6_K);
    }
    if (fused_qkv) {
      // q, k and v in one launch, straight into the fused row
      if ((rc = launch_q4k_rows_segs(s, sg, d->width, xq, qkv))) return rc;
    } else if (mixed_qkv) {
      // q|k with the rope and k's cache store on the Q4_K f16 tile, then v
      // on the Q6_K one, every row of which the same epilogue stores into
      // the v cache (as rows qw + kvw .. of a q|k|v launch: qw = -kvw)
      QkvRope rp{};
      rp.qw = qw;
      rp.kvw = (int)kvw;
      rp.head_dim = d->head_dim;
      rp.rope_dim = d->rope_dim;
      rp.pos = pos;
      rp.k_cache = (__half*)k_cache;
      rp.v_cache = (__half*)v_cache;
      rp.kv_index = kv_index;
      rp.steps = d->rope_steps;
      rp.factors = d->rope_factors;
      rp.cache_stride = cache_stride;
      rp.index_stride = index_stride;
      if ((rc = launch_htile_qkv_rope(s, qk, d->width, xq, hxn, tokens, qkv, qkv_stride, rp))) return rc;
      QkvRope rv = rp;
      rv.qw = -(int)kvw;
      if ((rc = launch_htile_qkv_rope(s, vs, d->width, xq, hxn, tokens, qkv, qkv_stride, rv, MI_Q6_K))) return rc;
      roped = true;
    } else if (tile_qkv) {
      // the same for a batch, on the matrix-core tile
      RowSegs tg{};
      tg.w[0] = (const uint8_t*)d->wq.data;
      tg.w[1] = (const uint8_t*)d->wk.data;
      tg.w[2] = (const uint8_t*)d->wv.data;
      tg.rb[0] = d->wq.row_bytes;
      tg.rb[1] = d->wk.row_bytes;
      tg.rb[2] = d->wv.row_bytes;
      tg.end[0] = qw;
      tg.end[1] = qw + (int32_t)kvw;
      tg.end[2] = qw + 2 * (int32_t)kvw;
      tg.nseg = 3;
      if (!d->neox && !q8) {
        // the rope and the f16 cache store in the tile's epilogue
        QkvRope rp{};
        rp.qw = qw;
        rp.kvw = (int)kvw;
        rp.head_dim = d->head_dim;
        rp.rope_dim = d->rope_dim;
        rp.pos = pos;
        rp.k_cache = (__half*)k_cache;
        rp.v_cache = (__half*)v_cache;
        rp.kv_index = kv_index;
        rp.steps = d->rope_steps;
        rp.factors = d->rope_factors;
        rp.cache_stride = cache_stride;
        rp.index_stride = index_stride;
        if (htile_qkv_rope_fits(tg, d->width, tokens, d->head_dim, d->rope_dim))
          rc = launch_htile_qkv_rope(s, tg, d->width, xq, hxn, tokens, qkv, qkv_stride, rp);
        else
          rc = launch_q4k_tile_qkv_rope(s, tg, d->width, xq, tokens, qkv, qkv_stride, rp);
        if (rc) return rc;
        roped = true;
      } else {
        // a q8_0 cache or neox pairing: unrotated q|k|v for rope_store, on
        // the f16 tile where its segments fit
        if (htile_qkv_rope_fits(tg, d->width, tokens, d->head_dim, d->rope_dim))
          rc = launch_htile(s, MI_Q4_K, tg, qw + 2 * (int32_t)kvw, d->width, xq, hxn, tokens, qkv, qkv_stride,
                            MI_EPI_NONE, nullptr);
        else
          rc = launch_q4k_tile_segs(s, tg, d->width, xq, tokens, qkv, qkv_stride);
        if (rc) return rc;
      }
    } else {
      if ((rc = launch_matvec(s, d->wq.kind, d->wq.data, d->wq.row_bytes, qw, d->width, xq, tokens, qkv,
                              qkv_stride, MI_EPI_NONE, nullptr)))
        return rc;
      if ((rc = launch_matvec(s, d->wk.kind, d->wk.data, d->wk.row_bytes, (int32_t)kvw, d->width, xq, tokens,
                              qkv + qw, qkv_stride, MI_EPI_NONE, nullptr)))
        return rc;
      if ((rc = launch_matvec(s, d->wv.kind, d->wv.data, d->wv.row_bytes, (int32_t)kvw, d->width, xq, tokens,
                              qkv + qw + kvw, qkv_stride, MI_EPI_NONE, nullptr)))
        return rc;
    }
    // rotate q and k; k and v into the cache (f16, or q8_0 blocks encoded by
    // the same launch once it holds every rotated key)
    if (!roped && (rc = launch_rope_store(s, qkv, d->heads, d->kv_heads, d->head_dim, d->rope_dim, d->neox,
                                d->rope_steps, pos, tokens, qkv_stride, k_cache, v_cache, cache_stride,
                                d->rope_factors, d->cache_form, kv_index, index_stride)))
      return rc;
  }
  // count = pos + 1 per sequence: the attention kernels read pos and add one.
  if ((rc = launch_attend(s, qkv, qkv_stride, k_cache, v_cache, cache_stride, d->heads, d->kv_heads,
                          d->head_dim, d->attn_scale, pos, -1, max_count, tokens, nullptr, xq, attn,
                          d->cache_form, kv_index, index_stride, hx)))
    return rc;
  const bool glu_tile = tokens >= 4 && d->gate.kind == MI_Q4_K && d->up.kind == MI_Q4_K &&
                        d->gate.row_bytes == d->up.row_bytes && htile_glu_fits(d->hidden, d->width, tokens);
  const bool wo_split = glu_tile && wo_split_norm(d, qw, tokens);
  if (!wo_split && (rc = launch_matvec(s, d->wo.kind, d->wo.data, d->wo.row_bytes, d->width, qw, xq, tokens, resid,
                                       d->width, MI_EPI_ADD, nullptr, hx)))
    return rc;

  // mlp_layer (block.mojo:429), gated silu
  if (tokens == 1 && d->gate.kind == MI_Q4_K && d->up.kind == MI_Q4_K && d->gate.row_bytes == d->up.row_bytes &&
      q4k_glu_norm_fits(d->hidden, d->width, resid, d->ffn_norm)) {
    // the norm inside the gate|up launch, which also writes down's input
    void* xq2 = base + c.xq2;
    if ((rc = launch_q4k_glu_norm(s, d->gate.data, d->up.data, d->gate.row_bytes, d->hidden, d->width, resid,
                                  d->ffn_norm, d->eps, gate, xq2)))
      return rc;
    return launch_matvec(s, d->down.kind, d->down.data, d->down.row_bytes, d->width, d->hidden, xq2, tokens,
                         resid, d->width, MI_EPI_ADD, nullptr);
  }
  if (glu_tile) {
    // a batch of 4..8: the norm (with the hx form), then gate and up on the
    // f16 matrix-core tile, which writes act(gate) * up straight into down's
    // xq and hx forms (at 4 tokens 3.084 against 3.115 ms a decode step with
    // the int8 GLU tile below, at 8 tokens 3.86 against 4.50 ms)
    void* hx2 = (uint8_t*)xq + (size_t)xq_token_bytes(d->width) * tokens;
    void* xq2 = base + c.xq2;
    if (wo_split) {
      if ((rc = launch_htile_split_norm(s, d->wo.kind, d->wo.data, d->wo.row_bytes, d->width, qw, xq, hx, tokens,
                                        resid, d->ffn_norm, d->eps, (float*)(base + c.part), xq, hx2, 2)))
        return rc;
    } else if ((rc = launch_rms_norm(s, resid, d->ffn_norm, d->width, tokens, d->eps, nullptr, xq, hx2))) {
      return rc;
    }
    if ((rc = launch_htile_glu(s, d->gate.data, d->up.data, d->gate.row_bytes, d->hidden, d->width, xq, hx2, tokens,
                               MI_EPI_NONE, xq2, down_htile(d, tokens))))
      return rc;
    return down_batch(s, d, xq2, tokens, resid, base + c.part, nn, xq);
  }
  if ((rc = launch_rms_norm(s, resid, d->ffn_norm, d->width, tokens, d->eps, nullptr, xq))) return rc;
  if (tokens == 1 && d->gate.kind == MI_Q4_K && d->up.kind == MI_Q4_K && d->gate.row_bytes == d->up.row_bytes &&
      q4k_rows_fits(d->width)) {
    // gate and up in one launch, silu(gate) * up written directly, and (up
    // to 4096 columns) in matvec form for the down projection
    if (d->width <= 4096) {
      void* xq2 = base + c.xq2;
      if ((rc = launch_q4k_glu(s, d->gate.data, d->up.data, d->gate.row_bytes, d->hidden, d->width, xq, gate,
                               MI_EPI_NONE, xq2)))
        return rc;
      return launch_matvec(s, d->down.kind, d->down.data, d->down.row_bytes, d->width, d->hidden, xq2, tokens,
                           resid, d->width, MI_EPI_ADD, nullptr);
    }
    if ((rc = launch_q4k_glu(s, d->gate.data, d->up.data, d->gate.row_bytes, d->hidden, d->width, xq, gate,
                             MI_EPI_NONE)))
      return rc;
  } else if (tokens > 1 && d->gate.kind == MI_Q4_K && d->up.kind == MI_Q4_K &&
             d->gate.row_bytes == d->up.row_bytes && q4k_tile_fits(d->width, tokens)) {
    // the tile quantizes its own output groups: no separate quantize launch
    void* xq2 = base + c.xq2;
    if ((rc = launch_q4k_tile_glu(s, d->gate.data, d->up.data, d->gate.row_bytes, d->hidden, d->width, xq, tokens,
                                  gate, d->hidden, down_htile(d, tokens) ? kEpiHx : MI_EPI_NONE, xq2)))
      return rc;
    return down_batch(s, d, xq2, tokens, resid, base + c.part, nn, xq);
  } else {
    if ((rc = launch_matvec(s, d->up.kind, d->up.data, d->up.row_bytes, d->hidden, d->width, xq, tokens, up,
                            d->hidden, MI_EPI_NONE, nullptr)))
      return rc;
    if ((rc = launch_matvec(s, d->gate.kind, d->gate.data, d->gate.row_bytes, d->hidden, d->width, xq, tokens,
                            gate, d->hidden, MI_EPI_GLU, up)))
      return rc;
  }
  if ((rc = launch_quantize(s, gate, d->hidden, tokens, xq))) return rc;
  return launch_matvec(s, d->down.kind, d->down.data, d->down.row_bytes, d->width, d->hidden, xq, tokens,
                       resid, d->width, MI_EPI_ADD, nullptr);
}

extern "C" {

size_t mi_layer_workspace(const mi_layer_desc* desc, int32_t max_count, int32_t tokens) {
  if (!desc || max_count <= 0 || tokens <= 0 || tokens > kMaxPrefill) return 0;
  if (tokens > kMaxTokens) return prefill_carve(desc, max_count, tokens).total;
  return carve(desc, max_count, tokens).total;
}

// The layer over per-sequence caches (kv_index null) or a paged pool.

int mi_decoder_layer(mi_stream stream, const mi_layer_desc* d, float* resid, uint16_t* k_cache,
                     uint16_t* v_cache, int64_t cache_stride, const int32_t* pos, int32_t max_count,
                     int32_t tokens, void* work, size_t work_bytes) {
  return decoder_layer(stream, d, resid, k_cache, v_cache, cache_stride, nullptr, 0, pos, max_count, tokens, work,
                       work_bytes);
}

int mi_decoder_layer_paged(mi_stream stream, const mi_layer_desc* d, float* resid, uint16_t* k_pool,
                           uint16_t* v_pool, const int32_t* kv_index, int64_t index_stride, const int32_t* pos,
                           int32_t max_count, int32_t tokens, void* work, size_t work_bytes) {
  if (!kv_index) return fail(MI_ERR_ARG, "layer: a paged layer needs its index");
  return decoder_layer(stream, d, resid, k_pool, v_pool, 0, kv_index, index_stride, pos, max_count, tokens, work,
                       work_bytes);
}

}  // extern "C"
