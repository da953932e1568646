// shim.cpp -- the C ABI (include/molla_mi.h): argument checks, refusals and
// error strings, then the launchers.  Every refusal happens before anything
// is queued, mirroring the reference's check_matvec / check_matvec_shapes
// (src/molla/nn/gpu.mojo:2056-2111).
#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>

#include "mi_internal.h"

namespace mi {

static thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int hip_check(hipError_t e, const char* what) {
  if (e == hipSuccess) return MI_OK;
  return fail(MI_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

int allow_lds(const void* fn, int bytes, bool* done, const char* what) {
  int dev = 0;
  int rc = hip_check(hipGetDevice(&dev), what);
  if (rc) return rc;
  if (dev < 0 || dev >= kMaxDevices) return fail(MI_ERR_DEVICE, "%s: device %d beyond %d", what, dev, kMaxDevices);
  if (done[dev]) return MI_OK;
  rc = hip_check(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes), what);
  if (!rc) done[dev] = true;
  return rc;
}

static bool quant_kind(int kind) {
  return kind == MI_Q4_0 || kind == MI_Q4_1 || kind == MI_Q5_0 || kind == MI_Q5_1 || kind == MI_Q8_0 ||
         kind == MI_Q4_K || kind == MI_Q5_K || kind == MI_Q6_K;
}
static bool k_quant(int kind) { return kind == MI_Q4_K || kind == MI_Q5_K || kind == MI_Q6_K; }

// The row geometry the kernels assume, checked once here.
int check_weight(const char* name, int kind, const void* w, int64_t row_bytes, int32_t rows,
                 int32_t cols) {
  if (!quant_kind(kind)) return fail(MI_ERR_KIND, "%s: ggml type %d has no device matvec", name, kind);
  if (!w) return fail(MI_ERR_ARG, "%s: null weight pointer", name);
  if (rows <= 0 || cols <= 0) return fail(MI_ERR_SHAPE, "%s: %d x %d is not a matrix", name, rows, cols);
  // 64-value units; K quants also whole 256-value superblocks
  const int unit = k_quant(kind) ? 256 : 64;
  if (cols % unit != 0)
    return fail(MI_ERR_SHAPE, "%s: %d columns is not a whole number of %d-value units for type %d", name,
                cols, unit, kind);
  const int64_t want = (int64_t)cols / mi_block_elements(kind) * mi_block_bytes(kind);
  if (row_bytes != want)
    return fail(MI_ERR_SHAPE, "%s: row_bytes %lld, but %d columns of type %d take %lld", name,
                (long long)row_bytes, cols, kind, (long long)want);
  const uintptr_t a = (uintptr_t)w;
  if (kind == MI_Q4_K ? (a & 15) != 0 : (a & 3) != 0)
    return fail(MI_ERR_ALIGN, "%s: weight pointer %p is not %d-byte aligned", name, w,
                kind == MI_Q4_K ? 16 : 4);
  return MI_OK;
}

// Tokens above the decode batch: the prefill tile where it fits, else the
// decode kernels over runs of eight tokens (the GLU aux and the output move
// with the run; a bias does not).  The caller has checked the weight, epi and
// aux; work holds prefill_prep_bytes(cols, tokens) at least.
int matmul_tokens(hipStream_t s, int kind, const void* w, int64_t row_bytes, int32_t rows, int32_t cols,
                  const float* x, int32_t tokens, float* y, int64_t ldy, int32_t epi, const float* aux, void* work,
                  size_t work_bytes) {
  if (prefill_fits(kind, cols, row_bytes, w))
    return launch_prefill(s, kind, w, row_bytes, rows, cols, x, tokens, y, ldy, epi, aux, work, work_bytes);
  for (int32_t t0 = 0; t0 < tokens; t0 += kMaxTokens) {
    const int32_t n = tokens - t0 < kMaxTokens ? tokens - t0 : kMaxTokens;
    int rc = launch_quantize(s, x + (int64_t)t0 * cols, cols, n, work);
    if (!rc) {
      const float* a = (epi & MI_EPI_GLU) ? aux + (int64_t)t0 * ldy : aux;
      rc = launch_matvec(s, kind, w, row_bytes, rows, cols, work, n, y + (int64_t)t0 * ldy, ldy, epi, a);
    }
    if (rc) return rc;
  }
  return MI_OK;
}

}  // namespace mi

using namespace mi;

extern "C" {

int mi_version(void) { return (0 << 16) | 1; }

const char* mi_last_error(void) { return g_err; }

int mi_sync(mi_stream stream) { return hip_check(hipStreamSynchronize((hipStream_t)stream), "sync"); }

int mi_block_elements(int kind) {
  switch (kind) {
    case MI_F32: case MI_F16: return 1;
    case MI_Q4_0: case MI_Q4_1: case MI_Q5_0: case MI_Q5_1: case MI_Q8_0: return 32;
    case MI_Q4_K: case MI_Q5_K: case MI_Q6_K: return 256;
  }
  return 0;
}

int mi_block_bytes(int kind) {
  switch (kind) {
    case MI_F32: return 4;
    case MI_F16: return 2;
    case MI_Q4_0: return 18;
    case MI_Q4_1: return 20;
    case MI_Q5_0: return 22;
    case MI_Q5_1: return 24;
    case MI_Q8_0: return 34;
    case MI_Q4_K: return 144;
    case MI_Q5_K: return 176;
    case MI_Q6_K: return 210;
  }
  return 0;
}

int64_t mi_row_bytes(int kind, int32_t cols) {
  const int per = mi_block_elements(kind);
  if (per == 0 || cols <= 0 || cols % per != 0) return -1;
  return (int64_t)(cols / per) * mi_block_bytes(kind);
}

int mi_dequant(mi_stream stream, int kind, const void* w, int64_t count, float* out) {
  if (!quant_kind(kind)) return fail(MI_ERR_KIND, "dequant: ggml type %d has no device decoder", kind);
  if (!w || !out) return fail(MI_ERR_ARG, "dequant: null pointer");
  const int per = mi_block_elements(kind);
  if (count < 0 || count % per != 0)
    return fail(MI_ERR_SHAPE, "dequant: %lld values is not a whole number of %d-value blocks",
                (long long)count, per);
  if (((uintptr_t)out & 15) != 0) return fail(MI_ERR_ALIGN, "dequant: output must be 16-byte aligned");
  return launch_dequant((hipStream_t)stream, kind, w, count, out);
}

size_t mi_matvec_workspace(int32_t cols, int32_t tokens) {
  if (cols <= 0 || tokens <= 0 || tokens > kMaxPrefill) return 0;
  if (tokens > kMaxTokens) return prefill_prep_bytes(cols, tokens);
  // 2..8 tokens: the xq form, then the hx form the f16 matrix-core tile reads
  return (size_t)xq_token_bytes(cols) * (size_t)tokens * (tokens > 1 ? 2 : 1);
}

// The hx form inside an activation workspace of 2..8 tokens, or null.
static void* hx_of(const void* xq, int32_t cols, int32_t tokens) {
  return tokens > 1 ? (uint8_t*)xq + xq_token_bytes(cols) * tokens : nullptr;
}

// 2..8 tokens: the activation forms, then (256-aligned) room for the parts
// of a Q4_K or Q6_K matvec split over K (launch_htile_split,
// launch_q4k_tile_split).
static size_t batch_act_bytes(int32_t cols, int32_t tokens) {
  return (mi_matvec_workspace(cols, tokens) + 255) & ~(size_t)255;
}
static size_t batch_split_bytes(int kind, int32_t rows, int32_t cols, int32_t tokens) {
  size_t b = 0;
  if ((kind == MI_Q4_K || kind == MI_Q6_K) && htile_split_fits(kind, rows, cols, tokens))
    b = htile_split_bytes(rows, cols, tokens);
  if (kind == MI_Q4_K && q4k_tile_split_fits(rows, cols, tokens)) b = std::max(b, q4k_tile_split_bytes(rows, tokens));
  return b;
}

size_t mi_matmul_workspace(int32_t rows, int32_t cols, int32_t tokens) {
  if (rows <= 0 || cols <= 0 || tokens <= 0 || tokens > kMaxPrefill) return 0;
  if (tokens > kMaxTokens) return prefill_workspace(rows, cols, tokens);
  const size_t split = tokens > 1 ? std::max(batch_split_bytes(MI_Q4_K, rows, cols, tokens),
                                             batch_split_bytes(MI_Q6_K, rows, cols, tokens))
                                  : 0;
  return split ? batch_act_bytes(cols, tokens) + split : mi_matvec_workspace(cols, tokens);
}

static int check_xq(const char* name, const void* xq, int32_t cols, int32_t tokens) {
  if (!xq) return fail(MI_ERR_WORKSPACE, "%s: null activation workspace", name);
  if (((uintptr_t)xq & 255) != 0) return fail(MI_ERR_ALIGN, "%s: workspace must be 256-byte aligned", name);
  if (cols <= 0 || cols % 32 != 0) return fail(MI_ERR_SHAPE, "%s: %d values is not a whole number of 32", name, cols);
  if (tokens < 1 || tokens > kMaxTokens) return fail(MI_ERR_ARG, "%s: tokens %d outside 1..8", name, tokens);
  return MI_OK;
}

int mi_quantize(mi_stream stream, const float* x, int32_t cols, int32_t tokens, void* xq) {
  if (!x) return fail(MI_ERR_ARG, "quantize: null input");
  int rc = check_xq("quantize", xq, cols, tokens);
  if (rc) return rc;
  return launch_quantize((hipStream_t)stream, x, cols, tokens, xq, hx_of(xq, cols, tokens));
}

static int check_epi(int32_t epi, const float* aux) {
  if (epi & ~(MI_EPI_BIAS | MI_EPI_ADD | MI_EPI_GLU | MI_ACT_GELU))
    return fail(MI_ERR_ARG, "matvec: unknown epilogue bits 0x%x", epi);
  if ((epi & MI_EPI_BIAS) && (epi & MI_EPI_GLU)) return fail(MI_ERR_ARG, "matvec: BIAS and GLU together");
  if ((epi & (MI_EPI_BIAS | MI_EPI_GLU)) && !aux) return fail(MI_ERR_ARG, "matvec: epilogue needs aux");
  return MI_OK;
}

int mi_matvec_xq(mi_stream stream, int kind, const void* w, int64_t row_bytes, int32_t rows,
                 int32_t cols, const void* xq, int32_t tokens, float* y, int32_t epi, const float* aux) {
  int rc = check_weight("matvec", kind, w, row_bytes, rows, cols);
  if (rc) return rc;
  if ((rc = check_xq("matvec", xq, cols, tokens))) return rc;
  if (!y) return fail(MI_ERR_ARG, "matvec: null output");
  if ((rc = check_epi(epi, aux))) return rc;
  return launch_matvec((hipStream_t)stream, kind, w, row_bytes, rows, cols, xq, tokens, y, rows, epi, aux,
                       hx_of(xq, cols, tokens));
}

static int matmul_many(mi_stream stream, int kind, const void* w, int64_t row_bytes, int32_t rows, int32_t cols,
                       const float* x, int32_t tokens, float* y, int32_t epi, const float* aux, void* work,
                       size_t work_bytes) {
  if (!work || ((uintptr_t)work & 255)) return fail(MI_ERR_ALIGN, "matvec: workspace must be 256-byte aligned");
  if (cols % 32) return fail(MI_ERR_SHAPE, "matvec: %d values is not a whole number of 32", cols);
  if (work_bytes < mi_matvec_workspace(cols, tokens))
    return fail(MI_ERR_WORKSPACE, "matvec: workspace of %zu bytes, %zu needed", work_bytes,
                mi_matvec_workspace(cols, tokens));
  return matmul_tokens((hipStream_t)stream, kind, w, row_bytes, rows, cols, x, tokens, y, rows, epi, aux, work,
                       work_bytes);
}

int mi_matvec(mi_stream stream, int kind, const void* w, int64_t row_bytes, int32_t rows, int32_t cols,
              const float* x, int32_t tokens, float* y, int32_t epi, const float* aux, void* work,
              size_t work_bytes) {
  int rc = check_weight("matvec", kind, w, row_bytes, rows, cols);
  if (rc) return rc;
  if (!x) return fail(MI_ERR_ARG, "matvec: null input");
  if (tokens > kMaxTokens) {
    if (tokens > kMaxPrefill) return fail(MI_ERR_ARG, "matvec: tokens %d above %d", tokens, kMaxPrefill);
    if (!y) return fail(MI_ERR_ARG, "matvec: null output");
    if (epi & ~(MI_EPI_BIAS | MI_EPI_ADD | MI_EPI_GLU | MI_ACT_GELU))
      return fail(MI_ERR_ARG, "matvec: unknown epilogue bits 0x%x", epi);
    if ((epi & MI_EPI_BIAS) && (epi & MI_EPI_GLU)) return fail(MI_ERR_ARG, "matvec: BIAS and GLU together");
    if ((epi & (MI_EPI_BIAS | MI_EPI_GLU)) && !aux) return fail(MI_ERR_ARG, "matvec: epilogue needs aux");
    return matmul_many(stream, kind, w, row_bytes, rows, cols, x, tokens, y, epi, aux, work, work_bytes);
  }
  if ((rc = check_xq("matvec", work, cols, tokens))) return rc;
  if (work_bytes < mi_matvec_workspace(cols, tokens))
    return fail(MI_ERR_WORKSPACE, "matvec: workspace of %zu bytes, %zu needed", work_bytes,
                mi_matvec_workspace(cols, tokens));
  // 2..8 tokens of a Q4_K or Q6_K matrix with too few 16-row tiles for its
  // long K, given room for the parts (mi_matmul_workspace): split over K, on
  // the f16 tile where it fits, else (Q4_K) the int8 tile
  const size_t act = batch_act_bytes(cols, tokens);
  const size_t sb = tokens > 1 ? batch_split_bytes(kind, rows, cols, tokens) : 0;
  const bool split = sb && work_bytes >= act + sb;
  if (!split) {
    if ((rc = mi_quantize(stream, x, cols, tokens, work))) return rc;
    return mi_matvec_xq(stream, kind, w, row_bytes, rows, cols, work, tokens, y, epi, aux);
  }
  if (!y) return fail(MI_ERR_ARG, "matvec: null output");
  if ((rc = check_epi(epi, aux))) return rc;
  if ((rc = mi_quantize(stream, x, cols, tokens, work))) return rc;
  hipStream_t s = (hipStream_t)stream;
  float* part = (float*)((char*)work + act);
  const int sbb = kind == MI_Q6_K ? 210 : 144;
  if (htile_split_fits(kind, rows, cols, tokens) && row_bytes == (int64_t)(cols / 256) * sbb &&
      !((uintptr_t)w & (kind == MI_Q6_K ? 3 : 7)))
    return launch_htile_split(s, kind, w, row_bytes, rows, cols, work, hx_of(work, cols, tokens), tokens, y, rows,
                              epi, aux, part);
  if (kind == MI_Q4_K && q4k_tile_split_fits(rows, cols, tokens))
    return launch_q4k_tile_split(s, w, row_bytes, rows, cols, work, tokens, y, rows, epi, aux, part);
  return launch_matvec(s, kind, w, row_bytes, rows, cols, work, tokens, y, rows, epi, aux, hx_of(work, cols, tokens));
}

int mi_matvec_route(int kind, int32_t rows, int32_t cols, int32_t tokens, size_t work_bytes, int32_t* part_cols) {
  if (mi_block_elements(kind) <= 0) return fail(MI_ERR_KIND, "route: ggml type %d has no device kernel", kind);
  if (rows <= 0 || cols <= 0 || cols % mi_block_elements(kind) || tokens <= 0 || tokens > kMaxPrefill)
    return fail(MI_ERR_SHAPE, "route: bad shape");
  if (part_cols) *part_cols = cols;
  if (tokens > kMaxTokens) return MI_ROUTE_PREFILL;
  const int64_t rb = mi_row_bytes(kind, cols);
  const void* w = (const void*)(uintptr_t)256;  // an aligned address, never dereferenced
  const size_t act = batch_act_bytes(cols, tokens);
  const size_t sb = tokens > 1 ? batch_split_bytes(kind, rows, cols, tokens) : 0;
  if (sb && work_bytes >= act + sb) {
    const int sbb = kind == MI_Q6_K ? 210 : 144;
    if (htile_split_fits(kind, rows, cols, tokens) && rb == (int64_t)(cols / 256) * sbb) {
      if (part_cols) *part_cols = cols / htile_nsplit(kind, cols);
      return MI_ROUTE_HTILE | MI_ROUTE_SPLIT_BIT;
    }
    if (kind == MI_Q4_K && q4k_tile_split_fits(rows, cols, tokens)) return MI_ROUTE_Q4K_TILE | MI_ROUTE_SPLIT_BIT;
  }
  return matvec_route(kind, w, rb, rows, cols, tokens, tokens > 1);
}

int mi_rms_norm(mi_stream stream, const float* x, const float* gain, int32_t n, int32_t tokens, float eps,
                float* out, void* xq) {
  if (!x || !gain || (!out && !xq)) return fail(MI_ERR_ARG, "rms_norm: null pointer");
  if (n <= 0 || tokens <= 0) return fail(MI_ERR_SHAPE, "rms_norm: bad shape %d x %d", tokens, n);
  if (!(eps > 0.0f)) return fail(MI_ERR_ARG, "rms_norm: epsilon must be positive");
  if (xq) {
    int rc = check_xq("rms_norm", xq, n, tokens);
    if (rc) return rc;
  }
  return launch_rms_norm((hipStream_t)stream, x, gain, n, tokens, eps, out, xq, xq ? hx_of(xq, n, tokens) : nullptr);
}

// rope.mojo:230 step_table: f32(exp(f64(y) * log(f64(base)))), y = f32(-2p) / f32(dim).
void mi_rope_steps(float* steps_host, int32_t dim, float base) {
  for (int32_t pair = 0; pair < dim / 2; pair++) {
    const float y = -2.0f * (float)pair / (float)dim;
    steps_host[pair] = base <= 0.0f ? 0.0f : (float)exp((double)y * log((double)base));
  }
}

int mi_rope(mi_stream stream, float* x, int32_t heads, int32_t head_dim, int32_t dim, int32_t neox,
            const float* steps, const int32_t* pos, int32_t tokens, int64_t row_stride) {
  if (!x || !steps || !pos) return fail(MI_ERR_ARG, "rope: null pointer");
  if (heads <= 0 || tokens <= 0 || dim <= 0 || dim % 2 || dim > head_dim)
    return fail(MI_ERR_SHAPE, "rope: rotary dimension %d in heads of %d", dim, head_dim);
  if (row_stride < (int64_t)heads * head_dim) return fail(MI_ERR_SHAPE, "rope: row stride too small");
  return launch_rope((hipStream_t)stream, x, heads, head_dim, dim, neox, steps, pos, tokens, row_stride);
}

int mi_store_kv(mi_stream stream, const float* k, const float* v, int32_t kv_width, uint16_t* k_cache,
                uint16_t* v_cache, int32_t slot) {
  if (!k || !v || !k_cache || !v_cache) return fail(MI_ERR_ARG, "store_kv: null pointer");
  if (kv_width <= 0 || slot < 0) return fail(MI_ERR_SHAPE, "store_kv: bad width or slot");
  return launch_store_kv((hipStream_t)stream, k, v, kv_width, k_cache, v_cache, nullptr, slot, 1, kv_width, 0);
}

int32_t mi_cache_row(int32_t form, int32_t kv_width) { return cache_row(form, kv_width); }

int mi_store_kv_form(mi_stream stream, int32_t form, const float* k, const float* v, int32_t kv_width,
                     uint16_t* k_cache, uint16_t* v_cache, int32_t slot) {
  if (!k || !v || !k_cache || !v_cache) return fail(MI_ERR_ARG, "store_kv: null pointer");
  if (slot < 0 || cache_row(form, kv_width) < 0)
    return fail(MI_ERR_SHAPE, "store_kv: cache form %d has no row of width %d (or slot %d)", form, kv_width, slot);
  if (form == MI_CACHE_Q8 && (((uintptr_t)k_cache | (uintptr_t)v_cache) & 15))
    return fail(MI_ERR_ALIGN, "store_kv: a q8_0 cache must be 16-byte aligned");
  return launch_store_kv((hipStream_t)stream, k, v, kv_width, k_cache, v_cache, nullptr, slot, 1, kv_width, 0,
                         form);
}

size_t mi_attend_workspace(int32_t heads, int32_t head_dim, int32_t count) {
  if (heads <= 0 || head_dim <= 0 || count <= 0) return 0;
  return attend_workspace(heads, head_dim, count, 1);
}

static int check_attn(const char* name, int32_t heads, int32_t kv_heads, int32_t head_dim) {
  if (heads <= 0 || kv_heads <= 0 || heads % kv_heads)
    return fail(MI_ERR_SHAPE, "%s: %d query heads over %d key heads", name, heads, kv_heads);
  const int group = heads / kv_heads;
  if (group != 1 && group != 2 && group != 4 && group != 8)
    return fail(MI_ERR_SHAPE, "%s: %d query heads per key head is not 1, 2, 4 or 8", name, group);
  if (head_dim <= 0 || head_dim % 32 || head_dim > 512)
    return fail(MI_ERR_SHAPE, "%s: head_dim %d is not a multiple of 32 up to 512", name, head_dim);
  return MI_OK;
}

int mi_attend(mi_stream stream, const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
              int32_t heads, int32_t kv_heads, int32_t head_dim, float scale, int32_t count, float* out,
              void* work, size_t work_bytes) {
  return mi_attend_form(stream, MI_CACHE_F16, q, k_cache, v_cache, heads, kv_heads, head_dim, scale, count, out,
                        work, work_bytes);
}

int mi_attend_form(mi_stream stream, int32_t form, const float* q, const uint16_t* k_cache,
                   const uint16_t* v_cache, int32_t heads, int32_t kv_heads, int32_t head_dim, float scale,
                   int32_t count, float* out, void* work, size_t work_bytes) {
  if (!q || !k_cache || !v_cache || !out) return fail(MI_ERR_ARG, "attend: null pointer");
  if (cache_row(form, kv_heads * head_dim) < 0) return fail(MI_ERR_SHAPE, "attend: unknown cache form %d", form);
  int rc = check_attn("attend", heads, kv_heads, head_dim);
  if (rc) return rc;
  if (count <= 0) return fail(MI_ERR_SHAPE, "attention needs at least one key to look at");
  if (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) & 15)
    return fail(MI_ERR_ALIGN, "attend: the query and the caches must be 16-byte aligned");
  if (!work || work_bytes < mi_attend_workspace(heads, head_dim, count))
    return fail(MI_ERR_WORKSPACE, "attend: workspace of %zu bytes, %zu needed", work_bytes,
                mi_attend_workspace(heads, head_dim, count));
  return launch_attend((hipStream_t)stream, q, (int64_t)heads * head_dim, k_cache, v_cache, 0, heads,
                       kv_heads, head_dim, scale, nullptr, count, count, 1, out, nullptr, work, form);
}

int mi_argmax(mi_stream stream, const float* x, int32_t n, int32_t tokens, int32_t* out) {
  if (!x || !out) return fail(MI_ERR_ARG, "argmax: null pointer");
  if (n <= 0 || tokens <= 0) return fail(MI_ERR_SHAPE, "argmax: empty row");
  return launch_argmax((hipStream_t)stream, x, n, tokens, out);
}

size_t mi_argmax_workspace(int32_t n, int32_t tokens) {
  if (n <= 0 || tokens <= 0) return 0;
  return argmax_workspace(n, tokens);
}

int mi_argmax_ws(mi_stream stream, const float* x, int32_t n, int32_t tokens, int32_t* out, void* work,
                 size_t work_bytes, int32_t* next_ids, int32_t* next_pos) {
  if (!x || !out) return fail(MI_ERR_ARG, "argmax: null pointer");
  if (n <= 0 || tokens <= 0) return fail(MI_ERR_SHAPE, "argmax: empty row");
  if (!work || work_bytes < argmax_workspace(n, tokens))
    return fail(MI_ERR_WORKSPACE, "argmax: workspace of %zu bytes, %zu needed", work_bytes,
                argmax_workspace(n, tokens));
  if ((uintptr_t)work & 7) return fail(MI_ERR_ALIGN, "argmax: the workspace must be 8-byte aligned");
  return launch_argmax_ws((hipStream_t)stream, x, n, tokens, out, work, next_ids, next_pos);
}

int mi_embed(mi_stream stream, const float* embedding, int32_t vocab, int32_t width, const int32_t* ids,
             int32_t tokens, float* out) {
  if (!embedding || !ids || !out) return fail(MI_ERR_ARG, "embed: null pointer");
  if (vocab <= 0 || width <= 0 || width % 4 || tokens <= 0)
    return fail(MI_ERR_SHAPE, "embed: bad shape vocab %d width %d", vocab, width);
  return launch_embed((hipStream_t)stream, embedding, vocab, width, ids, tokens, out);
}

}  // extern "C"
