// matvec.cpp -- routes mi_matvec / mi_matvec_xq to the kernel for its kind
// and batch: the batch-1 row kernel of matvec_rows.hip (Q4_K, Q4_0, Q8_0)
// and matvec_rows_more.hip (Q4_1, Q5_0, Q5_1, Q5_K), the batch-1 Q6_K
// kernel of matvec_q6k_rows.hip, the batched Q4_K / Q6_K f16 matrix-core
// tile of matvec_htile.hip (when the caller's activations carry the hx form)
// or the int8 one of matvec_tile.hip and its Q6_K and Q4_0 / Q8_0 siblings
// (matvec_tile_q6k.hip, matvec_tile_b32.hip), else the general
// kernel of matvec_kernel.h, instantiated per kind in matvec_<kind>.hip.
#include "matvec_rows.h"

namespace mi {

int launch_matvec_q4k(hipStream_t, const void*, int64_t, int32_t, int32_t, const void*, int32_t, float*, int64_t,
                      int32_t, const float*);
int launch_matvec_q6k(hipStream_t, const void*, int64_t, int32_t, int32_t, const void*, int32_t, float*, int64_t,
                      int32_t, const float*);
int launch_matvec_q40(hipStream_t, const void*, int64_t, int32_t, int32_t, const void*, int32_t, float*, int64_t,
                      int32_t, const float*);
int launch_matvec_q80(hipStream_t, const void*, int64_t, int32_t, int32_t, const void*, int32_t, float*, int64_t,
                      int32_t, const float*);
int launch_matvec_q41(hipStream_t, const void*, int64_t, int32_t, int32_t, const void*, int32_t, float*, int64_t,
                      int32_t, const float*);
int launch_matvec_q50(hipStream_t, const void*, int64_t, int32_t, int32_t, const void*, int32_t, float*, int64_t,
                      int32_t, const float*);
int launch_matvec_q51(hipStream_t, const void*, int64_t, int32_t, int32_t, const void*, int32_t, float*, int64_t,
                      int32_t, const float*);
int launch_matvec_q5k(hipStream_t, const void*, int64_t, int32_t, int32_t, const void*, int32_t, float*, int64_t,
                      int32_t, const float*);

int matvec_route(int kind, const void* w, int64_t row_bytes, int32_t rows, int32_t cols, int32_t tokens,
                 bool hx) {
  if (tokens == 1 && rows_fits(kind, cols)) return MI_ROUTE_ROWS;
  if (hx && htile_fits(kind, rows, cols, tokens) && ((uintptr_t)w & 7) == 0) return MI_ROUTE_HTILE;
  if (kind == MI_Q4_K && q4k_tile_fits(cols, tokens)) return MI_ROUTE_Q4K_TILE;
  if (b32_tile_fits(kind, cols, row_bytes, tokens) && ((uintptr_t)w & 15) == 0) return MI_ROUTE_B32_TILE;
  if (kind == MI_Q6_K && q6k_tile_fits(cols, row_bytes, tokens) && ((uintptr_t)w & 1) == 0)
    return MI_ROUTE_Q6K_TILE;
  if (tokens == 1 && kind == MI_Q6_K && q6k_rows_fits(cols, row_bytes) && ((uintptr_t)w & 3) == 0)
    return MI_ROUTE_Q6K_ROWS;
  return MI_ROUTE_GENERAL;
}

int launch_matvec(hipStream_t s, int kind, const void* w, int64_t row_bytes, int32_t rows,
                  int32_t cols, const void* xq, int32_t tokens, float* y, int64_t ldy, int32_t epi,
                  const float* aux, const void* hx) {
  switch (matvec_route(kind, w, row_bytes, rows, cols, tokens, hx != nullptr)) {
    case MI_ROUTE_ROWS: return launch_rows(s, kind, w, row_bytes, rows, cols, xq, y, epi, aux);
    case MI_ROUTE_HTILE:
      return launch_htile(s, kind, rows::one_matrix(w, row_bytes, rows), rows, cols, xq, hx, tokens, y, ldy, epi,
                          aux);
    case MI_ROUTE_Q4K_TILE: return launch_q4k_tile(s, w, row_bytes, rows, cols, xq, tokens, y, ldy, epi, aux);
    case MI_ROUTE_B32_TILE: return launch_b32_tile(s, kind, w, row_bytes, rows, cols, xq, tokens, y, ldy, epi, aux);
    case MI_ROUTE_Q6K_TILE: return launch_q6k_tile(s, w, row_bytes, rows, cols, xq, tokens, y, ldy, epi, aux);
    case MI_ROUTE_Q6K_ROWS: return launch_q6k_rows(s, w, row_bytes, rows, cols, xq, y, epi, aux);
    default: break;
  }
  switch (kind) {
    case MI_Q4_K: return launch_matvec_q4k(s, w, row_bytes, rows, cols, xq, tokens, y, ldy, epi, aux);
    case MI_Q6_K: return launch_matvec_q6k(s, w, row_bytes, rows, cols, xq, tokens, y, ldy, epi, aux);
    case MI_Q4_0: return launch_matvec_q40(s, w, row_bytes, rows, cols, xq, tokens, y, ldy, epi, aux);
    case MI_Q8_0: return launch_matvec_q80(s, w, row_bytes, rows, cols, xq, tokens, y, ldy, epi, aux);
    case MI_Q4_1: return launch_matvec_q41(s, w, row_bytes, rows, cols, xq, tokens, y, ldy, epi, aux);
    case MI_Q5_0: return launch_matvec_q50(s, w, row_bytes, rows, cols, xq, tokens, y, ldy, epi, aux);
    case MI_Q5_1: return launch_matvec_q51(s, w, row_bytes, rows, cols, xq, tokens, y, ldy, epi, aux);
    case MI_Q5_K: return launch_matvec_q5k(s, w, row_bytes, rows, cols, xq, tokens, y, ldy, epi, aux);
  }
  return fail(MI_ERR_KIND, "matvec: ggml type %d has no device kernel", kind);
}

}  // namespace mi
