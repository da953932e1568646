// mi_internal.h -- shared definitions of the gfx950 decode kernels.
//
// Activation format ("xq").  Every matvec multiplies packed GGUF integers by
// activations held as block fixed point: each run of 32 values (a "group",
// the sub-block size every supported quant kind divides into) gets a power of
// two scale 2^e, chosen so the largest |x| maps below 2^22, and each value
// becomes the integer X = rint(x / 2^e), split into three signed bytes
// X = L1*65536 + L2*256 + L3.  A weight dot is then three exact int8 dot
// products (v_dot4c_i32_i8) per four weights, recombined in float once per
// group.  The error against float32 x is at most 2^-23 of the group maximum
// per value, the same order as float32 rounding of x itself.
//
// Layout per token, G = cols/32 groups, eight planes of G 16-byte entries:
//   plane 2*j + hh (j = limb 0..2 most significant first, hh = which 16 of the
//   group's 32 values): the 16 limb bytes of those values, in value order.
//   plane 6: {float scale, float xsum, int lsum1[0], int lsum1[1]}
//   plane 7: {int lsum23[0], int lsum23[1], 0, 0}
// where xsum = scale * sum(X) over the group, lsum1[hh] = sum of L1 over the
// 16 values of half hh, lsum23[hh] = sum of (L2*256 + L3) over the same 16.
// A token's activations take 128*G = 4*cols bytes.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/molla_mi.h"

namespace mi {

constexpr int kWave = 64;
constexpr int kPlanes = 8;
constexpr int kMaxTokens = 8;

__host__ __device__ inline int64_t xq_token_bytes(int32_t cols) { return (int64_t)cols * 4; }

struct XMeta {
  float scale;
  float xsum;
  int lsum1[2];
};

// ---- error state (shim.cpp) ----------------------------------------------
int fail(int code, const char* fmt, ...);
int hip_check(hipError_t e, const char* what);
// Raises fn's dynamic-LDS limit to `bytes` on the current device, once per
// device (the attribute belongs to the device's copy of the kernel); `done`
// is the call site's own kMaxDevices flags.
constexpr int kMaxDevices = 64;
int allow_lds(const void* fn, int bytes, bool* done, const char* what);

// ---- launchers (no validation beyond what the kernel itself assumes; the
// ---- C-ABI layer in shim.cpp checks shapes before calling these) ----------
int launch_dequant(hipStream_t s, int kind, const void* w, int64_t count, float* out);
// hx: when not null, also the hx form of the same tokens (xq_device.h
// hx_group32), which the f16 matrix-core tile reads.
int launch_quantize(hipStream_t s, const float* x, int32_t cols, int32_t tokens, void* xq, void* hx = nullptr);
// Batch-1 Q4_K / Q4_0 / Q8_0 matvec (matvec_rows.hip); launch_matvec routes
// there itself.  _segs: rows of up to three Q4_K matrices of width cols
// numbered end to end (a layer's q, k, v into one fused row).  _glu:
// y = act(gate . x) * (up . x) for the same rows of two Q4_K matrices
// (act = silu, or gelu with MI_ACT_GELU; MI_EPI_ADD adds into y).
struct RowSegs;
bool rows_fits(int kind, int32_t cols);
bool q4k_rows_fits(int32_t cols);
int launch_rows(hipStream_t s, int kind, const void* w, int64_t row_bytes, int32_t rows, int32_t cols,
                const void* xq, float* y, int32_t epi, const float* aux);
int launch_q4k_rows_segs(hipStream_t s, const RowSegs& sg, int32_t cols, const void* xq, float* y);
// The same q|k|v launch for one token with the rope and the cache store in
// its epilogue (QkvRope in matvec_rows.h): q rotated into `q`, k rotated and
// v into the f16 caches at slot pos[0].  Adjacent-pair (Llama) rope only.
struct QkvRope;
bool q4k_qkv_rope_fits(int32_t cols, int32_t head_dim, int32_t rope_dim);
int launch_q4k_qkv_rope(hipStream_t s, const RowSegs& sg, int32_t cols, const void* xq, float* q,
                        const QkvRope& rp);
// xq_out (rows % 32 == 0, cols <= 4096, not overlapping xq): y also written
// in matvec form, each block quantizing the 32-row group it owns.
int launch_q4k_glu(hipStream_t s, const void* gate, const void* up, int64_t row_bytes, int32_t rows,
                   int32_t cols, const void* xq, float* y, int32_t epi, void* xq_out = nullptr);
// q|k|v with the rope epilogue, taking the RMSNorm of x (gain, eps) itself
// and computing its (cos, sin) from rp.steps / rp.factors: no norm launch.
bool q4k_qkv_norm_fits(int32_t cols, int32_t head_dim, int32_t rope_dim, const void* x, const void* gain);
// q8: the caches are q8_0 rows (rp.qw and rp.kvw multiples of 32); k and v
// go to them as whole 32-value blocks.
int launch_q4k_qkv_norm(hipStream_t s, const RowSegs& sg, int32_t cols, const float* x, const float* gain,
                        float eps, float* q, const QkvRope& rp, bool q8 = false);
// The same with the grouped xq_out, taking the RMSNorm of x (gain, eps)
// itself instead of an xq input: the layer's ffn norm needs no launch.
bool q4k_glu_norm_fits(int32_t rows, int32_t cols, const void* x, const void* gain);
int launch_q4k_glu_norm(hipStream_t s, const void* gate, const void* up, int64_t row_bytes, int32_t rows,
                        int32_t cols, const float* x, const float* gain, float eps, float* y, void* xq_out);
// Batch-1 Q6_K matvec for up to 4096 columns (matvec_q6k_rows.hip).
bool q6k_rows_fits(int32_t cols, int64_t row_bytes);
int launch_q6k_rows(hipStream_t s, const void* w, int64_t row_bytes, int32_t rows, int32_t cols, const void* xq,
                    float* y, int32_t epi, const float* aux);
// Batched (2..8 tokens) Q4_K matvec on the matrix cores (matvec_tile.hip).
// The tile with K split over two blocks and an ordered reduce launch
// q|k|v on the tile with the rope and the f16 cache store in its epilogue
// (Llama pairing): q rotated into q (row stride ldq), k and v into the cache.
int launch_q4k_tile_qkv_rope(hipStream_t s, const RowSegs& sg, int32_t cols, const void* xq, int32_t tokens,
                             float* q, int64_t ldq, const QkvRope& rp);
// (part: q4k_tile_split_bytes of scratch), for few tiles over a long K.
bool q4k_tile_split_fits(int32_t rows, int32_t cols, int32_t tokens);
size_t q4k_tile_split_bytes(int32_t rows, int32_t tokens);
int launch_q4k_tile_split(hipStream_t s, const void* w, int64_t row_bytes, int32_t rows, int32_t cols,
                          const void* xq, int32_t tokens, float* y, int64_t ldy, int32_t epi, const float* aux,
                          float* part);
bool q4k_tile_fits(int32_t cols, int32_t tokens);
int launch_q4k_tile(hipStream_t s, const void* w, int64_t row_bytes, int32_t rows, int32_t cols, const void* xq,
                    int32_t tokens, float* y, int64_t ldy, int32_t epi, const float* aux);
// ... with rows of up to three matrices end to end (q|k|v), and the
// gate/up pair with the GLU applied, as the batch-1 row kernel's variants.
int launch_q4k_tile_segs(hipStream_t s, const RowSegs& sg, int32_t cols, const void* xq, int32_t tokens, float* y,
                         int64_t ldy);
// xq_out (rows % 32 == 0, not overlapping xq): y also written in matvec form,
// each tile quantizing its own 32-row groups, for the next projection.
int launch_q4k_tile_glu(hipStream_t s, const void* gate, const void* up, int64_t row_bytes, int32_t rows,
                        int32_t cols, const void* xq, int32_t tokens, float* y, int64_t ldy, int32_t epi,
                        void* xq_out = nullptr);
// Batched (2..8 tokens) Q6_K matvec on the matrix cores (matvec_tile_q6k.hip).
bool q6k_tile_fits(int32_t cols, int64_t row_bytes, int32_t tokens);
int launch_q6k_tile(hipStream_t s, const void* w, int64_t row_bytes, int32_t rows, int32_t cols, const void* xq,
                    int32_t tokens, float* y, int64_t ldy, int32_t epi, const float* aux);
// Batched (2..8 tokens) Q4_0 / Q8_0 matvec on the matrix cores
// (matvec_tile_b32.hip).
bool b32_tile_fits(int kind, int32_t cols, int64_t row_bytes, int32_t tokens);
int launch_b32_tile(hipStream_t s, int kind, const void* w, int64_t row_bytes, int32_t rows, int32_t cols,
                    const void* xq, int32_t tokens, float* y, int64_t ldy, int32_t epi, const float* aux);
// prefill.hip -- tokens above the decode batch (up to kMaxPrefill) on the
// f16 matrix cores, from float activations; prefill_fits says whether the
// kind, width and alignment take the tile (else mi_matvec runs the decode
// kernels eight tokens at a time).  The workspace is prefill_prep_bytes for
// the activation halves, plus room for split-K partial sums up to
// prefill_workspace; with less, K is not split.
constexpr int kMaxPrefill = 65536;
bool prefill_fits(int kind, int32_t cols, int64_t row_bytes, const void* w);
size_t prefill_prep_bytes(int32_t cols, int32_t tokens);
size_t prefill_workspace(int32_t rows, int32_t cols, int32_t tokens);
int launch_prefill(hipStream_t s, int kind, const void* w, int64_t row_bytes, int32_t rows, int32_t cols,
                   const float* x, int32_t tokens, float* y, int64_t ldy, int32_t epi, const float* aux, void* work,
                   size_t work_bytes);
// The two halves of launch_prefill, for several matrices over one input
// (q|k|v, gate and up): prefill_prepare writes the activation halves into
// work, launch_prefill_segs runs rows of up to three matrices of one kind
// (RowSegs, matvec_rows.h) against them.
struct RowSegs;
int prefill_prepare(hipStream_t s, const float* x, int32_t cols, int32_t tokens, void* work);
int launch_prefill_segs(hipStream_t s, int kind, const RowSegs& sg, int32_t cols, int32_t tokens, float* y,
                        int64_t ldy, int32_t epi, const float* aux, void* work, size_t work_bytes);
// shim.cpp: the prefill tile where it fits, else the decode kernels eight
// tokens at a time; y[t * ldy + r]; work as launch_prefill.
int matmul_tokens(hipStream_t s, int kind, const void* w, int64_t row_bytes, int32_t rows, int32_t cols,
                  const float* x, int32_t tokens, float* y, int64_t ldy, int32_t epi, const float* aux, void* work,
                  size_t work_bytes);
// Every kind and batch: routes to the kernels above or the general
// matvec_kernel.h.  matvec_route names the kernel launch_matvec takes for a
// shape (MI_ROUTE_*, the codes mi_matvec_route reports); the split-K forms
// are chosen by mi_matvec itself (shim.cpp).
int matvec_route(int kind, const void* w, int64_t row_bytes, int32_t rows, int32_t cols, int32_t tokens, bool hx);
int launch_matvec(hipStream_t s, int kind, const void* w, int64_t row_bytes, int32_t rows,
                  int32_t cols, const void* xq, int32_t tokens, float* y, int64_t ldy, int32_t epi,
                  const float* aux, const void* hx = nullptr);
// The f16 matrix-core tile for 2..8 tokens (matvec_htile.hip): Q4_K or Q6_K
// rows of up to three matrices whose ends (but the last) are whole 16-row
// tiles, 8-byte aligned, reading the xq form (group scales) and the hx form
// of the same tokens.
// Internal epilogue bit of the GLU tiles: the quantized output xq_out is
// followed, tokens * 4 * rows bytes on, by its hx form (the f16 tile's input).
constexpr int kEpiHx = 1 << 16;
// Compute units of the current device (cached per device).
int cu_count();

bool htile_fits(int kind, int32_t rows, int32_t cols, int32_t tokens);
// Q4_K or Q6_K rows longer than 4096 columns on the f16 tile: K split over column
// parts (part: htile_split_bytes of scratch), then one reduce launch that adds
// the parts in order and applies the epilogue.
bool htile_split_fits(int kind, int32_t rows, int32_t cols, int32_t tokens, int nmin = 1);
// The parts a split f16 tile cuts cols into (0: none fits).
int htile_nsplit(int kind, int32_t cols, int nmin = 1);
// q|k|v (whole 16-row segments) with the rope and the f16 cache store in the
// epilogue, as launch_q4k_tile_qkv_rope.
// kind MI_Q6_K: a Q6_K segment (a Q4_K_M file's attn_v) in its own launch.
bool htile_qkv_rope_fits(const RowSegs& sg, int32_t cols, int32_t tokens, int32_t head_dim, int32_t rope_dim,
                         int kind = MI_Q4_K);
int launch_htile_qkv_rope(hipStream_t s, const RowSegs& sg, int32_t cols, const void* xq, const void* hx,
                          int32_t tokens, float* q, int64_t ldq, const QkvRope& rp, int kind = MI_Q4_K);
size_t htile_split_bytes(int32_t rows, int32_t cols, int32_t tokens, int nmin = 1);
int launch_htile_split(hipStream_t s, int kind, const void* w, int64_t row_bytes, int32_t rows, int32_t cols,
                       const void* xq, const void* hx, int32_t tokens, float* y, int64_t ldy, int32_t epi,
                       const float* aux, float* part);
// The same split with the residual add and the next RMSNorm after it in
// one launch: resid += the parts (added in order, as the reduce above with
// MI_EPI_ADD), then gain's norm of the new rows written in matvec form into
// xq_out and in the hx form into hx_out.  Up to kMaxNormSplit parts and
// 4096 rows.
constexpr int kMaxNormSplit = 4;
bool htile_split_norm_fits(int kind, int32_t rows, int32_t cols, int32_t tokens, int nmin = 1);
int launch_htile_split_norm(hipStream_t s, int kind, const void* w, int64_t row_bytes, int32_t rows, int32_t cols,
                            const void* xq, const void* hx, int32_t tokens, float* resid, const float* gain,
                            float eps, float* part, void* xq_out, void* hx_out, int nmin = 1);
// part[k][t][r] for k < nsplit, and the old residual in slot nsplit:
// resid[t][r] = old + (part 0 + ... + part nsplit-1), then its RMSNorm by
// gain (rms_norm_kernel's arithmetic) into xq and hx.
int launch_split_add_norm(hipStream_t s, const float* part, int nsplit, float* resid, const float* gain, int32_t n,
                          int32_t tokens, float eps, void* xq, void* hx);
int launch_htile(hipStream_t s, int kind, const RowSegs& sg, int32_t rows, int32_t cols, const void* xq,
                 const void* hx, int32_t tokens, float* y, int64_t ldy, int32_t epi, const float* aux);
// The gated MLP's input side on the same tile (Q4_K gate and up of `rows` x
// `cols`, rows a multiple of 32): act(gate) * up written only in matvec form
// into xq_out (`rows` values a token), for the down projection; with hx_out,
// also its hx form, tokens * 4 * rows bytes past xq_out.
bool htile_glu_fits(int32_t rows, int32_t cols, int32_t tokens);
int launch_htile_glu(hipStream_t s, const void* gate, const void* up, int64_t row_bytes, int32_t rows, int32_t cols,
                     const void* xq, const void* hx, int32_t tokens, int32_t act, void* xq_out,
                     bool hx_out = false);
// rms_norm_trig: also writes trig[p] = (cos, sin) of f32(pos[0]) * steps[p]
// (divided by factors[p] when factors is given) for p < pairs (float64 trig,
// as rope.mojo:253-285), for the fused q|k|v epilogue of the same layer.
int launch_rms_norm_trig(hipStream_t s, const float* x, const float* gain, int32_t n, float eps, void* xq,
                         const int32_t* pos, const float* steps, const float* factors, int32_t pairs,
                         float* trig);
int launch_rms_norm(hipStream_t s, const float* x, const float* gain, int32_t n, int32_t tokens,
                    float eps, float* out, void* xq, void* hx = nullptr);
// factors: rope_freqs.weight (one per pair), or null for none.
int launch_rope(hipStream_t s, float* x, int32_t heads, int32_t head_dim, int32_t dim, int32_t neox,
                const float* steps, const int32_t* pos, int32_t tokens, int64_t row_stride,
                const float* factors = nullptr);
// Halves one cached position occupies at a cache form (repack.mojo:221
// cache_row); -1 for an unknown form or a q8_0 width of partial blocks.
__host__ __device__ inline int32_t cache_row(int32_t form, int32_t kv_width) {
  if (kv_width <= 0) return -1;
  if (form == MI_CACHE_F16) return kv_width;
  if (form != MI_CACHE_Q8 || kv_width % 32) return -1;
  return (kv_width / 2 + kv_width / 32 + 7) / 8 * 8;
}
// cache_stride: halves from one sequence's cache to the next; form: MI_CACHE_*.
int launch_store_kv(hipStream_t s, const float* k, const float* v, int32_t kv_width,
                    uint16_t* k_cache, uint16_t* v_cache, const int32_t* slot_dev, int32_t slot_host,
                    int32_t tokens, int64_t src_stride, int64_t cache_stride, int32_t form = MI_CACHE_F16);
// Rotate q and k heads of a fused qkv row and store k (rotated) and v into
// the half caches at slot pos[t]; q is rotated in place.
int launch_rope_store(hipStream_t s, float* qkv, int32_t heads, int32_t kv_heads, int32_t head_dim,
                      int32_t dim, int32_t neox, const float* steps, const int32_t* pos,
                      int32_t tokens, int64_t row_stride, uint16_t* k_cache, uint16_t* v_cache,
                      int64_t cache_stride, const float* factors = nullptr, int32_t form = MI_CACHE_F16,
                      const int32_t* kv_index = nullptr, int64_t index_stride = 0);
size_t attend_workspace(int32_t heads, int32_t head_dim, int32_t max_count, int32_t tokens);
// Attention and the cache stores take an optional paged index: kv_index[t *
// index_stride + j] is the pool cell (one cache row) holding position j of
// sequence t, negative for a position it does not hold; null for
// per-sequence caches cache_stride halves apart.
int launch_attend(hipStream_t s, const float* q, int64_t q_stride, const uint16_t* k_cache,
                  const uint16_t* v_cache, int64_t cache_stride, int32_t heads, int32_t kv_heads,
                  int32_t head_dim, float scale, const int32_t* pos_dev, int32_t count_host,
                  int32_t max_count, int32_t tokens, float* out, void* xq_out, void* work,
                  int32_t form = MI_CACHE_F16, const int32_t* kv_index = nullptr, int64_t index_stride = 0,
                  void* hx_out = nullptr);
int launch_argmax(hipStream_t s, const float* x, int32_t n, int32_t tokens, int32_t* out);
size_t argmax_workspace(int32_t n, int32_t tokens);
int launch_argmax_ws(hipStream_t s, const float* x, int32_t n, int32_t tokens, int32_t* out, void* work,
                     int32_t* next_ids, int32_t* next_pos);
// The optional layer parts (ops.hip): per-head RMS norm of `heads` runs of n
// in each of `tokens` rows row_stride apart, in place; resid[t] +=
// rms_norm(y[t]) * gain; x = act(x) (silu, or gelu with MI_ACT_GELU).
int launch_head_norm(hipStream_t s, float* x, int32_t heads, int32_t n, int32_t tokens, int64_t row_stride,
                     const float* gain, float eps);
int launch_norm_add(hipStream_t s, float* resid, const float* y, int32_t n, int32_t tokens, const float* gain,
                    float eps);
int launch_act(hipStream_t s, float* x, int64_t n, int32_t act);
int launch_embed(hipStream_t s, const float* emb, int32_t vocab, int32_t width, const int32_t* ids,
                 int32_t tokens, float* out);

// ---- small device helpers -----------------------------------------------

__device__ __forceinline__ float half_bits_to_float(uint32_t h16) {
  return __half2float(__ushort_as_half((unsigned short)(h16 & 0xFFFFu)));
}

// ---- lane exchanges without the LDS unit ------------------------------------
// __shfl_xor is a ds_bpermute: an LDS-unit round trip (about a hundred
// cycles), and a reduction chains six of them.  These reductions use DPP
// (quad permutes and the 8- and 16-lane mirrors, which pair every lane with
// one of the other half once the halves are uniform) and gfx950's
// v_permlane16_swap / v_permlane32_swap (rows 0 <-> 1 and 2 <-> 3, or the
// wave's two halves), each a VALU instruction.  Every lane of the wave must
// be active.  Results are uniform over the reduced lanes; a float sum adds
// in a fixed order, so every call with the same inputs gives the same bits.
namespace lanes {
template <int CTRL>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, false);
}
constexpr int kXor1 = 0xB1, kXor2 = 0x4E, kHalfMirror = 0x141, kMirror = 0x140;
// within each 4 lanes, lane i reads lane i + 1 (kDown1) or i + 2 (kDown2);
// the last lanes read themselves (as __shfl_down(v, 1 or 2, 4))
constexpr int kDown1 = 0xF9, kDown2 = 0xEE;
struct Add {
  __device__ __forceinline__ float operator()(float a, float b) const { return a + b; }
  __device__ __forceinline__ int operator()(int a, int b) const { return a + b; }
};
struct Max {
  __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
__device__ __forceinline__ uint32_t bits(float v) { return __float_as_uint(v); }
__device__ __forceinline__ uint32_t bits(int v) { return (uint32_t)v; }
__device__ __forceinline__ float back(uint32_t b, float) { return __uint_as_float(b); }
__device__ __forceinline__ int back(uint32_t b, int) { return (int)b; }
// all-reduce over each group of N = 2, 4, 8, 16, 32 or 64 aligned lanes
template <int N, class T, class Op>
__device__ __forceinline__ T reduce(T v, Op op) {
  if constexpr (N >= 2) v = op(v, back(dpp<kXor1>(bits(v)), v));
  if constexpr (N >= 4) v = op(v, back(dpp<kXor2>(bits(v)), v));
  if constexpr (N >= 8) v = op(v, back(dpp<kHalfMirror>(bits(v)), v));
  if constexpr (N >= 16) v = op(v, back(dpp<kMirror>(bits(v)), v));
  if constexpr (N >= 32) {
    const auto p = __builtin_amdgcn_permlane16_swap(bits(v), bits(v), false, false);
    v = op(back(p[0], v), back(p[1], v));
  }
  if constexpr (N >= 64) {
    const auto p = __builtin_amdgcn_permlane32_swap(bits(v), bits(v), false, false);
    v = op(back(p[0], v), back(p[1], v));
  }
  return v;
}
// all-reduce of a float64 sum over each group of N aligned lanes, the two
// dwords moved together
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
  const uint64_t b = __double_as_longlong(v);
  const uint64_t lo = dpp<CTRL>((uint32_t)b), hi = dpp<CTRL>((uint32_t)(b >> 32));
  return __longlong_as_double((long long)(lo | (hi << 32)));
}
template <int N>
__device__ __forceinline__ double reduce_sum(double v) {
  if constexpr (N >= 2) v += dpp_d<kXor1>(v);
  if constexpr (N >= 4) v += dpp_d<kXor2>(v);
  if constexpr (N >= 8) v += dpp_d<kHalfMirror>(v);
  if constexpr (N >= 16) v += dpp_d<kMirror>(v);
  if constexpr (N >= 32) {
    const uint64_t b = __double_as_longlong(v);
    const auto lo = __builtin_amdgcn_permlane16_swap((uint32_t)b, (uint32_t)b, false, false);
    const auto hi = __builtin_amdgcn_permlane16_swap((uint32_t)(b >> 32), (uint32_t)(b >> 32), false, false);
    v = __longlong_as_double((long long)(lo[0] | ((uint64_t)hi[0] << 32))) +
        __longlong_as_double((long long)(lo[1] | ((uint64_t)hi[1] << 32)));
  }
  if constexpr (N >= 64) {
    const uint64_t b = __double_as_longlong(v);
    const auto lo = __builtin_amdgcn_permlane32_swap((uint32_t)b, (uint32_t)b, false, false);
    const auto hi = __builtin_amdgcn_permlane32_swap((uint32_t)(b >> 32), (uint32_t)(b >> 32), false, false);
    v = __longlong_as_double((long long)(lo[0] | ((uint64_t)hi[0] << 32))) +
        __longlong_as_double((long long)(lo[1] | ((uint64_t)hi[1] << 32)));
  }
  return v;
}
}  // namespace lanes

__device__ __forceinline__ float wave_sum(float v) { return lanes::reduce<64>(v, lanes::Add{}); }

}  // namespace mi
