/*
 * mh3_oracle.h — TEST INFRASTRUCTURE ONLY. A scalar CPU restatement of the H3 per-block hot-path ops, used by
 * tests/, the smoke check and bench.py's CPU-baseline leg to test the GPU results. Nothing in the product links,
 * loads or calls it.
 *
 * The reference's implementation of these ops lives in the un-vendored mako-common submodule (.gitmodules:1-3, empty
 * at external/mako-common), so this file restates the semantics the reference's documents and call sites fix, in the
 * reference's CPU idiom (src/video/audio_vae.cpp:386-416: per-row double accumulation, a float store):
 *   rms_mod_rows / gate_add_rows   docs/architecture.md:49-52,61,64-66
 *   swiglu_rows                     docs/architecture.md:65,112-114
 *   cube_pool / _scores / _topk     docs/architecture.md:118-133, README.md:81-87, docs/performance.md:175-181
 *   heads_partial                   docs/architecture.md:35-38,61-63,123-125
 *   quant_rows_i8, W8A16 fc1        docs/performance.md:120-136
 *   qkv / out / fc2 GEMMs           docs/performance.md:40-43,52-69,120-133, docs/architecture.md:61-66
 *   cube map (H3::Cubes)            docs/architecture.md:120-125
 *   time_embed / adaln_mod          docs/architecture.md:49-58, tools/check_pruned_curve.py:57-67
 *   curve_mods                      docs/architecture.md:53-58, tools/check_pruned_curve.py:69-73
 * bf16 results are rounded to nearest even exactly once, from the double value.
 *
 * How each function is pinned (tests/test_oracle.py): no reference vector exists for any of them (the reference
 * holds no fixture at the kernel level), so each is checked against a library routine or brute force written
 * independently of it, plus closed forms and invariants:
 *   mh3o_bf16_from_double      nearest-even property checked exhaustively on neighbours; torch's float->bf16
 *   mh3o_rms_mod_rows          torch.nn.functional.rms_norm (float64); RMS = 1 at w=1, shift=scale=0
 *   mh3o_gate_add_rows         closed form in numpy float64; gate = 0 leaves x bit-exact
 *   mh3o_rms_mod_gate_add_rows composition of the two above; gate = 0 gives residual bit-exact
 *   mh3o_swiglu_rows           torch.nn.functional.silu (float64); silu(0)=0, large |g| limits; split == fused
 *   mh3o_cube_pool             numpy reshape-mean over the (t, y, x) grid; brute force on padded grids;
 *                              permutation invariance inside a cube; gathered layout == grid layout
 *   mh3o_cube_scores           numpy matmul / sqrt(hd)
 *   mh3o_cube_topk             numpy lexsort; constructed scores with an analytic answer; ratio 1 selects all
 *   mh3o_cube_topk_sorted      equals mh3o_cube_topk on random and tie-heavy rows (the form bench.py's CPU
 *                              baseline times: a sort a row instead of the O(C^2) count)
 *   mh3o_attn_sparse(_tile)    torch scaled_dot_product_attention in float64 with a boolean mask built in numpy
 *                              from the pass lists; with every cube selected, the unmasked attention over all rows
 *   mh3o_heads_partial         torch float64: F.rms_norm per head, then the rotation as a complex product of the
 *                              (i, i + rot/2) pairs with e^(i angle) (torch.polar); rotation keeps each pair's
 *                              length; angle 0 is the plain norm, pi/2 maps (a, b) to (-b, a); map -1 gives zeros
 *   mh3o_quant_rows_i8         |q| <= 127, the row maximum maps to +-127, |w - q*s| <= s/2, numpy rint
 *   mh3o_gemm_w8a16_swiglu     torch.matmul in float64; exact integer results for w in {-1,0,1}, s = 1
 *   mh3o_gemm_bf16_swiglu      torch.matmul in float64; exact integer results for w in {-1,0,1}
 *   mh3o_gemm_i8_swiglu        torch.matmul of the int64 operands; exact integer results with unit scales
 *   mh3o_gemm                  torch.matmul in float64 for each form; the gate-add epilogue against gate_add_rows of
 *                              the rounded product (within one bf16 rounding); gate 0 leaves the residual bit-exact;
 *                              exact integer results for w in {-1,0,1}
 *   mh3o_cube_map              brute force in Python over padded grids (a gather per attention row, where the oracle
 *                              scatters per token); its map feeds mh3o_heads_partial to the same means as the grid
 *                              layout of mh3o_cube_pool; counts equal the per-axis product
 *   mh3o_time_embed            torch float64 restatement of tools/check_pruned_curve.py:57-67 (temb()): the
 *                              reference's own statement of the embedding and the MLP; t = 0 gives cos = 1, sin = 0
 *   mh3o_adaln_mod             torch.matmul in float64; exact integer results for small-integer inputs
 *   mh3o_curve_mods            numpy interp per coordinate, then matmul; t at a table point gives that row exactly
 *   (the order in which gemm_i8's epilogue applies the two scales is not documented: parity unpinned for it)
 */
#ifndef MH3_ORACLE_H
#define MH3_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { MH3O_F32 = 0, MH3O_BF16 = 1 };
enum { MH3O_SWIGLU_SPLIT = 0, MH3O_SWIGLU_FUSED = 1 };
enum { MH3O_CUBES_GRID = 0, MH3O_CUBES_GATHERED = 1 };

float mh3o_bf16_to_float(uint16_t h);
uint16_t mh3o_bf16_from_float(float f);
uint16_t mh3o_bf16_from_double(double d);
/* n values: bf16 -> float and double -> bf16, for the tests. */
void mh3o_bf16_to_float_n(const uint16_t* in, float* out, uint64_t n);
void mh3o_bf16_from_double_n(const double* in, uint16_t* out, uint64_t n);

void mh3o_rms_mod_rows(uint32_t rows, uint32_t dim, float eps, int dtype, const void* x, const float* w,
                       const float* shift, const float* scale, const uint8_t* set_of_row, void* y);
void mh3o_gate_add_rows(uint32_t rows, uint32_t dim, int dtype, void* x, const void* y, const float* gate,
                        const uint8_t* set_of_row);
/* The same with each row array's own element type: the reference's float residual stream (docs/architecture.md:
 * 69-70) with bf16 GEMM rows, x float and y (the norm's output, or gate_add's addend) bf16. */
void mh3o_rms_mod_rows2(uint32_t rows, uint32_t dim, float eps, int xdtype, int ydtype, const void* x, const float* w,
                        const float* shift, const float* scale, const uint8_t* set_of_row, void* y);
void mh3o_gate_add_rows2(uint32_t rows, uint32_t dim, int xdtype, int ydtype, void* x, const void* y,
                         const float* gate, const uint8_t* set_of_row);
void mh3o_rms_mod_gate_add_rows(uint32_t rows, uint32_t dim, float eps, int dtype, const void* x, const void* residual,
                                const float* w, const float* shift, const float* scale, const float* gate,
                                const uint8_t* set_of_row, void* out);

void mh3o_swiglu_rows(uint32_t rows, uint32_t dim, int layout, int dtype, const void* gate, const void* up, void* out);

int64_t mh3o_cube_count(uint32_t gt, uint32_t gh, uint32_t gw);
void mh3o_cube_pool(uint32_t heads, uint32_t head_dim, uint32_t gt, uint32_t gh, uint32_t gw, int layout,
                    uint64_t row0, uint64_t head_stride, uint64_t row_stride, const uint16_t* q, const uint16_t* k,
                    float* qc, float* kc, int32_t* counts);
/* Pools only the listed (head, cube) pairs: entries [i] = head * cubes + cube, results to qc/kc[i][head_dim]. */
void mh3o_cube_pool_some(uint32_t head_dim, uint32_t gt, uint32_t gh, uint32_t gw, int layout, uint64_t row0,
                         uint64_t head_stride, uint64_t row_stride, const uint16_t* q, const uint16_t* k,
                         const int64_t* entries, uint64_t n_entries, float* qc, float* kc);
void mh3o_cube_scores(uint32_t heads, uint32_t cubes, uint32_t head_dim, const float* qc, const float* kc, double* s);
int32_t mh3o_cube_topk_row(uint32_t gt, uint32_t gh, uint32_t gw, uint32_t k, uint32_t local, uint32_t out_stride,
                           uint64_t i, const double* row, int32_t* out);
void mh3o_cube_topk(uint32_t heads, uint32_t gt, uint32_t gh, uint32_t gw, uint32_t k, uint32_t local,
                    uint32_t out_stride, const double* s, int32_t* idx, int32_t* cnt);
void mh3o_cube_topk_sorted(uint32_t heads, uint32_t gt, uint32_t gh, uint32_t gw, uint32_t k, uint32_t local,
                           uint32_t out_stride, const double* s, int32_t* idx, int32_t* cnt);

void mh3o_attn_sparse_tile(uint32_t gt, uint32_t gh, uint32_t gw, int layout, uint64_t row0, uint64_t head_stride,
                           uint64_t row_stride, uint64_t dense_row0, uint32_t n_dense, double scale,
                           const uint16_t* q, const uint16_t* k, const uint16_t* v, const int32_t* idx,
                           const int32_t* cnt, uint32_t out_stride, uint32_t h, uint64_t tile, uint16_t* out);
void mh3o_attn_sparse(uint32_t heads, uint32_t gt, uint32_t gh, uint32_t gw, int layout, uint64_t row0,
                      uint64_t head_stride, uint64_t row_stride, uint64_t dense_row0, uint32_t n_dense, double scale,
                      const uint16_t* q, const uint16_t* k, const uint16_t* v, const int32_t* idx, const int32_t* cnt,
                      uint32_t out_stride, uint16_t* out);

/* heads_partial: qkv bf16 rows [q heads | k heads | v heads] -> per-head RMS norm (q, k) and rotary on the first rot
 * values, v copied; element (h, r, d) of each output at h * out_head_stride + r * out_row_stride + d. v may be NULL. */
void mh3o_heads_partial(uint32_t rows, uint32_t model_rows, uint32_t heads, uint32_t rot, float eps,
                        uint64_t qkv_stride, uint64_t out_head_stride, uint64_t out_row_stride, const uint16_t* qkv,
                        const float* q_w, const float* k_w, const float* cos_t, const float* sin_t,
                        const int32_t* map, uint16_t* q, uint16_t* k, uint16_t* v);

void mh3o_quant_rows_i8(uint32_t rows, uint32_t cols, int dtype, const void* w, int8_t* q, float* scale);

void mh3o_gemm_w8a16_swiglu(uint32_t m, uint32_t n, uint32_t k, const uint16_t* x, const int8_t* w,
                            const float* scale, uint16_t* out);
/* The dense bf16 fc1 with the SwiGLU epilogue: w bf16 [2n][k] (gate rows, then up rows), no scale. */
void mh3o_gemm_bf16_swiglu(uint32_t m, uint32_t n, uint32_t k, const uint16_t* x, const uint16_t* w, uint16_t* out);
/* The reference's W8A8 `gemm_i8` for fc1 with the SwiGLU epilogue: x int8 [m][k] with a scale per row, w int8 [2n][k]
 * with a scale per row; exact integer sums, then y = sum * x_scale[r] * w_scale[c] in double. */
void mh3o_gemm_i8_swiglu(uint32_t m, uint32_t n, uint32_t k, const int8_t* x, const float* x_scale, const int8_t* w,
                         const float* w_scale, uint16_t* out);
/* The qkv / out / fc2 projections: y = x w^T, w [n][k]; form 0 W8A16 (w int8 + w_scale), 1 bf16, 2 W8A8 (x int8 +
 * x_scale, w int8 + w_scale). epi 0: out = y (bf16); epi 1: out += gate[set][col] * y in place (the gate_add_rows
 * epilogue, bf16 out); epi 2: the same on a float out (the reference's float residual stream). */
void mh3o_gemm(uint32_t m, uint32_t n, uint32_t k, int form, int epi, const void* x, const float* x_scale,
               const void* w, const float* w_scale, const float* gate, const uint8_t* set_of_row, uint32_t gate_stride,
               void* out);

/* H3::Cubes' map: attention row -> model row (-1 for padding), then the dense rows; counts per cube (may be NULL).
 * Returns the number of map entries. */
int64_t mh3o_cube_map(uint32_t gt, uint32_t gh, uint32_t gw, uint32_t n_dense, uint64_t video_row0,
                      uint64_t dense_row0, int32_t* map, int32_t* counts);
/* The sinusoidal embedding (cos half first) through the time MLP; temb float, cond = bf16(silu(temb)) (may be NULL). */
void mh3o_time_embed(uint32_t levels, uint32_t freq_dim, uint32_t hidden, uint32_t out_dim, double max_period,
                     const float* t, const float* w_in, const float* b_in, const float* w_out, const float* b_out,
                     float* temb, uint16_t* cond);
/* mod[u][r] = w[r] . cond[u] + bias[r], bf16 operands, double accumulation. */
void mh3o_adaln_mod(uint32_t levels, uint32_t n, uint32_t k, const uint16_t* cond, const uint16_t* w,
                    const float* bias, float* mod);
/* The pruned checkpoints' curve: table interpolated at t (points - 1), through w [n][width] plus bias. */
void mh3o_curve_mods(uint32_t levels, uint32_t n, uint32_t points, uint32_t width, const float* t, const float* table,
                     const float* w, const float* bias, float* mod);

#ifdef __cplusplus
}
#endif

#endif
