/*
 * mako_h3.h — C-ABI of the MI355X (gfx950) kernels for the per-block hot path of mako-video's MiniMax-H3
 * transformer: the adaLN-modulated RMS norm and the gated residual (`rms_mod_rows`, `gate_add_rows`, fused),
 * `swiglu_rows`, the `--sparse` cube selector (`cube_pool`, `cube_scores`, `cube_topk`, fused `cube_select`),
 * the `--int8` weight quantizer (`quant_rows_i8`) and the int8 weight-only fc1 GEMM with its SwiGLU epilogue.
 *
 * The reference runs these as Metal kernels looked up by name in mako-common's TransformerRuntime
 * (`dispatch(enc, name, {buffers}, &args, sizeof args, grid, tg)`, the in-repo instance being
 * src/video/audio_vae.cpp:151-177 over src/kernels/video.metal:10-36). This header keeps that shape:
 *   - one entry point per reference kernel name, prefixed `mh3_`;
 *   - one argument struct of fixed-width fields per entry point, passed by pointer (the reference's setBytes);
 *   - device buffers as plain pointers, owned by the caller (the reference's reserve()/scratch());
 *   - an explicit stream (a hipStream_t; NULL is the null stream), the counterpart of the reference's encoder;
 *   - no allocation, no exceptions: every call returns an int, MH3_OK or a negative MH3_ERR_* code, and an
 *     invalid call launches nothing (the reference throws std::runtime_error on the host, audio_vae.cpp:231-232).
 * Calls are asynchronous on the given stream; all entry points are reentrant and may be called from several host
 * threads on distinct streams.
 *
 * Every pointer is a device pointer unless its comment says otherwise. Dense tensors are row-major and contiguous
 * unless a stride says otherwise. 16-byte vector accesses require the row widths and pointers the comments state.
 */
#ifndef MAKO_H3_H
#define MAKO_H3_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MH3_ABI_VERSION 5

/* ---- error codes ------------------------------------------------------------------------------------------------ */
enum {
    MH3_OK = 0,
    MH3_ERR_SHAPE = -1,       /* a size is zero where it may not be, too large, or not a required multiple */
    MH3_ERR_POINTER = -2,     /* a required pointer is NULL */
    MH3_ERR_ALIGN = -3,       /* a pointer is not aligned as required (16 bytes for vector rows) */
    MH3_ERR_PARAM = -4,       /* a scalar parameter is outside its domain (dtype, layout, ratio, local, k, eps) */
    MH3_ERR_HIP = -5,         /* the HIP runtime reported an error launching the kernel */
    MH3_ERR_UNSUPPORTED = -6, /* a valid request the library has no kernel for (e.g. head_dim != 128) */
};

/* Element types of activations. */
enum { MH3_F32 = 0, MH3_BF16 = 1 };

/* A hipStream_t, kept opaque so the header needs no HIP include. */
typedef void* mh3_stream_t;

/* ---- library ---------------------------------------------------------------------------------------------------- */
int mh3_abi_version(void);
/* A static string for an MH3_* code. */
const char* mh3_strerror(int code);
/* The last HIP error string seen by a launch on this thread ("" if none). */
const char* mh3_last_hip_error(void);

/* ---- H3 options (host only, no GPU needed) ---------------------------------------------------------------------- */
/* The transformer matrices kept as int8 (reference: H3::Int8 mask, engine.hpp:34; parse_int8 called at
 * tools/mako_video.cpp:110, src/server/video_models.cpp:128, tests/h3_ref_test.cpp:139). */
enum { MH3_INT8_QKV = 1u, MH3_INT8_OUT = 2u, MH3_INT8_FC1 = 4u, MH3_INT8_FC2 = 8u, MH3_INT8_ALL = 15u };
/* "none", "all", or a comma list of qkv, out, fc1, fc2 -> *mask (host memory). MH3_ERR_PARAM (mask untouched) for
 * anything else, as the reference's parse_int8 returns no value. */
int mh3_parse_int8(const char* text, uint32_t* mask);
/* H3::set_sparse's domain (reference: src/server/video_models.cpp:117-126): ratio in [0, 1], local in {0, 1, 3}. */
int mh3_check_sparse(float ratio, uint32_t local);
/* The cubes a query cube keeps by score: ceil(ratio * cubes), clamped to [0, cubes], with the float ratio read as the
 * decimal it stands for (a product within 2^-22 cubes above an integer counts as that integer: 0.1 of 660 cubes is
 * 66); a negative code (MH3_ERR_PARAM) for a ratio outside [0, 1]. */
int64_t mh3_topk_k(float ratio, uint32_t cubes);

/* ---- rows: rms_mod_rows, gate_add_rows, fused rms_mod_gate_add_rows ----------------------------------------------
 * Reference kernels `rms_mod_rows` and `gate_add_rows` (mako-common; named in docs/performance.md:44, semantics in
 * docs/architecture.md:49-52,61,64-65). A row r uses modulation set s(r) = set_of_row[r] (uint8, device memory) when
 * set_of_row is non-NULL, else 0; a value >= n_sets is read as n_sets - 1. shift, scale and gate are [n_sets][dim]
 * float, w is [dim] float (NULL: all 1). x, residual, y and out are [rows][dim] of `dtype`. bf16 rows need
 * dim % 8 == 0, float rows dim % 4 == 0; every pointer, the float vectors included, 16-byte aligned. Math is float,
 * the sum of squares accumulated in float, and bf16 results are rounded to nearest even once, at the store. An output
 * may equal an input row array where stated below; any other overlap of an output with an input (the float vectors
 * and set_of_row included) or with another output is refused (MH3_ERR_PARAM). */
typedef struct MH3RowsArgs {
    uint32_t rows;
    uint32_t dim;
    uint32_t n_sets; /* 1 .. 256 */
    uint32_t dtype;  /* MH3_F32 or MH3_BF16 */
    float eps;       /* > 0 (H3: 1e-6) */
    /* Floats from set s's shift, scale and gate vectors to set s + 1's; 0 means dim (separate [n_sets][dim]
     * arrays). Otherwise a multiple of 4 and at least dim: shift, scale and gate may then point into one table of
     * interleaved vectors, such as the reference's [U][3][6][D] modulation table (h3_ref_test.cpp:229-241), whose
     * (level, tag) sets are 6 D floats apart. */
    uint32_t set_stride;
    uint32_t flags; /* 0, or MH3_ROWS_* below (dtype MH3_F32 only) */
    uint32_t reserved;
} MH3RowsArgs;
/* The reference's float residual stream (docs/architecture.md:69-70: activations are fp32 and go into the bf16 GEMMs
 * rounded to bf16). With dtype MH3_F32, x (and the residual) are float rows and these flags make the GEMMs' rows bf16:
 *   MH3_ROWS_NORM_BF16: the modulated norm's output (y of mh3_rms_mod_rows, h of mh3_gate_add_rms_mod_rows) is bf16,
 *                       the float result rounded once to nearest even: the next GEMM's input;
 *   MH3_ROWS_Y_BF16:    the gated addend y (mh3_gate_add_rows, mh3_gate_add_rms_mod_rows) is bf16, a GEMM's output.
 * mh3_rms_mod_rows takes NORM_BF16, mh3_gate_add_rows Y_BF16, mh3_gate_add_rms_mod_rows NORM_BF16 alone or with
 * Y_BF16 (its results then equal, bit for bit, mh3_gate_add_rows and mh3_rms_mod_rows with the same flags), and
 * mh3_rms_mod_gate_add_rows none; any other flag, or a flag with dtype MH3_BF16, is MH3_ERR_PARAM. Under a flag
 * dim % 8 == 0 and dim <= 6144 (MH3_ERR_UNSUPPORTED beyond), and a bf16 row array may not share memory with a float
 * one (MH3_ERR_PARAM). */
enum { MH3_ROWS_NORM_BF16 = 1u, MH3_ROWS_Y_BF16 = 2u };

/* y = x * rsqrt(mean(x^2) + eps) * w * (1 + scale[s]) + shift[s]. y may equal x. */
int mh3_rms_mod_rows(const MH3RowsArgs* args, const void* x, const float* w, const float* shift, const float* scale,
                     const uint8_t* set_of_row, void* y, mh3_stream_t stream);
/* x += gate[s] * y, in place (the reference's residual update after out-proj and after fc2). y may equal x. */
int mh3_gate_add_rows(const MH3RowsArgs* args, void* x, const void* y, const float* gate, const uint8_t* set_of_row,
                      mh3_stream_t stream);
/* out = residual + gate[s] * (x * rsqrt(mean(x^2) + eps) * w * (1 + scale[s]) + shift[s]): the two reference
 * kernels fused into one HBM pass (reads x and residual once, writes out once). out may equal residual or x. */
int mh3_rms_mod_gate_add_rows(const MH3RowsArgs* args, const void* x, const void* residual, const float* w,
                              const float* shift, const float* scale, const float* gate, const uint8_t* set_of_row,
                              void* out, mh3_stream_t stream);
/* The block's own order after the out projection and after fc2 (docs/architecture.md:61-66): x += gate[s] * y,
 * then h = the modulated RMS norm of the updated x with this half's w, shift[s] and scale[s], as the next GEMM's
 * input. One HBM pass (reads x and y, writes x and h) with the same results, bit for bit, as mh3_gate_add_rows
 * followed by mh3_rms_mod_rows on the updated x. h may not overlap x or y; y may equal x. */
int mh3_gate_add_rms_mod_rows(const MH3RowsArgs* args, void* x, const void* y, const float* gate, const float* w,
                              const float* shift, const float* scale, const uint8_t* set_of_row, void* h,
                              mh3_stream_t stream);

/* ---- swiglu_rows -------------------------------------------------------------------------------------------------
 * Reference kernel `swiglu_rows` (mako-common; docs/architecture.md:65,112-114): out = silu(gate) * up with
 * silu(g) = g / (1 + exp(-g)), float math, out rounded once. fc1's row is [gate (dim) | up (dim)].
 *   MH3_SWIGLU_SPLIT: gate and up are separate [rows][dim] tensors.
 *   MH3_SWIGLU_FUSED: gate points at [rows][2*dim] rows (gate = columns [0, dim), up = [dim, 2*dim)); up is NULL.
 * out is [rows][dim]. dim % 8 == 0 (bf16) or % 4 == 0 (float); 16-byte aligned pointers. In the split layout out may
 * equal gate or up; otherwise it may not overlap them (MH3_ERR_PARAM). */
enum { MH3_SWIGLU_SPLIT = 0, MH3_SWIGLU_FUSED = 1 };
typedef struct MH3SwigluArgs {
    uint32_t rows;
    uint32_t dim;
    uint32_t layout; /* MH3_SWIGLU_SPLIT or MH3_SWIGLU_FUSED */
    uint32_t dtype;  /* MH3_F32 or MH3_BF16 */
} MH3SwigluArgs;
int mh3_swiglu_rows(const MH3SwigluArgs* args, const void* gate, const void* up, void* out, mh3_stream_t stream);

/* ---- the sparse-attention cube selector ---------------------------------------------------------------------------
 * Reference: H3::Cubes and cube_pool / cube_scores / cube_topk (mako-common; docs/architecture.md:118-133,
 * README.md:81-87, docs/performance.md:162-181). The generated video rows form a grid of grid_t latent frames x
 * grid_h patch rows x grid_w patch columns, frame-major then row-major. Cubes are 4x4x4 blocks of it, the grid padded
 * up to multiples of 4 with rows that are no token; cube c = (ct * ch + cy) * cw + cx with ch = ceil(grid_h / 4),
 * cw = ceil(grid_w / 4). Q and K are bf16 per head: element (head, row, d) at
 * head * head_stride + row * row_stride + d, head_dim = 128 contiguous, row_stride and head_stride multiples of 8.
 *   MH3_CUBES_GRID:     video row (t, y, x) is row row0 + (t * grid_h + y) * grid_w + x (the model's order).
 *   MH3_CUBES_GATHERED: rows already gathered cube by cube (the reference's heads_partial with the cube map):
 *                       cube c's 64 rows are rows row0 + 64 c ... + 63, in (dt, dy, dx) order; padding rows are
 *                       skipped by their grid position, whatever they hold.
 * cube_pool:  qc[h][c][:] = mean of q over cube c's valid rows (float), same for k; counts[c] = valid rows (int32,
 *             may be NULL).
 * cube_scores: s[h][i][j] = qc[h][i] . kc[h][j] / sqrt(head_dim), float [heads][cubes][cubes]. The dot products
 *             are the four bf16 MFMA products of each float's bf16 high and low parts, accumulated in float: within
 *             about 1e-5 of the row's largest score (a float contraction: 1e-6); a 16 x 16 block with a non-finite
 *             score (infinite or NaN operands, or ones beyond bf16's range) is computed by float FMAs instead.
 *             cube_select computes the same scores bit for bit.
 * cube_topk:  per (h, query cube i): the k cubes of highest s[h][i][:] (equal scores: lower cube index first),
 *             united with the local cubes (local 1: i itself; 3: also the cubes of the same (cy, cx) one frame group
 *             before and after, where they exist), written as ascending int32 cube indices
 *             idx[h][i][0 .. cnt[h][i]) with idx[h][i][cnt .. out_stride) = -1; cnt[h][i] = k + the local cubes not
 *             already among the k. out_stride >= k + local.
 * cube_select: cube_scores and cube_topk fused; the scores stay on chip. Up to 2048 cubes (MH3_ERR_UNSUPPORTED
 *             beyond: use cube_scores + cube_topk, which take up to 4096). `workspace` (device memory, 16-byte
 *             aligned, at least mh3_cube_select_workspace_bytes(args) bytes, MH3_ERR_SHAPE if smaller; the call
 *             overwrites it, so calls that overlap in time need their own) holds kc split into the bf16 parts the
 *             matrix cores take, prepared once a call for all of its query cubes.
 * Each call's outputs may not overlap its inputs or each other (MH3_ERR_PARAM): for q and k the span from the array's
 * start to the last head's last row read.
 * mh3_cube_count() gives the number of cubes of a grid; mh3_topk_k() gives k for a ratio. */
enum { MH3_CUBES_GRID = 0, MH3_CUBES_GATHERED = 1 };
typedef struct MH3CubeArgs {
    uint32_t heads;
    uint32_t head_dim; /* 128 */
    uint32_t grid_t, grid_h, grid_w;
    uint32_t layout;      /* MH3_CUBES_GRID or MH3_CUBES_GATHERED */
    uint64_t row0;        /* first video row */
    uint64_t head_stride; /* elements between heads of q / k */
    uint64_t row_stride;  /* elements between rows of q / k */
    uint32_t k;           /* cubes kept by score, 1 <= k <= cubes (cube_topk, cube_select) */
    uint32_t local;       /* 0, 1 or 3 */
    uint32_t out_stride;  /* int32 entries per (head, query cube) in idx, >= k + local */
    uint32_t reserved;
} MH3CubeArgs;
int64_t mh3_cube_count(uint32_t grid_t, uint32_t grid_h, uint32_t grid_w);
int mh3_cube_pool(const MH3CubeArgs* args, const uint16_t* q, const uint16_t* k, float* qc, float* kc,
                  int32_t* counts, mh3_stream_t stream);
int mh3_cube_scores(const MH3CubeArgs* args, const float* qc, const float* kc, float* s, mh3_stream_t stream);
int mh3_cube_topk(const MH3CubeArgs* args, const float* s, int32_t* idx, int32_t* cnt, mh3_stream_t stream);
int64_t mh3_cube_select_workspace_bytes(const MH3CubeArgs* args); /* a negative code for invalid args */
int mh3_cube_select(const MH3CubeArgs* args, const float* qc, const float* kc, void* workspace,
                    uint64_t workspace_bytes, int32_t* idx, int32_t* cnt, mh3_stream_t stream);

/* The query-cube order for mh3_flash_attn_sparse_128_ordered. No counterpart in the reference: a scheduling input for
 * this library's attention. For each head h, order[h][r] (int32 [heads][cubes]) is the cube of rank r when the head's
 * cubes are sorted by the middle entry idx[h][c][n / 2] of their pass lists, n = cnt[h][c] clamped to
 * [0, out_stride] as the attention clamps it (the median of the ascending lists cube_topk and cube_select write; an
 * empty list, or an entry outside [0, cubes), sorts as `cubes`), equal entries by cube index: a permutation of
 * [0, cubes). Uses heads, grid and out_stride (>= 1) of args; up to 4096
 * cubes (MH3_ERR_UNSUPPORTED beyond). Pointers 4-byte aligned; order may not overlap idx or cnt (MH3_ERR_PARAM). */
int mh3_cube_order(const MH3CubeArgs* args, const int32_t* idx, const int32_t* cnt, int32_t* order,
                   mh3_stream_t stream);

/* H3::Cubes' map (docs/architecture.md:120-125), built in the reference's begin(): the attention's row order, the
 * generated video rows in 4x4x4 cubes of (latent frame, patch row, patch column), the grid padded to multiples of 4
 * with rows that are no token, then the dense rows (text, keyframe and audio), which every query attends. For
 * attention row r < cubes * 64 (cube c = r / 64, slot l = r % 64 = (dt * 4 + dy) * 4 + dx, token
 * (t, y, x) = (4 ct + dt, 4 cy + dy, 4 cx + dx)): map[r] = video_row0 + (t * grid_h + y) * grid_w + x, the token's
 * model row, or -1 where (t, y, x) lies in the padding (the row's validity is map[r] >= 0). For r = cubes * 64 + j,
 * j < n_dense: map[r] = dense_row0 + j. counts[c] = cube c's token count (int32 [cubes], may be NULL). map is int32
 * [cubes * 64 + n_dense], the map mh3_heads_partial gathers through (its rows then come out in the MH3_CUBES_GATHERED
 * order). Model rows must fit int32, and the dense rows may not overlap the video rows (MH3_ERR_PARAM); nor may map
 * and counts overlap (MH3_ERR_PARAM). */
typedef struct MH3CubeMapArgs {
    uint32_t grid_t, grid_h, grid_w;
    uint32_t n_dense;    /* dense rows after the cubes; 0 allowed */
    uint64_t video_row0; /* model row of video token (0, 0, 0); the grid follows frame-major, then row-major */
    uint64_t dense_row0; /* model row of the first dense row; the dense rows are consecutive model rows */
} MH3CubeMapArgs;
int mh3_cube_map(const MH3CubeMapArgs* args, int32_t* map, int32_t* counts, mh3_stream_t stream);

/* ---- heads_partial ------------------------------------------------------------------------------------------------
 * Reference kernel `heads_partial` (mako-common; docs/architecture.md:35-38,61-63,123-125; docs/performance.md:44):
 * the step between the QKV GEMM and attention. qkv holds one model row a row, [q (heads x 128) | k (heads x 128) |
 * v (heads x 128)] bf16, the order the reference stacks the fused QKV weight in (docs/architecture.md:61-62). For
 * output row r, its model row src = map[r] (r when map is NULL), and head h:
 *   q: y = x * rsqrt(mean(x^2) + eps) * q_w over the head's 128 values, in float; then the rotary positions on the
 *      first `rot` values: value i < rot / 2 pairs with value i + rot / 2,
 *      (a, b) -> (a cos - b sin, b cos + a sin), cos = cos_t[src][i], sin = sin_t[src][i];
 *      values rot .. 127 pass unrotated; one rounding to bf16;
 *   k: the same with k_w;
 *   v: copied (skipped when v is NULL).
 * A map entry outside [0, model_rows) (-1: a cube's padding slot at the grid's edge) writes zeros to every output of
 * its row and reads nothing. The outputs put element (h, r, d) at h * out_head_stride + r * out_row_stride + d: the head tiles
 * [heads][rows][128], or the model's own [rows][heads * 128] order. With a cube map the rows come out in the order
 * cube_pool, cube_select and flash_attn_sparse_128 take as MH3_CUBES_GATHERED (cube c's 64 slots at rows 64 c ..,
 * then the dense rows). cos_t and sin_t are float [model_rows][rot / 2] (NULL when rot is 0); q_w and k_w are
 * float [128] shared by the heads (NULL: all 1). The outputs may overwrite their own inputs in place (map NULL, each
 * output at its input's position); otherwise they may not overlap qkv. No output may overlap q_w, k_w, cos_t, sin_t
 * or map (MH3_ERR_PARAM). */
typedef struct MH3HeadsArgs {
    uint32_t rows;       /* output rows */
    uint32_t model_rows; /* rows of qkv, cos_t and sin_t */
    uint32_t heads;
    uint32_t head_dim;   /* 128 */
    uint32_t rot;        /* rotating values a head: a multiple of 16, <= head_dim (H3: 96) */
    float eps;           /* > 0 */
    uint64_t qkv_stride; /* elements between model rows of qkv: >= 3 heads head_dim, a multiple of 8 */
    uint64_t out_head_stride, out_row_stride; /* elements, multiples of 8 */
} MH3HeadsArgs;
int mh3_heads_partial(const MH3HeadsArgs* args, const uint16_t* qkv, const float* q_w, const float* k_w,
                      const float* cos_t, const float* sin_t, const int32_t* map, uint16_t* q, uint16_t* k,
                      uint16_t* v, mh3_stream_t stream);
/* heads_partial and cube_pool in one pass: the outputs of mh3_heads_partial(args, qkv, q_w, k_w, cos_t, sin_t, map,
 * q, k, v) followed by mh3_cube_pool(cubes, q, k, qc, kc, counts), bit for bit, without reading q and k back. The
 * reference runs the two kernels one after the other (docs/architecture.md:123-128: the head tiles are gathered
 * through the cube map, then the selector pools them); this entry point has no reference counterpart of its own.
 * cubes must describe the head tiles this call writes: the same heads and head_dim, head_stride = out_head_stride
 * and row_stride = out_row_stride (MH3_ERR_PARAM otherwise), in either layout:
 *   MH3_CUBES_GATHERED: the cube rows row0 .. row0 + 64 cubes - 1, gathered through map (or not), within args->rows;
 *   MH3_CUBES_GRID: no map (MH3_ERR_PARAM), output rows in the model's order, the grid's tokens at rows
 *                   row0 .. row0 + T H W - 1 within args->rows.
 * (MH3_ERR_SHAPE when the rows do not fit.) Rows outside them (the dense rows) get heads_partial alone. qc and kc are
 * float [heads][cubes][128], 16-byte aligned. qc, kc and counts may not overlap each other, any input, or q, k and v
 * (each taken as the span from its start to the last head's last row), else MH3_ERR_PARAM. */
int mh3_heads_partial_pool(const MH3HeadsArgs* args, const MH3CubeArgs* cubes, const uint16_t* qkv, const float* q_w,
                           const float* k_w, const float* cos_t, const float* sin_t, const int32_t* map, uint16_t* q,
                           uint16_t* k, uint16_t* v, float* qc, float* kc, int32_t* counts, mh3_stream_t stream);

/* ---- flash_attn_sparse_128 ---------------------------------------------------------------------------------------
 * Reference kernel `flash_attn_sparse_128` (mako-common; docs/architecture.md:123-130, docs/performance.md:162-181):
 * flash attention, head_dim 128, over the pass lists of cube_topk / cube_select. Per head h:
 *   - the queries of cube i attend the tokens of cubes idx[h][i][0 .. cnt[h][i]) and every dense row;
 *   - a dense row's query attends every token of the grid and every dense row;
 *   - out[row] = softmax(q[row] . k * scale) v over those keys, bf16, accumulated in float.
 * q, k, v and out share the cube geometry of `cubes` (rows addressed as for cube_pool, in the grid or gathered
 * layout); the dense rows are rows dense_row0 .. + n_dense of the same arrays and may not overlap the video rows.
 * Output rows are written where the queries lie: the grid layout writes the token rows and the dense rows (the
 * reference's write-back to the model's rows, with no gather or scatter pass); the gathered layout also writes a
 * cube's padding slots, as zeros. idx entries outside [0, cubes) are skipped; cnt is clamped to [0, out_stride].
 * out may not overlap q, k, v, idx or cnt, q, k, v and out each taken as the span from its start to the last head's
 * last row read or written (MH3_ERR_PARAM). cubes.k and cubes.local are not used. */
typedef struct MH3AttnArgs {
    MH3CubeArgs cubes;   /* heads, head_dim (128), grid, layout, row0, head_stride, row_stride; out_stride: idx's
                            int32 entries per (head, query cube) */
    uint64_t dense_row0; /* first dense row (text, keyframe and audio rows) */
    uint32_t n_dense;    /* dense rows; 0 allowed */
    float scale;         /* score scale; 0 means 1 / sqrt(128) */
} MH3AttnArgs;
int mh3_flash_attn_sparse_128(const MH3AttnArgs* args, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                              const int32_t* idx, const int32_t* cnt, uint16_t* out, mh3_stream_t stream);
/* The same attention with the query cubes of each head scheduled in `order` (int32 [heads][cubes], a permutation of
 * [0, cubes) per head, as mh3_cube_order writes; entries are clamped to [0, cubes), and a non-permutation leaves
 * some cubes unwritten and computes others twice). No counterpart in the reference: it is flash_attn_sparse_128 with
 * a scheduling input. When the cubes and the heads' dense tiles divide into eighths, each XCD takes a contiguous
 * eighth of a head's cubes in this order (otherwise the cube tiles simply follow it), so cubes whose pass lists
 * centre on the same keys run together and share K/V tiles in that XCD's L2. The outputs equal the plain call's up to the softmax's summation
 * order. order may not overlap out (MH3_ERR_PARAM) and must be 4-byte aligned. */
int mh3_flash_attn_sparse_128_ordered(const MH3AttnArgs* args, const uint16_t* q, const uint16_t* k,
                                      const uint16_t* v, const int32_t* idx, const int32_t* cnt, const int32_t* order,
                                      uint16_t* out, mh3_stream_t stream);

/* ---- int8 weights: quant_rows_i8 (weight side) ---------------------------------------------------------------------
 * Reference kernel `quant_rows_i8` (mako-common; docs/performance.md:122-123, docs/architecture.md:54-56): each row
 * of a [rows][cols] matrix (the weight's [out][in] rows) to symmetric int8 with one float scale:
 * scale = max|row| / 127 (float), q = round-to-nearest-even(w / scale) in [-127, 127]; an all-zero row gets
 * scale 0 and q 0. w is float or bf16 (`dtype`), cols % 16 == 0, 16-byte aligned. q and scale may not overlap w or
 * each other (MH3_ERR_PARAM). */
typedef struct MH3QuantArgs {
    uint32_t rows;
    uint32_t cols;
    uint32_t dtype; /* MH3_F32 or MH3_BF16 */
    uint32_t reserved;
} MH3QuantArgs;
int mh3_quant_rows_i8(const MH3QuantArgs* args, const void* w, int8_t* q, float* scale, mh3_stream_t stream);

/* ---- the int8 weight-only fc1 GEMM with the SwiGLU epilogue --------------------------------------------------------
 * Replaces fc1's `gemm_i8` + `swiglu_rows` pair (mako-common; docs/performance.md:120-136, docs/architecture.md:65).
 * x is bf16 [m][k]; w is int8 [2n][k], the weight's output-channel rows as quant_rows_i8 leaves them (rows [0, n)
 * the gate, [n, 2n) the up projection); scale is float [2n]. With W the [k][2n] matrix w^T:
 *   y = x * (W * diag(scale)) in float accumulation, out = silu(y[:, 0:n]) * y[:, n:2n], bf16 [m][n].
 * The int8 -> bf16 widening is exact (|w| <= 127); the scale is applied to the float accumulator.
 * k % 64 == 0, n % 128 == 0, m >= 1; x, w and out 16-byte aligned. The kernel addresses w and a 256-row block of x
 * with 32-bit offsets: n * k < 2^30 and k < 2^22, else MH3_ERR_UNSUPPORTED (H3's fc1, n = 14,336 and k = 5376,
 * uses 7.7e7). For every GEMM entry point, out (the residual for mh3_gemm_gate_add) may not overlap x, w or the
 * scale, gate and set_of_row vectors (MH3_ERR_PARAM): other tiles are still reading them. */
typedef struct MH3GemmArgs {
    uint32_t m;
    uint32_t n;           /* output columns; w has 2n rows with a SwiGLU epilogue, n rows otherwise */
    uint32_t k;
    uint32_t n_sets;      /* mh3_gemm_gate_add: gate sets (0 means 1); unused by the other calls */
    uint32_t gate_stride; /* mh3_gemm_gate_add: floats between consecutive gate sets (0 means n) */
    uint32_t reserved;
} MH3GemmArgs;
int mh3_gemm_w8a16_swiglu(const MH3GemmArgs* args, const uint16_t* x, const int8_t* w, const float* scale,
                          uint16_t* out, mh3_stream_t stream);
/* The dense bf16 fc1 with the same epilogue: the reference's bf16 `Gemm::encode` for fc1 (docs/performance.md:52-69,
 * the `--int8 none` path) + `swiglu_rows`. w is bf16 [2n][k] (gate rows, then up rows), no scale:
 *   y = x * w^T in float accumulation, out = silu(y[:, 0:n]) * y[:, n:2n], bf16 [m][n].
 * Same shape rules as mh3_gemm_w8a16_swiglu, with n * k < 2^29. */
int mh3_gemm_bf16_swiglu(const MH3GemmArgs* args, const uint16_t* x, const uint16_t* w, uint16_t* out,
                         mh3_stream_t stream);
/* The reference's own `--int8` fc1 (docs/performance.md:120-133): W8A8 `gemm_i8` on the int8 MFMA with the SwiGLU
 * epilogue. x is int8 [m][k] with x_scale float [m] (mh3_quant_rows_i8 of the bf16 activations), w int8 [2n][k] with
 * w_scale float [2n]; int32 accumulation (exact), then
 *   y = sum * x_scale[row] * w_scale[col] in float, out = silu(y[:, 0:n]) * y[:, n:2n], bf16 [m][n].
 * k % 128 == 0, n % 128 == 0, m >= 1; x, w and out 16-byte aligned; n * k < 2^30. */
int mh3_gemm_i8_swiglu(const MH3GemmArgs* args, const int8_t* x, const float* x_scale, const int8_t* w,
                       const float* w_scale, uint16_t* out, mh3_stream_t stream);

/* ---- the block's other GEMMs: the qkv, out and fc2 projections -------------------------------------------------
 * The reference's bf16 `Gemm::encode` for the QKV, output and fc2 projections, and its `gemm_i8` for them under
 * --int8 qkv,out,fc2 (mako-common; docs/performance.md:40-43,52-69,120-133; docs/architecture.md:61-66), on the fc1
 * kernel with two other epilogues. w is [n][k], the weight's output-channel rows. `form` picks the operands:
 *   MH3_GEMM_BF16:  x bf16 [m][k], w bf16, no scales (x_scale and w_scale unused);
 *   MH3_GEMM_W8A16: x bf16, w int8 with w_scale float [n] (weight-only, the int8 -> bf16 widening exact);
 *   MH3_GEMM_W8A8:  x int8 with x_scale float [m] (mh3_quant_rows_i8 of the activations), w int8 with w_scale [n],
 *                   on the int8 MFMA with exact int32 sums.
 * y = x w^T in float accumulation, times w_scale[col] and x_scale[row] where the form has them.
 *   mh3_gemm:          out[m][n] = y, bf16 (the qkv projection: n = 3 heads 128, its rows [q | k | v]).
 *   mh3_gemm_gate_add: residual[row][col] += gate[s][col] * y, bf16 in place with one rounding, s = set_of_row[row]
 *                      (NULL: set 0), gate float [n_sets][gate_stride]: the out projection and fc2 with the block's
 *                      `gate_add_rows` folded into the epilogue (docs/architecture.md:64-66).
 * k % 64 == 0 (k % 128 == 0 for W8A8), n % 256 == 0, m >= 1; x, w and out 16-byte aligned; w below 2^31 bytes and
 * 256 k below 2^31 bytes of x, else MH3_ERR_UNSUPPORTED. */
enum { MH3_GEMM_W8A16 = 0, MH3_GEMM_BF16 = 1, MH3_GEMM_W8A8 = 2 };
int mh3_gemm(const MH3GemmArgs* args, uint32_t form, const void* x, const float* x_scale, const void* w,
             const float* w_scale, uint16_t* out, mh3_stream_t stream);
int mh3_gemm_gate_add(const MH3GemmArgs* args, uint32_t form, const void* x, const float* x_scale, const void* w,
                      const float* w_scale, const float* gate, const uint8_t* set_of_row, uint16_t* residual,
                      mh3_stream_t stream);
/* mh3_gemm_gate_add on the reference's float residual stream (docs/architecture.md:69-70: the GEMMs take bf16 rows,
 * the residual stays float): residual is float [m][n], residual[row][col] = fmaf(gate[s][col], y, residual[row][col])
 * with y the scaled float accumulator, in place; x is the bf16 (or int8) row the GEMM takes. The same shape, form and
 * aliasing rules as mh3_gemm_gate_add. */
int mh3_gemm_gate_add_f32(const MH3GemmArgs* args, uint32_t form, const void* x, const float* x_scale, const void* w,
                          const float* w_scale, const float* gate, const uint8_t* set_of_row, float* residual,
                          mh3_stream_t stream);

/* ---- time conditioning: the producer of the modulation table ---------------------------------------------------
 * What turns a step's distinct noise levels t = 1 - sigma (one to three in H3) into the [U][3][6][D] modulation
 * table that the row kernels read through set_stride (docs/architecture.md:49-58; written out in torch in
 * tools/check_pruned_curve.py:57-73; compared in tests/h3_ref_test.cpp:226-241).
 *
 * mh3_time_embed: for each level u,
 *   emb = [cos(t[u] f_0) .. cos(t[u] f_{h-1}), sin(t[u] f_0) .. sin(t[u] f_{h-1})], h = freq_dim / 2,
 *         f_i = exp(-ln(max_period) i / h)  (the sinusoidal embedding, cos half first);
 *   hid = silu(w_in emb + b_in)              (w_in float [hidden][freq_dim], b_in [hidden]);
 *   temb[u] = w_out hid + b_out              (w_out float [out_dim][hidden], b_out [out_dim]): the F32 time MLP;
 *   cond[u] = bf16(silu(temb[u]))            (rounded once, to nearest even): the AdaLN projections' input.
 * t is float [levels] in device memory; temb is float [levels][out_dim]; cond is bf16 [levels][out_dim] (may be
 * NULL); b_in and b_out may be NULL (zero). The embedding is computed in double, the MLP in float. `workspace` holds
 * the hidden layer: at least mh3_time_embed_workspace_bytes(args) bytes of device memory, 16-byte aligned, which the
 * call overwrites (a negative code from the query for invalid args). temb, cond and the workspace may not overlap
 * each other or an input (MH3_ERR_PARAM). */
typedef struct MH3TimeArgs {
    uint32_t levels;   /* 1 .. 64 */
    uint32_t freq_dim; /* a multiple of 8, <= 1024 (H3: 256) */
    uint32_t hidden;   /* a multiple of 4, <= 8192 (H3: 5376) */
    uint32_t out_dim;  /* >= 1 (H3: 2688) */
    float max_period;  /* > 1 (H3: 10000) */
    uint32_t reserved[3];
} MH3TimeArgs;
int64_t mh3_time_embed_workspace_bytes(const MH3TimeArgs* args);
int mh3_time_embed(const MH3TimeArgs* args, const float* t, const float* w_in, const float* b_in, const float* w_out,
                   const float* b_out, void* workspace, uint64_t workspace_bytes, float* temb, uint16_t* cond,
                   mh3_stream_t stream);
/* mh3_time_embed without a workspace: it calls no allocator of any kind, so callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc) can produce the
 * conditioning. This entry point has no counterpart in the reference. The hidden layer lives in a 256 KiB array of
 * the library's own, one per GPU, held until the process ends: levels * hidden must be at most 65,536 floats (H3's
 * 3 levels of 5376 use 16,128), else MH3_ERR_UNSUPPORTED. Every call on a GPU shares that GPU's array, so calls that
 * overlap in time on one GPU (on different streams, or from several host threads) race; calls on one stream, or
 * ordered by events, do not. Each call writes the part of the array it reads before reading it. Same results as
 * mh3_time_embed, bit for bit. The call uses the current device's array, so a non-NULL stream must belong to the
 * current device (MH3_ERR_PARAM otherwise). MH3_ERR_HIP if the array's address on the current device cannot be
 * obtained. */
int mh3_time_embed_noalloc(const MH3TimeArgs* args, const float* t, const float* w_in, const float* b_in,
                           const float* w_out, const float* b_out, float* temb, uint16_t* cond, mh3_stream_t stream);
/* A block's AdaLN projection (and the final layer's, n = 2 D): mod[u][r] = w[r] . cond[u] + bias[r] in float
 * accumulation, u < args->m levels, r < args->n. cond is bf16 [m][k] (mh3_time_embed's output), w bf16 [n][k] (the
 * weight's output rows), bias float [n] (may be NULL), mod float [m][n]. With n = 3 * 6 * D the rows of a level are
 * its [3 tags][6 vectors][D], so mod is the [U][3][6][D] table whose set (u, tag) the row kernels take at
 * set_stride = 6 D. k % 8 == 0 and k <= 4096, else MH3_ERR_SHAPE / MH3_ERR_UNSUPPORTED; m <= 64; cond and w 16-byte
 * aligned; mod may not overlap cond, w or bias (MH3_ERR_PARAM). args->n_sets and gate_stride are not used. */
int mh3_adaln_mod(const MH3GemmArgs* args, const uint16_t* cond, const uint16_t* w, const float* bias, float* mod,
                  mh3_stream_t stream);
/* The pruned checkpoints' path (docs/architecture.md:53-58, tools/check_pruned_curve.py:69-73): no time MLP; a curve
 * c(t) is tabulated at `points` values of t over [0, 1] (table float [points][width], H3: [1025][8]) and read with
 * linear interpolation at pos = t (points - 1), clamped to [0, points - 1]: i0 = min(floor(pos), points - 2),
 * f = pos - i0, c = (1 - f) table[i0] + f table[i0 + 1]; then mod[u][r] = w[r] . c(t[u]) + bias[r] in float, with w
 * float [n][width] and no silu. t is float [levels] in device memory; bias may be NULL; mod may not overlap an input
 * (MH3_ERR_PARAM). */
typedef struct MH3CurveArgs {
    uint32_t levels; /* 1 .. 64 */
    uint32_t n;      /* outputs a level */
    uint32_t points; /* >= 2 */
    uint32_t width;  /* 1 .. 32 (H3: 8) */
} MH3CurveArgs;
int mh3_curve_mods(const MH3CurveArgs* args, const float* t, const float* table, const float* w, const float* bias,
                   float* mod, mh3_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MAKO_H3_H */
