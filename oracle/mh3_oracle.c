/*
 * mh3_oracle.c — TEST INFRASTRUCTURE ONLY: the scalar CPU restatement of the H3 per-block hot path that the tests,
 * the smoke check and bench.py's CPU-baseline leg compare the GPU results with. See mh3_oracle.h for what each
 * function follows in the reference and how it is pinned. Single-threaded, double accumulation, one rounding at the
 * store (the reference's CPU idiom, src/video/audio_vae.cpp:386-416).
 */
#include "mh3_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- bf16 ----------------------------------------------------------------------------------------------------- */

float mh3o_bf16_to_float(uint16_t h)
{
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t mh3o_bf16_from_float(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u)
        return (uint16_t)((u >> 16) | 0x40u); /* NaN stays NaN (quiet) */
    u += 0x7fffu + ((u >> 16) & 1u);         /* round to nearest, ties to even */
    return (uint16_t)(u >> 16);
}

/* Nearest-even bf16 of a double, rounded once (no intermediate float rounding). bf16 keeps 8 significant bits. */
uint16_t mh3o_bf16_from_double(double d)
{
    if (isnan(d))
        return 0x7fc0u;
    if (isinf(d) || fabs(d) < 0x1p-126) /* infinities, zeros and the subnormal range: the float path is exact enough */
        return mh3o_bf16_from_float((float)d);
    int e;
    const double m = frexp(d, &e);                /* d = m * 2^e, 0.5 <= |m| < 1 */
    const double r = nearbyint(ldexp(m, 8));      /* 8 significant bits, ties to even (default rounding mode) */
    const double v = ldexp(r, e - 8);
    if (fabs(v) > 0x1.fep127)                     /* beyond bf16's largest finite value */
        return d > 0 ? 0x7f80u : 0xff80u;
    const float f = (float)v;                     /* exact: v has <= 8 significant bits */
    uint32_t u;
    memcpy(&u, &f, 4);
    return (uint16_t)(u >> 16);
}

void mh3o_bf16_to_float_n(const uint16_t* in, float* out, uint64_t n)
{
    for (uint64_t i = 0; i < n; ++i)
        out[i] = mh3o_bf16_to_float(in[i]);
}

void mh3o_bf16_from_double_n(const double* in, uint16_t* out, uint64_t n)
{
    for (uint64_t i = 0; i < n; ++i)
        out[i] = mh3o_bf16_from_double(in[i]);
}

static double load(int dtype, const void* p, uint64_t i)
{
    return dtype == MH3O_BF16 ? (double)mh3o_bf16_to_float(((const uint16_t*)p)[i]) : (double)((const float*)p)[i];
}

static void store(int dtype, void* p, uint64_t i, double v)
{
    if (dtype == MH3O_BF16)
        ((uint16_t*)p)[i] = mh3o_bf16_from_double(v);
    else
        ((float*)p)[i] = (float)v;
}

/* ---- rows ------------------------------------------------------------------------------------------------------ */

/* 1 / sqrt(mean(x^2) + eps) of row r, the sum of squares in double. */
static double inv_rms(uint32_t dim, float eps, int dtype, const void* x, uint64_t r)
{
    double ss = 0;
    for (uint32_t c = 0; c < dim; ++c) {
        const double v = load(dtype, x, r * dim + c);
        ss += v * v;
    }
    return 1.0 / sqrt(ss / (double)dim + (double)eps);
}

/* docs/architecture.md:61: "RMS norm with weight times (1 + scale) plus shift, per row"; the row's set through
 * the offset table (architecture.md:49-52). */
void mh3o_rms_mod_rows2(uint32_t rows, uint32_t dim, float eps, int xdtype, int ydtype, const void* x, const float* w,
                        const float* shift, const float* scale, const uint8_t* set_of_row, void* y)
{
    for (uint64_t r = 0; r < rows; ++r) {
        const double inv = inv_rms(dim, eps, xdtype, x, r);
        const uint64_t s = set_of_row ? set_of_row[r] : 0;
        const float* sh = shift + s * dim;
        const float* sc = scale + s * dim;
        for (uint32_t c = 0; c < dim; ++c) {
            const double n = load(xdtype, x, r * dim + c) * inv * (w ? (double)w[c] : 1.0);
            store(ydtype, y, r * dim + c, n * (1.0 + (double)sc[c]) + (double)sh[c]);
        }
    }
}

void mh3o_rms_mod_rows(uint32_t rows, uint32_t dim, float eps, int dtype, const void* x, const float* w,
                       const float* shift, const float* scale, const uint8_t* set_of_row, void* y)
{
    mh3o_rms_mod_rows2(rows, dim, eps, dtype, dtype, x, w, shift, scale, set_of_row, y);
}

/* docs/architecture.md:64-65: "the output projection times the row's gate added back" (and the same after fc2). */
void mh3o_gate_add_rows2(uint32_t rows, uint32_t dim, int xdtype, int ydtype, void* x, const void* y,
                         const float* gate, const uint8_t* set_of_row)
{
    for (uint64_t r = 0; r < rows; ++r) {
        const uint64_t s = set_of_row ? set_of_row[r] : 0;
        const float* g = gate + s * dim;
        for (uint32_t c = 0; c < dim; ++c) {
            const uint64_t i = r * dim + c;
            store(xdtype, x, i, load(xdtype, x, i) + (double)g[c] * load(ydtype, y, i));
        }
    }
}

void mh3o_gate_add_rows(uint32_t rows, uint32_t dim, int dtype, void* x, const void* y, const float* gate,
                        const uint8_t* set_of_row)
{
    mh3o_gate_add_rows2(rows, dim, dtype, dtype, x, y, gate, set_of_row);
}

/* The fused form: out = residual + gate * modRMS(x), each output rounded once. */
void mh3o_rms_mod_gate_add_rows(uint32_t rows, uint32_t dim, float eps, int dtype, const void* x, const void* residual,
                                const float* w, const float* shift, const float* scale, const float* gate,
                                const uint8_t* set_of_row, void* out)
{
    for (uint64_t r = 0; r < rows; ++r) {
        const double inv = inv_rms(dim, eps, dtype, x, r);
        const uint64_t s = set_of_row ? set_of_row[r] : 0;
        const float* sh = shift + s * dim;
        const float* sc = scale + s * dim;
        const float* g = gate + s * dim;
        for (uint32_t c = 0; c < dim; ++c) {
            const uint64_t i = r * dim + c;
            const double n = load(dtype, x, i) * inv * (w ? (double)w[c] : 1.0);
            const double m = n * (1.0 + (double)sc[c]) + (double)sh[c];
            store(dtype, out, i, load(dtype, residual, i) + (double)g[c] * m);
        }
    }
}

/* ---- swiglu ---------------------------------------------------------------------------------------------------- */

/* docs/architecture.md:65,112-114: fc1's row is [gate; value], SwiGLU = silu(gate) * value. */
void mh3o_swiglu_rows(uint32_t rows, uint32_t dim, int layout, int dtype, const void* gate, const void* up, void* out)
{
    const uint64_t gs = layout == MH3O_SWIGLU_FUSED ? 2ull * dim : dim;
    const uint64_t uoff = layout == MH3O_SWIGLU_FUSED ? dim : 0;
    const void* ub = layout == MH3O_SWIGLU_FUSED ? gate : up;
    for (uint64_t r = 0; r < rows; ++r)
        for (uint32_t c = 0; c < dim; ++c) {
            const double g = load(dtype, gate, r * gs + c);
            const double u = load(dtype, ub, r * gs + uoff + c);
            store(dtype, out, r * dim + c, g / (1.0 + exp(-g)) * u);
        }
}

/* ---- cubes ----------------------------------------------------------------------------------------------------- */

int64_t mh3o_cube_count(uint32_t gt, uint32_t gh, uint32_t gw)
{
    return (int64_t)((gt + 3) / 4) * ((gh + 3) / 4) * ((gw + 3) / 4);
}

/* The row of video position (t, y, x) of cube c's slot (dt, dy, dx), docs/architecture.md:120-125. */
static uint64_t cube_row(int layout, uint64_t row0, uint32_t gh, uint32_t gw, uint64_t c, uint32_t t, uint32_t y,
                         uint32_t x, uint32_t dt, uint32_t dy, uint32_t dx)
{
    if (layout == MH3O_CUBES_GATHERED)
        return row0 + c * 64 + (dt * 4 + dy) * 4 + dx;
    return row0 + ((uint64_t)t * gh + y) * gw + x;
}

static void pool_one(uint32_t head_dim, uint32_t gt, uint32_t gh, uint32_t gw, int layout, uint64_t row0,
                     uint64_t head_stride, uint64_t row_stride, const uint16_t* src, uint64_t h, uint64_t c,
                     double* acc, float* dst, int32_t* count_out)
{
    const uint32_t ch = (gh + 3) / 4, cw = (gw + 3) / 4;
    const uint32_t ct = (uint32_t)(c / ((uint64_t)ch * cw)), cy = (uint32_t)(c / cw % ch), cx = (uint32_t)(c % cw);
    memset(acc, 0, sizeof(double) * head_dim);
    int32_t n = 0;
    for (uint32_t dt = 0; dt < 4; ++dt)
        for (uint32_t dy = 0; dy < 4; ++dy)
            for (uint32_t dx = 0; dx < 4; ++dx) {
                const uint32_t t = ct * 4 + dt, y = cy * 4 + dy, x = cx * 4 + dx;
                if (t >= gt || y >= gh || x >= gw)
                    continue; /* padding: no token */
                const uint64_t row = cube_row(layout, row0, gh, gw, c, t, y, x, dt, dy, dx);
                const uint16_t* p = src + h * head_stride + row * row_stride;
                for (uint32_t d = 0; d < head_dim; ++d)
                    acc[d] += (double)mh3o_bf16_to_float(p[d]);
                ++n;
            }
    for (uint32_t d = 0; d < head_dim; ++d)
        dst[d] = (float)(acc[d] / (double)n); /* divisor: the cube's token count (architecture.md:124) */
    if (count_out)
        *count_out = n;
}

void mh3o_cube_pool(uint32_t heads, uint32_t head_dim, uint32_t gt, uint32_t gh, uint32_t gw, int layout,
                    uint64_t row0, uint64_t head_stride, uint64_t row_stride, const uint16_t* q, const uint16_t* k,
                    float* qc, float* kc, int32_t* counts)
{
    const uint64_t C = (uint64_t)mh3o_cube_count(gt, gh, gw);
    double* acc = (double*)malloc(sizeof(double) * head_dim);
    for (uint64_t h = 0; h < heads; ++h)
        for (uint64_t c = 0; c < C; ++c) {
            int32_t n = 0;
            pool_one(head_dim, gt, gh, gw, layout, row0, head_stride, row_stride, q, h, c, acc,
                     qc + (h * C + c) * head_dim, &n);
            pool_one(head_dim, gt, gh, gw, layout, row0, head_stride, row_stride, k, h, c, acc,
                     kc + (h * C + c) * head_dim, NULL);
            if (counts && h == 0)
                counts[c] = n;
        }
    free(acc);
}

void mh3o_cube_pool_some(uint32_t head_dim, uint32_t gt, uint32_t gh, uint32_t gw, int layout, uint64_t row0,
                         uint64_t head_stride, uint64_t row_stride, const uint16_t* q, const uint16_t* k,
                         const int64_t* entries, uint64_t n_entries, float* qc, float* kc)
{
    const uint64_t C = (uint64_t)mh3o_cube_count(gt, gh, gw);
    double* acc = (double*)malloc(sizeof(double) * head_dim);
    for (uint64_t i = 0; i < n_entries; ++i) {
        const uint64_t h = (uint64_t)entries[i] / C, c = (uint64_t)entries[i] % C;
        pool_one(head_dim, gt, gh, gw, layout, row0, head_stride, row_stride, q, h, c, acc, qc + i * head_dim, NULL);
        pool_one(head_dim, gt, gh, gw, layout, row0, head_stride, row_stride, k, h, c, acc, kc + i * head_dim, NULL);
    }
    free(acc);
}

/* docs/architecture.md:126: "scores every cube pair per head" from the pooled means; scaled by 1/sqrt(head_dim) as
 * attention scores are (the scale does not change a ranking). */
void mh3o_cube_scores(uint32_t heads, uint32_t cubes, uint32_t head_dim, const float* qc, const float* kc, double* s)
{
    const double scale = 1.0 / sqrt((double)head_dim);
    for (uint64_t h = 0; h < heads; ++h)
        for (uint64_t i = 0; i < cubes; ++i) {
            const float* a = qc + (h * cubes + i) * head_dim;
            for (uint64_t j = 0; j < cubes; ++j) {
                const float* b = kc + (h * cubes + j) * head_dim;
                double acc = 0;
                for (uint32_t d = 0; d < head_dim; ++d)
                    acc += (double)a[d] * (double)b[d];
                s[(h * cubes + i) * cubes + j] = acc * scale;
            }
        }
}

/* docs/architecture.md:126-130, README.md:81-87: for one (head, query cube i) the top k cubes by score (higher first,
 * equal scores the lower index first), united with the local cubes, as ascending indices; returns the count. O(C^2)
 * on purpose: a cube j is in the top k iff fewer than k cubes precede it in (score desc, index asc) order. */
int32_t mh3o_cube_topk_row(uint32_t gt, uint32_t gh, uint32_t gw, uint32_t k, uint32_t local, uint32_t out_stride,
                           uint64_t i, const double* row, int32_t* out)
{
    const uint32_t ch = (gh + 3) / 4, cw = (gw + 3) / 4, cth = (gt + 3) / 4;
    const uint64_t C = (uint64_t)cth * ch * cw, plane = (uint64_t)ch * cw;
    unsigned char* sel = (unsigned char*)malloc(C);
    for (uint64_t j = 0; j < C; ++j) {
        uint64_t ahead = 0;
        for (uint64_t o = 0; o < C; ++o)
            ahead += row[o] > row[j] || (row[o] == row[j] && o < j);
        sel[j] = ahead < k;
    }
    if (local >= 1)
        sel[i] = 1;
    if (local == 3) {
        const uint64_t ct = i / plane;
        if (ct > 0)
            sel[i - plane] = 1;
        if (ct + 1 < cth)
            sel[i + plane] = 1;
    }
    int32_t n = 0;
    for (uint64_t j = 0; j < C; ++j)
        if (sel[j])
            out[n++] = (int32_t)j;
    for (uint32_t j = (uint32_t)n; j < out_stride; ++j)
        out[j] = -1;
    free(sel);
    return n;
}

void mh3o_cube_topk(uint32_t heads, uint32_t gt, uint32_t gh, uint32_t gw, uint32_t k, uint32_t local,
                    uint32_t out_stride, const double* s, int32_t* idx, int32_t* cnt)
{
    const uint64_t C = (uint64_t)mh3o_cube_count(gt, gh, gw);
    for (uint64_t h = 0; h < heads; ++h)
        for (uint64_t i = 0; i < C; ++i)
            cnt[h * C + i] = mh3o_cube_topk_row(gt, gh, gw, k, local, out_stride, i, s + (h * C + i) * C,
                                                idx + (h * C + i) * out_stride);
}

/* The same selection by sorting each row once, O(C log C) a row: the form a CPU implementation would take, timed by
 * bench.py's CPU baseline. (score desc, index asc) is a total order, so it selects exactly what mh3o_cube_topk does. */
typedef struct {
    double s;
    int32_t j;
} mh3o_scored;

static int mh3o_scored_cmp(const void* pa, const void* pb)
{
    const mh3o_scored* a = (const mh3o_scored*)pa;
    const mh3o_scored* b = (const mh3o_scored*)pb;
    if (a->s != b->s)
        return a->s > b->s ? -1 : 1;
    return a->j < b->j ? -1 : (a->j > b->j);
}

void mh3o_cube_topk_sorted(uint32_t heads, uint32_t gt, uint32_t gh, uint32_t gw, uint32_t k, uint32_t local,
                           uint32_t out_stride, const double* s, int32_t* idx, int32_t* cnt)
{
    const uint32_t ch = (gh + 3) / 4, cw = (gw + 3) / 4, cth = (gt + 3) / 4;
    const uint64_t C = (uint64_t)cth * ch * cw, plane = (uint64_t)ch * cw;
    mh3o_scored* row = (mh3o_scored*)malloc(sizeof(mh3o_scored) * C);
    unsigned char* sel = (unsigned char*)malloc(C);
    for (uint64_t h = 0; h < heads; ++h)
        for (uint64_t i = 0; i < C; ++i) {
            const double* r = s + (h * C + i) * C;
            for (uint64_t j = 0; j < C; ++j) {
                row[j].s = r[j];
                row[j].j = (int32_t)j;
                sel[j] = 0;
            }
            qsort(row, C, sizeof(mh3o_scored), mh3o_scored_cmp);
            for (uint64_t j = 0; j < C && j < k; ++j)
                sel[row[j].j] = 1;
            if (local >= 1)
                sel[i] = 1;
            if (local == 3) {
                const uint64_t ct = i / plane;
                if (ct > 0)
                    sel[i - plane] = 1;
                if (ct + 1 < cth)
                    sel[i + plane] = 1;
            }
            int32_t* out = idx + (h * C + i) * out_stride;
            int32_t n = 0;
            for (uint64_t j = 0; j < C; ++j)
                if (sel[j])
                    out[n++] = (int32_t)j;
            for (uint32_t j = (uint32_t)n; j < out_stride; ++j)
                out[j] = -1;
            cnt[h * C + i] = n;
        }
    free(sel);
    free(row);
}

/* ---- heads_partial ------------------------------------------------------------------------------------------ */

/* docs/architecture.md:35-38 ("96 of each head's 128 values rotate (the first 48 with the second 48)"), :61-63 ("RMS
 * norms per head, rotary positions"), :123-125 (the head tiles gathered through the cube map, padding rows zero).
 * qkv rows are [q heads | k heads | v heads] (:61-62). Per output row r (model row map[r], or r) and head h:
 * q and k: y = x / sqrt(mean(x^2) + eps) * w, then (y_i, y_{i+half}) -> (y_i c - y_{i+half} s, y_{i+half} c + y_i s)
 * for i < half = rot / 2 with c, s = cos_t, sin_t [src][i]; one rounding. v: copied. A map entry outside
 * [0, model_rows) writes zeros. */
void mh3o_heads_partial(uint32_t rows, uint32_t model_rows, uint32_t heads, uint32_t rot, float eps,
                        uint64_t qkv_stride, uint64_t out_head_stride, uint64_t out_row_stride, const uint16_t* qkv,
                        const float* q_w, const float* k_w, const float* cos_t, const float* sin_t,
                        const int32_t* map, uint16_t* q, uint16_t* k, uint16_t* v)
{
    const uint32_t half = rot / 2;
    uint16_t* outs[3] = {q, k, v};
    const float* ws[2] = {q_w, k_w};
    for (uint64_t r = 0; r < rows; ++r) {
        const int64_t m = map ? (int64_t)map[r] : (int64_t)r;
        const int valid = m >= 0 && m < (int64_t)model_rows;
        for (uint32_t kind = 0; kind < 3; ++kind) {
            if (!outs[kind])
                continue;
            for (uint32_t h = 0; h < heads; ++h) {
                uint16_t* dst = outs[kind] + h * out_head_stride + r * out_row_stride;
                if (!valid) {
                    memset(dst, 0, 128 * sizeof(uint16_t));
                    continue;
                }
                const uint16_t* src = qkv + (uint64_t)m * qkv_stride + ((uint64_t)kind * heads + h) * 128;
                if (kind == 2) {
                    memcpy(dst, src, 128 * sizeof(uint16_t));
                    continue;
                }
                double y[128], ss = 0.0;
                for (int d = 0; d < 128; ++d) {
                    y[d] = (double)mh3o_bf16_to_float(src[d]);
                    ss += y[d] * y[d];
                }
                const double inv = 1.0 / sqrt(ss / 128.0 + (double)eps);
                for (int d = 0; d < 128; ++d)
                    y[d] *= inv * (ws[kind] ? (double)ws[kind][d] : 1.0);
                double o[128];
                memcpy(o, y, sizeof o);
                for (uint32_t i = 0; i < half; ++i) {
                    const double c = cos_t[(uint64_t)m * half + i], s = sin_t[(uint64_t)m * half + i];
                    o[i] = y[i] * c - y[i + half] * s;
                    o[i + half] = y[i + half] * c + y[i] * s;
                }
                for (int d = 0; d < 128; ++d)
                    dst[d] = mh3o_bf16_from_double(o[d]);
            }
        }
    }
}

/* ---- int8 ------------------------------------------------------------------------------------------------------ */

/* docs/performance.md:122-123: "int8 rows with a float scale each (symmetric, the row's maximum at 127)". The scale
 * and the division are float, as the device computes them; rounding to nearest even. */
void mh3o_quant_rows_i8(uint32_t rows, uint32_t cols, int dtype, const void* w, int8_t* q, float* scale)
{
    for (uint64_t r = 0; r < rows; ++r) {
        float mx = 0.0f;
        for (uint32_t c = 0; c < cols; ++c) {
            const float v = fabsf((float)load(dtype, w, r * cols + c));
            mx = v > mx ? v : mx;
        }
        const float s = mx / 127.0f;
        scale[r] = s;
        for (uint32_t c = 0; c < cols; ++c) {
            if (s == 0.0f) {
                q[r * cols + c] = 0;
                continue;
            }
            float v = nearbyintf((float)load(dtype, w, r * cols + c) / s);
            v = v > 127.0f ? 127.0f : (v < -127.0f ? -127.0f : v);
            q[r * cols + c] = (int8_t)v;
        }
    }
}

/* docs/performance.md:124-126 (the int8 GEMM scaled in the epilogue) and architecture.md:65 (fc1's [gate; value]
 * rows, then SwiGLU), in the weight-only form: y = x * (W * diag s), out = silu(y_gate) * y_up. */
void mh3o_gemm_w8a16_swiglu(uint32_t m, uint32_t n, uint32_t k, const uint16_t* x, const int8_t* w,
                            const float* scale, uint16_t* out)
{
    double* xr = (double*)malloc(sizeof(double) * k);
    for (uint64_t r = 0; r < m; ++r) {
        for (uint32_t i = 0; i < k; ++i)
            xr[i] = (double)mh3o_bf16_to_float(x[r * k + i]);
        for (uint64_t c = 0; c < n; ++c) {
            const int8_t* wg = w + c * k;
            const int8_t* wu = w + (n + c) * k;
            double g = 0, u = 0;
            for (uint32_t i = 0; i < k; ++i) {
                g += xr[i] * (double)wg[i];
                u += xr[i] * (double)wu[i];
            }
            g *= (double)scale[c];
            u *= (double)scale[n + c];
            out[r * n + c] = mh3o_bf16_from_double(g / (1.0 + exp(-g)) * u);
        }
    }
    free(xr);
}

void mh3o_gemm_bf16_swiglu(uint32_t m, uint32_t n, uint32_t k, const uint16_t* x, const uint16_t* w, uint16_t* out)
{
    double* xr = (double*)malloc(sizeof(double) * k);
    double* wg = (double*)malloc(sizeof(double) * k);
    double* wu = (double*)malloc(sizeof(double) * k);
    for (uint64_t c = 0; c < n; ++c) {
        for (uint32_t i = 0; i < k; ++i) {
            wg[i] = (double)mh3o_bf16_to_float(w[c * k + i]);
            wu[i] = (double)mh3o_bf16_to_float(w[(n + c) * k + i]);
        }
        for (uint64_t r = 0; r < m; ++r) {
            double g = 0, u = 0;
            for (uint32_t i = 0; i < k; ++i) {
                const double xv = (double)mh3o_bf16_to_float(x[r * k + i]);
                g += xv * wg[i];
                u += xv * wu[i];
            }
            out[r * n + c] = mh3o_bf16_from_double(g / (1.0 + exp(-g)) * u);
        }
    }
    free(xr);
    free(wg);
    free(wu);
}

void mh3o_gemm_i8_swiglu(uint32_t m, uint32_t n, uint32_t k, const int8_t* x, const float* x_scale, const int8_t* w,
                         const float* w_scale, uint16_t* out)
{
    for (uint64_t r = 0; r < m; ++r) {
        const int8_t* xr = x + r * k;
        for (uint64_t c = 0; c < n; ++c) {
            const int8_t* wg = w + c * k;
            const int8_t* wu = w + (n + c) * k;
            int64_t ig = 0, iu = 0;
            for (uint32_t i = 0; i < k; ++i) {
                ig += (int64_t)xr[i] * wg[i];
                iu += (int64_t)xr[i] * wu[i];
            }
            const double g = (double)ig * (double)x_scale[r] * (double)w_scale[c];
            const double u = (double)iu * (double)x_scale[r] * (double)w_scale[n + c];
            out[r * n + c] = mh3o_bf16_from_double(g / (1.0 + exp(-g)) * u);
        }
    }
}

/* The qkv, out and fc2 projections (docs/performance.md:40-43,52-69,120-133; docs/architecture.md:61-66): y = x w^T
 * with w [n][k] in one of three forms (form 0: x bf16, w int8 with w_scale; 1: both bf16; 2: x int8 with x_scale, w
 * int8 with w_scale), exact products summed in double (int64 for the int8 pair). epi 0: out = y (bf16); epi 1:
 * out += gate[s][col] * y with s = set_of_row[row] (NULL: 0), out bf16 in place, one rounding. */
void mh3o_gemm(uint32_t m, uint32_t n, uint32_t k, int form, int epi, const void* x, const float* x_scale,
               const void* w, const float* w_scale, const float* gate, const uint8_t* set_of_row, uint32_t gate_stride,
               void* out)
{
    double* xr = (double*)malloc(sizeof(double) * k);
    for (uint64_t r = 0; r < m; ++r) {
        for (uint32_t i = 0; i < k; ++i)
            xr[i] = form == 2 ? (double)((const int8_t*)x)[r * k + i]
                              : (double)mh3o_bf16_to_float(((const uint16_t*)x)[r * k + i]);
        const uint64_t set = set_of_row ? set_of_row[r] : 0;
        for (uint64_t c = 0; c < n; ++c) {
            double y = 0;
            if (form == 2) {
                int64_t acc = 0;
                for (uint32_t i = 0; i < k; ++i)
                    acc += (int64_t)xr[i] * ((const int8_t*)w)[c * k + i];
                y = (double)acc * (double)x_scale[r] * (double)w_scale[c];
            } else {
                for (uint32_t i = 0; i < k; ++i)
                    y += xr[i] * (form == 0 ? (double)((const int8_t*)w)[c * k + i]
                                            : (double)mh3o_bf16_to_float(((const uint16_t*)w)[c * k + i]));
                if (form == 0)
                    y *= (double)w_scale[c];
            }
            uint16_t* o = (uint16_t*)out + r * n + c;
            float* of = (float*)out + r * n + c;
            if (epi == 0)
                *o = mh3o_bf16_from_double(y);
            else if (epi == 1)
                *o = mh3o_bf16_from_double((double)mh3o_bf16_to_float(*o) + (double)gate[set * gate_stride + c] * y);
            else
                *of = (float)((double)*of + (double)gate[set * gate_stride + c] * y);
        }
    }
    free(xr);
}

/* ---- flash_attn_sparse_128 -------------------------------------------------------------------------------------- */

/* Row of slot l (0..63) of attention tile `tile`: tiles 0 .. nd-1 are the dense rows in runs of 64 (row
 * dense_row0 + 64 tile + l, valid below n_dense), tile nd + c is cube c (slot l = (dt, dy, dx) = (l / 16, l / 4 % 4,
 * l % 4), valid where its grid position is a token). Returns the row, or -1 for a slot that is no token. */
static int64_t attn_tile_row(uint32_t gt, uint32_t gh, uint32_t gw, int layout, uint64_t row0, uint64_t dense_row0,
                             uint32_t n_dense, uint64_t tile, uint32_t l)
{
    const uint64_t nd = ((uint64_t)n_dense + 63) / 64;
    if (tile < nd) {
        const uint64_t r = 64 * tile + l;
        return r < n_dense ? (int64_t)(dense_row0 + r) : -1;
    }
    const uint64_t c = tile - nd;
    const uint32_t ch = (gh + 3) / 4, cw = (gw + 3) / 4;
    const uint32_t ct = (uint32_t)(c / ((uint64_t)ch * cw)), cy = (uint32_t)(c / cw % ch), cx = (uint32_t)(c % cw);
    const uint32_t dt = l / 16, dy = l / 4 % 4, dx = l % 4;
    const uint32_t t = ct * 4 + dt, y = cy * 4 + dy, x = cx * 4 + dx;
    if (t >= gt || y >= gh || x >= gw)
        return -1;
    return (int64_t)cube_row(layout, row0, gh, gw, c, t, y, x, dt, dy, dx);
}

/* docs/architecture.md:123-130: flash attention over a pass list. The queries of cube i (head h) attend the rows of
 * the cubes idx[h][i][0 .. cnt[h][i]) and every dense row; a dense row's query attends every row (all cubes and
 * dense rows); padding slots are neither keys nor outputs. softmax(q . k * scale) v per query, in double, rounded
 * to bf16 once. One query tile (the numbering of attn_tile_row) of one head; in the gathered layout a cube's
 * padding slots are written zero. */
void mh3o_attn_sparse_tile(uint32_t gt, uint32_t gh, uint32_t gw, int layout, uint64_t row0, uint64_t head_stride,
                           uint64_t row_stride, uint64_t dense_row0, uint32_t n_dense, double scale,
                           const uint16_t* q, const uint16_t* k, const uint16_t* v, const int32_t* idx,
                           const int32_t* cnt, uint32_t out_stride, uint32_t h, uint64_t tile, uint16_t* out)
{
    const uint32_t hd = 128;
    const uint64_t C = (uint64_t)mh3o_cube_count(gt, gh, gw), nd = ((uint64_t)n_dense + 63) / 64;
    /* the key tiles of this query tile */
    uint64_t n_kt = 0;
    uint64_t* kt = (uint64_t*)malloc(sizeof(uint64_t) * (C + nd));
    if (tile < nd) {
        for (uint64_t c = 0; c < C; ++c)
            kt[n_kt++] = nd + c;
    } else {
        const uint64_t i = tile - nd;
        const int32_t* list = idx + ((uint64_t)h * C + i) * out_stride;
        for (int32_t e = 0; e < cnt[(uint64_t)h * C + i]; ++e)
            kt[n_kt++] = nd + (uint64_t)list[e];
    }
    for (uint64_t d = 0; d < nd; ++d)
        kt[n_kt++] = d;
    double* s = (double*)malloc(sizeof(double) * 64 * (n_kt ? n_kt : 1));
    int64_t* krow = (int64_t*)malloc(sizeof(int64_t) * 64 * (n_kt ? n_kt : 1));
    uint64_t nk = 0;
    for (uint64_t e = 0; e < n_kt; ++e)
        for (uint32_t l = 0; l < 64; ++l) {
            const int64_t r = attn_tile_row(gt, gh, gw, layout, row0, dense_row0, n_dense, kt[e], l);
            if (r >= 0)
                krow[nk++] = r;
        }
    double acc[128];
    for (uint32_t l = 0; l < 64; ++l) {
        const int64_t qr = attn_tile_row(gt, gh, gw, layout, row0, dense_row0, n_dense, tile, l);
        if (qr < 0) {
            if (layout == MH3O_CUBES_GATHERED && tile >= nd) { /* gathered: the padding slot's row exists; it is written zero */
                uint16_t* o = out + (uint64_t)h * head_stride + (row0 + 64 * (tile - nd) + l) * row_stride;
                memset(o, 0, sizeof(uint16_t) * hd);
            }
            continue;
        }
        const uint16_t* qp = q + (uint64_t)h * head_stride + (uint64_t)qr * row_stride;
        double mx = -INFINITY;
        for (uint64_t j = 0; j < nk; ++j) {
            const uint16_t* kp = k + (uint64_t)h * head_stride + (uint64_t)krow[j] * row_stride;
            double dot = 0;
            for (uint32_t d = 0; d < hd; ++d)
                dot += (double)mh3o_bf16_to_float(qp[d]) * (double)mh3o_bf16_to_float(kp[d]);
            s[j] = dot * scale;
            mx = s[j] > mx ? s[j] : mx;
        }
        double sum = 0;
        memset(acc, 0, sizeof acc);
        for (uint64_t j = 0; j < nk; ++j) {
            const double p = exp(s[j] - mx);
            const uint16_t* vp = v + (uint64_t)h * head_stride + (uint64_t)krow[j] * row_stride;
            sum += p;
            for (uint32_t d = 0; d < hd; ++d)
                acc[d] += p * (double)mh3o_bf16_to_float(vp[d]);
        }
        uint16_t* o = out + (uint64_t)h * head_stride + (uint64_t)qr * row_stride;
        for (uint32_t d = 0; d < hd; ++d)
            o[d] = mh3o_bf16_from_double(sum > 0 ? acc[d] / sum : 0.0);
    }
    free(krow);
    free(s);
    free(kt);
}

void mh3o_attn_sparse(uint32_t heads, uint32_t gt, uint32_t gh, uint32_t gw, int layout, uint64_t row0,
                      uint64_t head_stride, uint64_t row_stride, uint64_t dense_row0, uint32_t n_dense, double scale,
                      const uint16_t* q, const uint16_t* k, const uint16_t* v, const int32_t* idx, const int32_t* cnt,
                      uint32_t out_stride, uint16_t* out)
{
    const uint64_t tiles = ((uint64_t)n_dense + 63) / 64 + (uint64_t)mh3o_cube_count(gt, gh, gw);
    for (uint32_t h = 0; h < heads; ++h)
        for (uint64_t t = 0; t < tiles; ++t)
            mh3o_attn_sparse_tile(gt, gh, gw, layout, row0, head_stride, row_stride, dense_row0, n_dense, scale, q,
                                  k, v, idx, cnt, out_stride, h, t, out);
}

/* ---- H3::Cubes' map (docs/architecture.md:120-125) -------------------------------------------------------------- */

/* Written as a scatter: every slot starts as padding (-1), then each video token (t, y, x) of the grid is placed at
 * its cube's slot ((t % 4) * 4 + y % 4) * 4 + x % 4 and counted; the dense rows follow the cubes. */
int64_t mh3o_cube_map(uint32_t gt, uint32_t gh, uint32_t gw, uint32_t n_dense, uint64_t video_row0,
                      uint64_t dense_row0, int32_t* map, int32_t* counts)
{
    const uint32_t ch = (gh + 3u) / 4u, cw = (gw + 3u) / 4u;
    const int64_t cubes = mh3o_cube_count(gt, gh, gw);
    for (int64_t r = 0; r < cubes * 64; ++r)
        map[r] = -1;
    if (counts)
        for (int64_t c = 0; c < cubes; ++c)
            counts[c] = 0;
    for (uint32_t t = 0; t < gt; ++t)
        for (uint32_t y = 0; y < gh; ++y)
            for (uint32_t x = 0; x < gw; ++x) {
                const uint64_t c = ((uint64_t)(t / 4u) * ch + y / 4u) * cw + x / 4u;
                const uint32_t slot = ((t % 4u) * 4u + y % 4u) * 4u + x % 4u;
                map[c * 64u + slot] = (int32_t)(video_row0 + ((uint64_t)t * gh + y) * gw + x);
                if (counts)
                    counts[c] += 1;
            }
    for (uint32_t j = 0; j < n_dense; ++j)
        map[cubes * 64 + j] = (int32_t)(dense_row0 + j);
    return cubes * 64 + n_dense;
}

/* ---- time conditioning (docs/architecture.md:49-58, tools/check_pruned_curve.py:57-73) ------------------------- */

static double silu_d(double v) { return v / (1.0 + exp(-v)); }

void mh3o_time_embed(uint32_t levels, uint32_t freq_dim, uint32_t hidden, uint32_t out_dim, double max_period,
                     const float* t, const float* w_in, const float* b_in, const float* w_out, const float* b_out,
                     float* temb, uint16_t* cond)
{
    const uint32_t half = freq_dim / 2;
    double* emb = malloc(sizeof(double) * freq_dim);
    double* hid = malloc(sizeof(double) * hidden);
    for (uint32_t u = 0; u < levels; ++u) {
        for (uint32_t i = 0; i < half; ++i) {
            const double arg = (double)t[u] * exp(-log(max_period) * (double)i / (double)half);
            emb[i] = cos(arg);
            emb[half + i] = sin(arg);
        }
        for (uint32_t r = 0; r < hidden; ++r) {
            double s = b_in ? b_in[r] : 0.0;
            for (uint32_t i = 0; i < freq_dim; ++i)
                s += (double)w_in[(uint64_t)r * freq_dim + i] * emb[i];
            hid[r] = silu_d(s);
        }
        for (uint32_t j = 0; j < out_dim; ++j) {
            double s = b_out ? b_out[j] : 0.0;
            for (uint32_t i = 0; i < hidden; ++i)
                s += (double)w_out[(uint64_t)j * hidden + i] * hid[i];
            temb[(uint64_t)u * out_dim + j] = (float)s;
            if (cond)
                cond[(uint64_t)u * out_dim + j] = mh3o_bf16_from_double(silu_d(s));
        }
    }
    free(emb);
    free(hid);
}

void mh3o_adaln_mod(uint32_t levels, uint32_t n, uint32_t k, const uint16_t* cond, const uint16_t* w,
                    const float* bias, float* mod)
{
    for (uint32_t u = 0; u < levels; ++u)
        for (uint32_t r = 0; r < n; ++r) {
            double s = bias ? bias[r] : 0.0;
            for (uint32_t i = 0; i < k; ++i)
                s += (double)mh3o_bf16_to_float(w[(uint64_t)r * k + i]) *
                     (double)mh3o_bf16_to_float(cond[(uint64_t)u * k + i]);
            mod[(uint64_t)u * n + r] = (float)s;
        }
}

void mh3o_curve_mods(uint32_t levels, uint32_t n, uint32_t points, uint32_t width, const float* t, const float* table,
                     const float* w, const float* bias, float* mod)
{
    double* c = malloc(sizeof(double) * width);
    for (uint32_t u = 0; u < levels; ++u) {
        double pos = (double)t[u] * (double)(points - 1);
        pos = pos < 0 ? 0 : (pos > (double)(points - 1) ? (double)(points - 1) : pos);
        uint32_t i0 = (uint32_t)floor(pos);
        if (i0 > points - 2)
            i0 = points - 2;
        const double f = pos - (double)i0;
        for (uint32_t j = 0; j < width; ++j)
            c[j] = (1.0 - f) * table[(uint64_t)i0 * width + j] + f * table[(uint64_t)(i0 + 1) * width + j];
        for (uint32_t r = 0; r < n; ++r) {
            double s = bias ? bias[r] : 0.0;
            for (uint32_t j = 0; j < width; ++j)
                s += (double)w[(uint64_t)r * width + j] * c[j];
            mod[(uint64_t)u * n + r] = (float)s;
        }
    }
    free(c);
}
