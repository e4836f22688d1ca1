// Row kernels of the H3 block: the adaLN-modulated RMS norm (`rms_mod_rows`), the gated residual add
// (`gate_add_rows`), the two fused into one HBM pass, and `swiglu_rows`. Reference semantics: the mako-common
// kernels of these names, described in docs/architecture.md:49-52,61-66 and docs/performance.md:44.
//
// Design (gfx950): one wavefront owns a row at a time and keeps all of it in VGPRs (16-byte loads, 8 bf16 or 4
// float a lane per vector), so x is read from HBM once: the sum of squares is a lane-local sum plus a 6-step
// butterfly, and the second pass runs from registers. The per-column coefficients of a modulation set
// (a = w (1 + scale) gate, b = shift gate) are folded once per workgroup into LDS and read from there for every row
// the workgroup's waves stream through (a persistent grid), so the parameter vectors cost no HBM or L2 traffic per
// row. Streaming data uses non-temporal loads and stores.
#include "mh3_common.hpp"

namespace mh3 {

enum RowOp { kRmsMod = 0, kGateAdd = 1, kFused = 2 };

// A 16-byte vector of row elements.
template <int DT>
struct RowVec;

template <>
struct RowVec<MH3_BF16> {
    static constexpr int N = 8;
    __device__ static void unpack(const uint4& r, float (&f)[8])
    {
        f[0] = bf16_lo(r.x), f[1] = bf16_hi(r.x), f[2] = bf16_lo(r.y), f[3] = bf16_hi(r.y);
        f[4] = bf16_lo(r.z), f[5] = bf16_hi(r.z), f[6] = bf16_lo(r.w), f[7] = bf16_hi(r.w);
    }
    __device__ static uint4 pack(const float (&f)[8])
    {
        return uint4{pack_bf16(f[0], f[1]), pack_bf16(f[2], f[3]), pack_bf16(f[4], f[5]), pack_bf16(f[6], f[7])};
    }
};

template <>
struct RowVec<MH3_F32> {
    static constexpr int N = 4;
    __device__ static void unpack(const uint4& r, float (&f)[4])
    {
        f[0] = __uint_as_float(r.x), f[1] = __uint_as_float(r.y), f[2] = __uint_as_float(r.z);
        f[3] = __uint_as_float(r.w);
    }
    __device__ static uint4 pack(const float (&f)[4])
    {
        return uint4{__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3])};
    }
};

struct RowsParams {
    const uint4* x;   // rms_mod / fused: the normed input; gate_add: the addend y
    const uint4* res; // fused: the residual; gate_add: x (in/out)
    uint4* out;
    const float* w;
    const float* shift;
    const float* scale;
    const float* gate;
    const uint8_t* set_of_row;
    uint32_t rows, dim, nvec, n_sets;
    float eps, inv_dim;
    int coef_in_lds;
};

// The per-column coefficients of set s: y = (x * inv) * a + b (rms_mod), out = res + (x * inv) * a + b (fused),
// out = res + a * y (gate_add).
template <int OP>
__device__ __forceinline__ void coef(const RowsParams& p, uint32_t s, uint32_t c, float& a, float& b)
{
    const uint64_t i = uint64_t(s) * p.dim + c;
    if constexpr (OP == kGateAdd) {
        a = p.gate[i];
        b = 0.0f;
    } else {
        const float w = p.w ? p.w[c] : 1.0f;
        const float m = w * (1.0f + p.scale[i]);
        if constexpr (OP == kFused) {
            const float g = p.gate[i];
            a = m * g;
            b = p.shift[i] * g;
        } else {
            a = m;
            b = p.shift[i];
        }
    }
}

template <int DT, int NV, int OP>
__global__ __launch_bounds__(512) void rows_kernel(RowsParams p)
{
    using V = RowVec<DT>;
    constexpr int E = V::N;
    extern __shared__ float lds[]; // a[n_sets][dim], then b[n_sets][dim]
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;

    if (p.coef_in_lds) {
        const uint32_t total = p.n_sets * p.dim;
        for (uint32_t i = threadIdx.x; i < total; i += blockDim.x) {
            const uint32_t s = i / p.dim, c = i - s * p.dim;
            float a, b;
            coef<OP>(p, s, c, a, b);
            lds[i] = a;
            lds[total + i] = b;
        }
        __syncthreads();
    }
    const uint32_t coef_total = p.n_sets * p.dim;

    for (uint32_t row = blockIdx.x * waves + wave; row < p.rows; row += gridDim.x * waves) {
        const uint32_t set = p.set_of_row ? min(uint32_t(p.set_of_row[row]), p.n_sets - 1u) : 0u;
        const uint64_t base = uint64_t(row) * p.nvec;
        uint4 xv[NV], rv[NV];
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const uint32_t v = lane + 64u * j;
            if (v < p.nvec) {
                xv[j] = ld_stream(p.x + base + v);
                if constexpr (OP != kRmsMod)
                    rv[j] = ld_stream(p.res + base + v);
            }
        }
        float inv = 1.0f;
        if constexpr (OP != kGateAdd) {
            float ss = 0.0f;
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const uint32_t v = lane + 64u * j;
                if (v < p.nvec) {
                    float f[E];
                    V::unpack(xv[j], f);
#pragma unroll
                    for (int e = 0; e < E; ++e)
                        ss = fmaf(f[e], f[e], ss);
                }
            }
            ss = wave_sum(ss);
            inv = 1.0f / sqrtf(fmaf(ss, p.inv_dim, p.eps));
        }
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const uint32_t v = lane + 64u * j;
            if (v >= p.nvec)
                continue;
            float f[E], r[E], o[E];
            V::unpack(xv[j], f);
            if constexpr (OP != kRmsMod)
                V::unpack(rv[j], r);
            const uint32_t c0 = v * E;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                float a, b;
                if (p.coef_in_lds) {
                    a = lds[set * p.dim + c0 + e];
                    b = lds[coef_total + set * p.dim + c0 + e];
                } else {
                    coef<OP>(p, set, c0 + e, a, b);
                }
                if constexpr (OP == kRmsMod)
                    o[e] = fmaf(f[e] * inv, a, b);
                else if constexpr (OP == kFused)
                    o[e] = r[e] + fmaf(f[e] * inv, a, b);
                else
                    o[e] = fmaf(a, f[e], r[e]);
            }
            st_stream(p.out + base + v, V::pack(o));
        }
    }
}

// ---- swiglu ---------------------------------------------------------------------------------------------------------

// n / d for any 32-bit n by a multiply-high and shifts (Granlund & Montgomery 1994, fig. 4.1).
struct FastDiv {
    uint32_t m, s1, s2;
    __host__ static FastDiv make(uint32_t d)
    {
        uint32_t l = 0;
        while ((uint64_t(1) << l) < d)
            ++l;
        FastDiv f;
        f.m = uint32_t(((uint64_t(1) << 32) * ((uint64_t(1) << l) - d)) / d + 1);
        f.s1 = l < 1 ? l : 1;
        f.s2 = l > 1 ? l - 1 : 0;
        return f;
    }
    __device__ __forceinline__ uint32_t div(uint32_t n) const
    {
        const uint32_t t = __umulhi(n, m);
        return (t + ((n - t) >> s1)) >> s2;
    }
};

// silu(g) * u = g / (1 + exp(-g)) * u, with exp from v_exp_f32 and one reciprocal.
__device__ __forceinline__ float silu_mul(float g, float u)
{
    const float e = __expf(-g);
    return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

template <int DT, int U>
__global__ __launch_bounds__(256) void swiglu_kernel(const uint4* gate, const uint4* up, uint4* out, uint32_t vpr,
                                                     uint32_t gstride, uint32_t ustride, uint32_t total, FastDiv div)
{
    using V = RowVec<DT>;
    constexpr int E = V::N;
    const uint32_t first = blockIdx.x * (256u * U) + threadIdx.x;
    uint4 gv[U], uv[U];
#pragma unroll
    for (int j = 0; j < U; ++j) {
        const uint32_t i = first + 256u * j;
        if (i < total) {
            const uint32_t r = div.div(i), c = i - r * vpr;
            gv[j] = ld_stream(gate + uint64_t(r) * gstride + c);
            uv[j] = ld_stream(up + uint64_t(r) * ustride + c);
        }
    }
#pragma unroll
    for (int j = 0; j < U; ++j) {
        const uint32_t i = first + 256u * j;
        if (i < total) {
            float g[E], u[E], o[E];
            V::unpack(gv[j], g);
            V::unpack(uv[j], u);
#pragma unroll
            for (int e = 0; e < E; ++e)
                o[e] = silu_mul(g[e], u[e]);
            st_stream(out + i, V::pack(o));
        }
    }
}

} // namespace mh3

// ---- C-ABI ----------------------------------------------------------------------------------------------------------
namespace {

using namespace mh3;

constexpr int kRowsBlock = 512;
constexpr size_t kCoefLdsMax = 64 * 1024;

template <int DT, int OP>
int launch_rows_dt(const RowsParams& p, hipStream_t stream)
{
    const uint32_t need = (p.nvec + 63u) / 64u;
    const void* k = nullptr;
    if (need <= 1)
        k = reinterpret_cast<const void*>(&rows_kernel<DT, 1, OP>);
    else if (need <= 2)
        k = reinterpret_cast<const void*>(&rows_kernel<DT, 2, OP>);
    else if (need <= 4)
        k = reinterpret_cast<const void*>(&rows_kernel<DT, 4, OP>);
    else if (need <= 8)
        k = reinterpret_cast<const void*>(&rows_kernel<DT, 8, OP>);
    else if (need <= 10)
        k = reinterpret_cast<const void*>(&rows_kernel<DT, 10, OP>);
    else if (need <= 12)
        k = reinterpret_cast<const void*>(&rows_kernel<DT, 12, OP>);
    else if (need <= 16)
        k = reinterpret_cast<const void*>(&rows_kernel<DT, 16, OP>);
    else
        return MH3_ERR_UNSUPPORTED;
    const size_t lds = p.coef_in_lds ? size_t(p.n_sets) * p.dim * 2 * sizeof(float) : 0;
    const int per_cu = host::blocks_per_cu(k, kRowsBlock, lds);
    const uint64_t waves = kRowsBlock / 64;
    uint64_t blocks = (p.rows + waves - 1) / waves;
    const uint64_t cap = uint64_t(host::cu_count()) * per_cu;
    if (blocks > cap)
        blocks = cap;
    RowsParams arg = p;
    void* args[] = {&arg};
    if (hipLaunchKernel(k, dim3(uint32_t(blocks)), dim3(kRowsBlock), args, lds, stream) != hipSuccess)
        return host::check_launch() == MH3_OK ? MH3_ERR_HIP : MH3_ERR_HIP;
    return host::check_launch();
}

template <int OP>
int launch_rows(const MH3RowsArgs* a, RowsParams p, hipStream_t stream)
{
    const uint32_t e = a->dtype == MH3_BF16 ? 8u : 4u;
    p.rows = a->rows;
    p.dim = a->dim;
    p.nvec = a->dim / e;
    p.n_sets = a->n_sets;
    p.eps = a->eps;
    p.inv_dim = 1.0f / float(a->dim);
    p.coef_in_lds = size_t(a->n_sets) * a->dim * 2 * sizeof(float) <= kCoefLdsMax;
    return a->dtype == MH3_BF16 ? launch_rows_dt<MH3_BF16, OP>(p, stream) : launch_rows_dt<MH3_F32, OP>(p, stream);
}

// Shared validation of the row entry points. `needs_eps` for the normed ops.
int check_rows(const MH3RowsArgs* a, bool needs_eps)
{
    if (!a)
        return MH3_ERR_POINTER;
    if (a->dtype != MH3_F32 && a->dtype != MH3_BF16)
        return MH3_ERR_PARAM;
    if (needs_eps && !(a->eps > 0.0f))
        return MH3_ERR_PARAM;
    const uint32_t e = a->dtype == MH3_BF16 ? 8u : 4u;
    if (a->dim == 0 || a->dim % e != 0 || a->n_sets == 0 || a->n_sets > 256)
        return MH3_ERR_SHAPE;
    if (a->dim / e > 16u * 64u)
        return MH3_ERR_UNSUPPORTED;
    if (a->rows >= (1u << 31))
        return MH3_ERR_SHAPE;
    return MH3_OK;
}

} // namespace

extern "C" {

int mh3_rms_mod_rows(const MH3RowsArgs* args, const void* x, const float* w, const float* shift, const float* scale,
                     const uint8_t* set_of_row, void* y, mh3_stream_t stream)
{
    int rc = check_rows(args, true);
    if (rc != MH3_OK)
        return rc;
    if (args->rows == 0)
        return MH3_OK;
    if (!x || !shift || !scale || !y)
        return MH3_ERR_POINTER;
    if (!host::aligned16(x) || !host::aligned16(y))
        return MH3_ERR_ALIGN;
    RowsParams p{};
    p.x = static_cast<const uint4*>(x);
    p.out = static_cast<uint4*>(y);
    p.w = w;
    p.shift = shift;
    p.scale = scale;
    p.set_of_row = set_of_row;
    return launch_rows<kRmsMod>(args, p, static_cast<hipStream_t>(stream));
}

int mh3_gate_add_rows(const MH3RowsArgs* args, void* x, const void* y, const float* gate, const uint8_t* set_of_row,
                      mh3_stream_t stream)
{
    int rc = check_rows(args, false);
    if (rc != MH3_OK)
        return rc;
    if (args->rows == 0)
        return MH3_OK;
    if (!x || !y || !gate)
        return MH3_ERR_POINTER;
    if (!host::aligned16(x) || !host::aligned16(y))
        return MH3_ERR_ALIGN;
    RowsParams p{};
    p.x = static_cast<const uint4*>(y);
    p.res = static_cast<const uint4*>(x);
    p.out = static_cast<uint4*>(x);
    p.gate = gate;
    p.set_of_row = set_of_row;
    return launch_rows<kGateAdd>(args, p, static_cast<hipStream_t>(stream));
}

int mh3_rms_mod_gate_add_rows(const MH3RowsArgs* args, const void* x, const void* residual, const float* w,
                              const float* shift, const float* scale, const float* gate, const uint8_t* set_of_row,
                              void* out, mh3_stream_t stream)
{
    int rc = check_rows(args, true);
    if (rc != MH3_OK)
        return rc;
    if (args->rows == 0)
        return MH3_OK;
    if (!x || !residual || !shift || !scale || !gate || !out)
        return MH3_ERR_POINTER;
    if (!host::aligned16(x) || !host::aligned16(residual) || !host::aligned16(out))
        return MH3_ERR_ALIGN;
    RowsParams p{};
    p.x = static_cast<const uint4*>(x);
    p.res = static_cast<const uint4*>(residual);
    p.out = static_cast<uint4*>(out);
    p.w = w;
    p.shift = shift;
    p.scale = scale;
    p.gate = gate;
    p.set_of_row = set_of_row;
    return launch_rows<kFused>(args, p, static_cast<hipStream_t>(stream));
}

int mh3_swiglu_rows(const MH3SwigluArgs* a, const void* gate, const void* up, void* out, mh3_stream_t stream)
{
    if (!a)
        return MH3_ERR_POINTER;
    if (a->dtype != MH3_F32 && a->dtype != MH3_BF16)
        return MH3_ERR_PARAM;
    if (a->layout != MH3_SWIGLU_SPLIT && a->layout != MH3_SWIGLU_FUSED)
        return MH3_ERR_PARAM;
    const uint32_t e = a->dtype == MH3_BF16 ? 8u : 4u;
    if (a->dim == 0 || a->dim % e != 0)
        return MH3_ERR_SHAPE;
    const uint32_t vpr = a->dim / e;
    if (uint64_t(a->rows) * vpr >= (uint64_t(1) << 32) - 4096u * 4u)
        return MH3_ERR_SHAPE;
    if (a->rows == 0)
        return MH3_OK;
    if (!gate || !out || (a->layout == MH3_SWIGLU_SPLIT && !up))
        return MH3_ERR_POINTER;
    if (a->layout == MH3_SWIGLU_FUSED && up)
        return MH3_ERR_PARAM;
    if (!host::aligned16(gate) || !host::aligned16(out) || (up && !host::aligned16(up)))
        return MH3_ERR_ALIGN;
    const uint4* g = static_cast<const uint4*>(gate);
    const uint4* u = a->layout == MH3_SWIGLU_FUSED ? g + vpr : static_cast<const uint4*>(up);
    const uint32_t stride = a->layout == MH3_SWIGLU_FUSED ? 2u * vpr : vpr;
    const uint32_t total = a->rows * vpr;
    constexpr int U = 4;
    const uint32_t blocks = (total + 256u * U - 1) / (256u * U);
    const FastDiv div = FastDiv::make(vpr);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (a->dtype == MH3_BF16)
        hipLaunchKernelGGL((swiglu_kernel<MH3_BF16, U>), dim3(blocks), dim3(256), 0, s, g, u,
                           static_cast<uint4*>(out), vpr, stride, stride, total, div);
    else
        hipLaunchKernelGGL((swiglu_kernel<MH3_F32, U>), dim3(blocks), dim3(256), 0, s, g, u, static_cast<uint4*>(out),
                           vpr, stride, stride, total, div);
    return host::check_launch();
}

} // extern "C"
