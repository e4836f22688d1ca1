// `quant_rows_i8`: each row to symmetric int8 with one float scale. Weights go through it once at load; under the
// W8A8 fc1 the bf16 activations go through it every step, so it is a streaming kernel on the hot path.
// Reference: the mako-common kernel of this name, described in docs/performance.md:122-126 and
// docs/architecture.md:54-56 ("int8 rows with a float scale each (symmetric, the row's maximum at 127)").
// One wavefront per row. Rows of up to 8192 elements are read once and held in registers between the max-|w| step
// and the quantize step; wider rows are read twice.
#include "mh3_common.hpp"

namespace mh3 {

// 16 row elements as loaded: bf16 two 16-byte vectors, float four. Held raw and widened where used, so a row kept
// in registers costs 8 VGPRs a chunk in bf16 instead of 16.
template <int DT>
struct Chunk {
    static constexpr int kVecs = DT == MH3_BF16 ? 2 : 4;
    uint4 v[kVecs];
};

template <int DT>
__device__ __forceinline__ Chunk<DT> load_chunk(const void* p, uint64_t chunk)
{
    const uint4* q = static_cast<const uint4*>(p) + chunk * Chunk<DT>::kVecs;
    Chunk<DT> c;
#pragma unroll
    for (int i = 0; i < Chunk<DT>::kVecs; ++i)
        c.v[i] = q[i];
    return c;
}

template <int DT>
__device__ __forceinline__ void widen(const Chunk<DT>& c, float (&v)[16])
{
#pragma unroll
    for (int i = 0; i < Chunk<DT>::kVecs; ++i) {
        const uint32_t w[4] = {c.v[i].x, c.v[i].y, c.v[i].z, c.v[i].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if constexpr (DT == MH3_BF16) {
                v[8 * i + 2 * j] = bf16_lo(w[j]);
                v[8 * i + 2 * j + 1] = bf16_hi(w[j]);
            } else {
                v[4 * i + j] = __uint_as_float(w[j]);
            }
        }
    }
}

template <int DT>
__device__ __forceinline__ float chunk_absmax(const Chunk<DT>& c, float mx)
{
    float v[16];
    widen(c, v);
#pragma unroll
    for (int i = 0; i < 16; ++i)
        mx = fmaxf(mx, fabsf(v[i]));
    return mx;
}

// The quotient v / s rounded to nearest, bit-identical to IEEE division for 2^-100 <= s <= 2^100 and |v| <= 128 s.
// y is the refined reciprocal of s from row_recip. This is the Newton-Raphson / Markstein sequence (P. Markstein,
// IBM J. Res. Dev. 34(1), 1990) that the AMDGPU backend emits for a correctly rounded f32 division, with the steps
// that depend on s alone done once a row. The backend's sequence also brackets it with v_div_scale / v_div_fmas /
// v_div_fixup, which rescale operands near the ends of the exponent range and handle zero and non-finite operands. In
// this range of s they change nothing whose quotient can round away from 0: they rescale only when |v| < 2^-103 or
// v / s is subnormal, where |v / s| < 1/8 and both forms round to 0, and v == 0 gives 0 here as through v_div_fixup.
__device__ __forceinline__ float row_recip(float s)
{
    const float r = __builtin_amdgcn_rcpf(s);
    return fmaf(fmaf(-s, r, 1.0f), r, r);
}

__device__ __forceinline__ float div_by(float v, float s, float y)
{
    const float q0 = v * y;
    const float q1 = fmaf(fmaf(-s, q0, v), y, q0);
    return fmaf(fmaf(-s, q1, v), y, q1);
}

// 16 values to int8, rint(v / s) clamped to +-127, packed little-endian into one 16-byte vector. FAST: s in the
// range where div_by equals the division; otherwise s is any non-zero scale.
template <bool FAST>
__device__ __forceinline__ uint4 quant16(const float (&v)[16], float s, float y)
{
    uint32_t packed[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        float r = rintf(FAST ? div_by(v[i], s, y) : v[i] / s);
        r = fminf(fmaxf(r, -127.0f), 127.0f);
        packed[i >> 2] |= (uint32_t(int32_t(r)) & 0xffu) << (8 * (i & 3));
    }
    return uint4{packed[0], packed[1], packed[2], packed[3]};
}

// The largest |v| of a row, wave-uniform. Non-negative floats order as their bit patterns, so the DPP maximum of the
// patterns is the float maximum (NaN elements were already skipped by fmaxf).
__device__ __forceinline__ float row_absmax(float mx)
{
    return __uint_as_float(wave_max_u32(__float_as_uint(mx)));
}

// CPL > 0: the row is at most 64 * CPL chunks of 16 and each lane keeps its CPL chunks in registers (one HBM read).
// CPL == 0: any width; the quantize step reads the row again.
template <int DT, int CPL>
__global__ __launch_bounds__(256) void quant_rows_kernel(const void* __restrict__ w, int8_t* __restrict__ q,
                                                         float* __restrict__ scale, uint32_t rows, uint32_t cols)
{
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t row = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (row >= rows)
        return;
    const uint32_t chunks = cols / 16u;
    const uint64_t base = uint64_t(row) * chunks;
    uint4* qrow = reinterpret_cast<uint4*>(q) + base;
    float mx = 0.0f;
    if constexpr (CPL > 0) {
        Chunk<DT> r[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j)
            if (lane + 64u * j < chunks)
                r[j] = load_chunk<DT>(w, base + lane + 64u * j);
#pragma unroll
        for (int j = 0; j < CPL; ++j)
            if (lane + 64u * j < chunks)
                mx = chunk_absmax(r[j], mx);
        const float s = row_absmax(mx) / 127.0f;
        // The three cases are wave-uniform: s is the same in every lane.
        auto each = [&](auto quant) {
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const uint32_t c = lane + 64u * j;
                if (c < chunks) {
                    float v[16];
                    widen(r[j], v);
                    qrow[c] = quant(v);
                }
            }
        };
        if (s == 0.0f)
            each([](const float(&)[16]) { return uint4{0u, 0u, 0u, 0u}; });
        else if (s >= 0x1p-100f && s <= 0x1p100f)
            each([s, y = row_recip(s)](const float(&v)[16]) { return quant16<true>(v, s, y); });
        else
            each([s](const float(&v)[16]) { return quant16<false>(v, s, 0.0f); });
        if (lane == 0)
            scale[row] = s;
    } else {
        for (uint32_t c = lane; c < chunks; c += 64u)
            mx = chunk_absmax(load_chunk<DT>(w, base + c), mx);
        const float s = row_absmax(mx) / 127.0f;
        const bool fast = s >= 0x1p-100f && s <= 0x1p100f;
        const float y = fast ? row_recip(s) : 0.0f;
        for (uint32_t c = lane; c < chunks; c += 64u) {
            float v[16];
            widen(load_chunk<DT>(w, base + c), v);
            qrow[c] = s == 0.0f ? uint4{0u, 0u, 0u, 0u} : fast ? quant16<true>(v, s, y) : quant16<false>(v, s, y);
        }
        if (lane == 0)
            scale[row] = s;
    }
}

// Dynamic LDS the kernel does not use, so that at most four workgroups (16 rows) share a CU: 2-3% faster at
// 129,536 x 5120 bf16 than the occupancy the registers allow (0.334 against 0.341-0.350 ms, alternating runs); two
// workgroups were 15% slower.
constexpr size_t kQuantLdsFloor = 40 * 1024;

template <int DT>
void launch_quant(dim3 grid, hipStream_t s, const void* w, int8_t* q, float* scale, uint32_t rows, uint32_t cols)
{
    const uint32_t cpl = (cols / 16u + 63u) / 64u;
    if (cpl <= 2)
        hipLaunchKernelGGL((quant_rows_kernel<DT, 2>), grid, dim3(256), kQuantLdsFloor, s, w, q, scale, rows,
                           cols);
    else if (cpl <= 4)
        hipLaunchKernelGGL((quant_rows_kernel<DT, 4>), grid, dim3(256), kQuantLdsFloor, s, w, q, scale, rows,
                           cols);
    else if (cpl <= 8)
        hipLaunchKernelGGL((quant_rows_kernel<DT, 8>), grid, dim3(256), kQuantLdsFloor, s, w, q, scale, rows,
                           cols);
    else if (cpl <= 14) // fc2's input rows (13,824 or 14,336 bf16) in registers: one HBM read instead of two
        hipLaunchKernelGGL((quant_rows_kernel<DT, 14>), grid, dim3(256), kQuantLdsFloor, s, w, q, scale, rows,
                           cols);
    else
        hipLaunchKernelGGL((quant_rows_kernel<DT, 0>), grid, dim3(256), kQuantLdsFloor, s, w, q, scale, rows,
                           cols);
}

} // namespace mh3

extern "C" int mh3_quant_rows_i8(const MH3QuantArgs* a, const void* w, int8_t* q, float* scale, mh3_stream_t stream)
{
    using namespace mh3;
    if (!a)
        return MH3_ERR_POINTER;
    if (a->dtype != MH3_F32 && a->dtype != MH3_BF16)
        return MH3_ERR_PARAM;
    if (a->cols == 0 || a->cols % 16 != 0)
        return MH3_ERR_SHAPE;
    if (a->rows == 0)
        return MH3_OK;
    if (a->rows >= (1u << 31))
        return MH3_ERR_SHAPE;
    if (!w || !q || !scale)
        return MH3_ERR_POINTER;
    if (!host::aligned16(w) || !host::aligned16(q))
        return MH3_ERR_ALIGN;
    // The outputs may not overlap w (other workgroups still read it) or each other.
    const uint64_t w_bytes = uint64_t(a->rows) * a->cols * (a->dtype == MH3_BF16 ? 2u : 4u);
    const uint64_t q_bytes = uint64_t(a->rows) * a->cols, s_bytes = uint64_t(a->rows) * 4u;
    if (host::overlaps(q, q_bytes, w, w_bytes) || host::overlaps(scale, s_bytes, w, w_bytes) ||
        host::overlaps(q, q_bytes, scale, s_bytes))
        return MH3_ERR_PARAM;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid((a->rows + 3u) / 4u);
    if (a->dtype == MH3_BF16)
        launch_quant<MH3_BF16>(grid, s, w, q, scale, a->rows, a->cols);
    else
        launch_quant<MH3_F32>(grid, s, w, q, scale, a->rows, a->cols);
    return host::check_launch();
}
