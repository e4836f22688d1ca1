// `quant_rows_i8`, weight side: each [out][in] weight row to symmetric int8 with one float scale, at load time.
// Reference: the mako-common kernel of this name, described in docs/performance.md:122-126 and
// docs/architecture.md:54-56 ("int8 rows with a float scale each (symmetric, the row's maximum at 127)").
// One wavefront per row: a max-|w| pass, then a quantize pass (the row is re-read from L2).
#include "mh3_common.hpp"

namespace mh3 {

// 16 row elements from `p` (bf16: two 16-byte vectors; float: four).
template <int DT>
__device__ __forceinline__ void load16(const void* p, uint64_t chunk, float (&v)[16])
{
    if constexpr (DT == MH3_BF16) {
        const uint4* q = static_cast<const uint4*>(p) + chunk * 2u;
        const uint4 a = q[0], b = q[1];
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v[2 * i] = bf16_lo(w[i]);
            v[2 * i + 1] = bf16_hi(w[i]);
        }
    } else {
        const float4* q = static_cast<const float4*>(p) + chunk * 4u;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 t = q[i];
            v[4 * i] = t.x, v[4 * i + 1] = t.y, v[4 * i + 2] = t.z, v[4 * i + 3] = t.w;
        }
    }
}

template <int DT>
__global__ __launch_bounds__(256) void quant_rows_kernel(const void* __restrict__ w, int8_t* __restrict__ q,
                                                         float* __restrict__ scale, uint32_t rows, uint32_t cols)
{
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t row = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (row >= rows)
        return;
    const uint32_t chunks = cols / 16u;
    const uint64_t base = uint64_t(row) * chunks;
    float mx = 0.0f;
    for (uint32_t c = lane; c < chunks; c += 64u) {
        float v[16];
        load16<DT>(w, base + c, v);
#pragma unroll
        for (int i = 0; i < 16; ++i)
            mx = fmaxf(mx, fabsf(v[i]));
    }
    mx = wave_max(mx);
    const float s = mx / 127.0f;
    for (uint32_t c = lane; c < chunks; c += 64u) {
        float v[16];
        load16<DT>(w, base + c, v);
        uint32_t packed[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float r = s == 0.0f ? 0.0f : rintf(v[i] / s);
            r = fminf(fmaxf(r, -127.0f), 127.0f);
            packed[i >> 2] |= (uint32_t(int32_t(r)) & 0xffu) << (8 * (i & 3));
        }
        reinterpret_cast<uint4*>(q)[base + c] = uint4{packed[0], packed[1], packed[2], packed[3]};
    }
    if (lane == 0)
        scale[row] = s;
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
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid((a->rows + 3u) / 4u);
    if (a->dtype == MH3_BF16)
        hipLaunchKernelGGL(quant_rows_kernel<MH3_BF16>, grid, dim3(256), 0, s, w, q, scale, a->rows, a->cols);
    else
        hipLaunchKernelGGL(quant_rows_kernel<MH3_F32>, grid, dim3(256), 0, s, w, q, scale, a->rows, a->cols);
    return host::check_launch();
}
