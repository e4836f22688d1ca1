// The `--sparse` block-sparse attention selector: cube_pool, cube_scores, cube_topk and the fused cube_select.
// Reference: H3::Cubes and the mako-common kernels cube_pool / cube_scores / cube_topk, described in
// docs/architecture.md:118-133, README.md:81-87 and docs/performance.md:162-181.
//
// Design (gfx950):
// - cube_pool: one wavefront per (head, cube) pools q and k together. The wave's four 16-lane quarters take the cube's
//   four x positions, so each load instruction reads four adjacent rows (1 KiB contiguous per head in the grid
//   layout); all 32 loads of a lane are in flight at once. Lane sums in float, then a 2-step butterfly.
// - scores: v_mfma_f32_16x16x4_f32 on 16 x 16 blocks; the 128-long contraction is split over the MFMA's 4 k-lanes
//   as 4 runs of 32 consecutive dimensions, so every lane's q and k operands are 128 contiguous bytes.
// - top-k: one wavefront per (head, query cube) holds the row's scores as order-preserving 32-bit keys in VGPRs,
//   finds the k-th largest key by a wave-uniform binary search over the key range (ballot + popcount counts), then
//   emits the selection in ascending cube order with a ballot prefix sum; equal keys are taken lowest index first.
// - cube_select keeps a 16 x C score tile in LDS between the two phases, so the scores never reach HBM.
#include "mh3_common.hpp"

namespace mh3 {

typedef float floatx4 __attribute__((ext_vector_type(4)));

struct CubeGeo {
    uint32_t gt, gh, gw;   // video grid
    uint32_t cth, ch, cw;  // cubes per axis
    uint32_t cubes, plane; // cth * ch * cw, ch * cw
    uint32_t heads, layout;
    uint64_t row0, head_stride, row_stride;
};

__global__ __launch_bounds__(256) void cube_pool_kernel(CubeGeo g, const uint16_t* __restrict__ q,
                                                        const uint16_t* __restrict__ k, float* __restrict__ qc,
                                                        float* __restrict__ kc, int32_t* __restrict__ counts)
{
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t item = blockIdx.x * 4u + wave;
    if (item >= g.heads * g.cubes)
        return;
    const uint32_t h = item / g.cubes, c = item - h * g.cubes;
    const uint32_t ct = c / g.plane, rem = c - ct * g.plane, cy = rem / g.cw, cx = rem - cy * g.cw;
    const uint32_t dx = lane >> 4, part = lane & 15u; // x slot of the cube; 8 of the 128 dimensions
    const uint32_t x = cx * 4u + dx;
    const uint16_t* qh = q + h * g.head_stride + part * 8u;
    const uint16_t* kh = k + h * g.head_stride + part * 8u;
    uint4 qv[16], kv[16];
#pragma unroll
    for (int s = 0; s < 16; ++s) {
        const uint32_t dt = uint32_t(s) >> 2, dy = uint32_t(s) & 3u;
        const uint32_t t = ct * 4u + dt, y = cy * 4u + dy;
        const bool ok = x < g.gw && t < g.gt && y < g.gh;
        const uint64_t row = g.layout == MH3_CUBES_GATHERED
                                 ? g.row0 + uint64_t(c) * 64u + uint32_t(s) * 4u + dx
                                 : g.row0 + (uint64_t(t) * g.gh + y) * g.gw + x;
        if (ok) {
            qv[s] = ld_stream(reinterpret_cast<const uint4*>(qh + row * g.row_stride));
            kv[s] = ld_stream(reinterpret_cast<const uint4*>(kh + row * g.row_stride));
        } else {
            qv[s] = uint4{0u, 0u, 0u, 0u};
            kv[s] = uint4{0u, 0u, 0u, 0u};
        }
    }
    float aq[8], ak[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
        aq[e] = ak[e] = 0.0f;
#pragma unroll
    for (int s = 0; s < 16; ++s) {
        const uint32_t qw[4] = {qv[s].x, qv[s].y, qv[s].z, qv[s].w};
        const uint32_t kw[4] = {kv[s].x, kv[s].y, kv[s].z, kv[s].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            aq[2 * e] += bf16_lo(qw[e]);
            aq[2 * e + 1] += bf16_hi(qw[e]);
            ak[2 * e] += bf16_lo(kw[e]);
            ak[2 * e + 1] += bf16_hi(kw[e]);
        }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        aq[e] += __shfl_xor(aq[e], 16, 64);
        aq[e] += __shfl_xor(aq[e], 32, 64);
        ak[e] += __shfl_xor(ak[e], 16, 64);
        ak[e] += __shfl_xor(ak[e], 32, 64);
    }
    const uint32_t nt = min(4u, g.gt - ct * 4u), ny = min(4u, g.gh - cy * 4u), nx = min(4u, g.gw - cx * 4u);
    const float n = float(nt * ny * nx);
    if (dx == 0) {
        float4* oq = reinterpret_cast<float4*>(qc + (uint64_t(h) * g.cubes + c) * 128u + part * 8u);
        float4* ok = reinterpret_cast<float4*>(kc + (uint64_t(h) * g.cubes + c) * 128u + part * 8u);
        oq[0] = float4{aq[0] / n, aq[1] / n, aq[2] / n, aq[3] / n};
        oq[1] = float4{aq[4] / n, aq[5] / n, aq[6] / n, aq[7] / n};
        ok[0] = float4{ak[0] / n, ak[1] / n, ak[2] / n, ak[3] / n};
        ok[1] = float4{ak[4] / n, ak[5] / n, ak[6] / n, ak[7] / n};
    }
    if (counts && h == 0 && lane == 0)
        counts[c] = int32_t(nt * ny * nx);
}

// The 32 contraction operands of lane l for a 16-row block starting at r0: row r0 + l % 16 (clamped to the last row),
// dimensions [32 (l / 16), 32 (l / 16) + 32).
__device__ __forceinline__ void load_operand(const float* __restrict__ base, uint32_t r0, uint32_t rows, float (&v)[32])
{
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t r = r0 + (lane & 15u);
    r = r < rows ? r : rows - 1u;
    const float4* p = reinterpret_cast<const float4*>(base + uint64_t(r) * 128u + (lane >> 4) * 32u);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 t = p[i];
        v[4 * i] = t.x, v[4 * i + 1] = t.y, v[4 * i + 2] = t.z, v[4 * i + 3] = t.w;
    }
}

// acc[v] = q[i0 + 4 (l / 16) + v] . k[j0 + l % 16] over the 128 dimensions (v_mfma_f32_16x16x4_f32 layout).
__device__ __forceinline__ floatx4 score_block(const float (&qa)[32], const float (&kb)[32])
{
    floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 32; ++s)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[s], kb[s], acc, 0, 0, 0);
    return acc;
}

constexpr float kScoreScale = 0.08838834764831845f; // 1 / sqrt(128)

// Scores of query block [i0, i0 + 16) of head h against every key cube; the wave takes key blocks wave, wave + waves...
// Writes s[r][j] for r < 16, j < cubes into `dst` with row stride `ld` (rows past the last query cube skipped).
__device__ __forceinline__ void score_rows(const CubeGeo& g, const float* __restrict__ qh, const float* __restrict__ kh,
                                           uint32_t i0, float* dst, uint64_t ld, uint32_t wave, uint32_t waves)
{
    const uint32_t lane = threadIdx.x & 63u;
    float qa[32];
    load_operand(qh, i0, g.cubes, qa);
    const uint32_t kblocks = (g.cubes + 15u) / 16u;
    uint32_t kb_i = wave;
    if (kb_i >= kblocks)
        return;
    float kb[32];
    load_operand(kh, kb_i * 16u, g.cubes, kb);
    while (true) {
        const uint32_t next = kb_i + waves;
        float kn[32];
        if (next < kblocks)
            load_operand(kh, next * 16u, g.cubes, kn);
        const floatx4 acc = score_block(qa, kb);
        const uint32_t j = kb_i * 16u + (lane & 15u);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint32_t r = (lane >> 4) * 4u + uint32_t(v);
            if (j < g.cubes && i0 + r < g.cubes)
                dst[r * ld + j] = acc[v] * kScoreScale;
        }
        if (next >= kblocks)
            break;
        kb_i = next;
#pragma unroll
        for (int i = 0; i < 32; ++i)
            kb[i] = kn[i];
    }
}

__global__ __launch_bounds__(256) void cube_scores_kernel(CubeGeo g, const float* __restrict__ qc,
                                                          const float* __restrict__ kc, float* __restrict__ s)
{
    const uint32_t h = blockIdx.y, i0 = blockIdx.x * 16u;
    const uint64_t plane = uint64_t(g.cubes) * 128u;
    score_rows(g, qc + h * plane, kc + h * plane, i0, s + (uint64_t(h) * g.cubes + i0) * g.cubes, g.cubes,
               threadIdx.x >> 6, blockDim.x >> 6);
}

// Order-preserving key of a float score (larger score, larger key); -0 ranks as +0; key 0 is below every score.
__device__ __forceinline__ uint32_t score_key(float f)
{
    uint32_t u = __float_as_uint(f);
    u = u == 0x80000000u ? 0u : u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Top-k plus local cubes of one (head, query cube i) row of `cubes` scores, by one wavefront.
template <int KPL>
__device__ __forceinline__ void topk_row(const float* srow, const CubeGeo& g, uint32_t i, uint32_t k, uint32_t local,
                                         int32_t* __restrict__ out, uint32_t out_stride, int32_t* __restrict__ cnt)
{
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t C = g.cubes;
    uint32_t key[KPL];
    uint32_t mn = 0xffffffffu, mx = 0u;
#pragma unroll
    for (int m = 0; m < KPL; ++m) {
        const uint32_t j = lane + 64u * m;
        key[m] = j < C ? score_key(srow[j]) : 0u;
        if (j < C) {
            mn = key[m] < mn ? key[m] : mn;
            mx = key[m] > mx ? key[m] : mx;
        }
    }
    uint32_t lo = wave_min_u32(mn), hi = wave_max_u32(mx);
    // The k-th largest key: the largest t with #{key >= t} >= k. Invariant: #{key >= lo} >= k.
    while (lo < hi) {
        const uint32_t d = hi - lo;
        const uint32_t mid = lo + (d >> 1) + (d & 1u);
        uint32_t n = 0;
#pragma unroll
        for (int m = 0; m < KPL; ++m)
            n += __popcll(__ballot(key[m] >= mid));
        if (n >= k)
            lo = mid;
        else
            hi = mid - 1u;
    }
    const uint32_t t = lo;
    uint32_t above = 0;
#pragma unroll
    for (int m = 0; m < KPL; ++m)
        above += __popcll(__ballot(key[m] > t));
    const uint32_t need_eq = k - above; // >= 1
    const uint32_t ct = i / g.plane;
    const bool prev = local == 3u && ct > 0u, next = local == 3u && ct + 1u < g.cth;
    const uint64_t below = lanes_below(int(lane));
    uint32_t pos = 0, eq_seen = 0;
#pragma unroll
    for (int m = 0; m < KPL; ++m) {
        const uint32_t j = lane + 64u * m;
        const bool eq = key[m] == t;
        const uint64_t eqm = __ballot(eq);
        const uint32_t rank = eq_seen + uint32_t(__popcll(eqm & below));
        const bool loc = j < C && ((local >= 1u && j == i) || (prev && j == i - g.plane) || (next && j == i + g.plane));
        const bool sel = key[m] > t || (eq && rank < need_eq) || loc;
        const uint64_t selm = __ballot(sel);
        if (sel)
            out[pos + uint32_t(__popcll(selm & below))] = int32_t(j);
        pos += uint32_t(__popcll(selm));
        eq_seen += uint32_t(__popcll(eqm));
    }
    for (uint32_t j = pos + lane; j < out_stride; j += 64u)
        out[j] = -1;
    if (lane == 0)
        *cnt = int32_t(pos);
}

template <int KPL>
__global__ __launch_bounds__(256) void cube_topk_kernel(CubeGeo g, const float* __restrict__ s, uint32_t k,
                                                        uint32_t local, uint32_t out_stride, int32_t* __restrict__ idx,
                                                        int32_t* __restrict__ cnt)
{
    const uint32_t item = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (item >= g.heads * g.cubes)
        return;
    const uint32_t i = item % g.cubes;
    topk_row<KPL>(s + uint64_t(item) * g.cubes, g, i, k, local, idx + uint64_t(item) * out_stride, out_stride,
                  cnt + item);
}

constexpr int kSelectThreads = 512;
constexpr uint32_t kSelectRows = 16;

template <int KPL>
__global__ __launch_bounds__(kSelectThreads) void cube_select_kernel(CubeGeo g, const float* __restrict__ qc,
                                                                     const float* __restrict__ kc, uint32_t k,
                                                                     uint32_t local, uint32_t out_stride,
                                                                     int32_t* __restrict__ idx,
                                                                     int32_t* __restrict__ cnt)
{
    extern __shared__ float tile[]; // [16][cubes]
    const uint32_t h = blockIdx.y, i0 = blockIdx.x * kSelectRows;
    const uint32_t wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    const uint64_t plane = uint64_t(g.cubes) * 128u;
    score_rows(g, qc + h * plane, kc + h * plane, i0, tile, g.cubes, wave, waves);
    __syncthreads();
    for (uint32_t r = wave; r < kSelectRows; r += waves) {
        const uint32_t i = i0 + r;
        if (i >= g.cubes)
            break;
        const uint64_t item = uint64_t(h) * g.cubes + i;
        topk_row<KPL>(tile + r * g.cubes, g, i, k, local, idx + item * out_stride, out_stride, cnt + item);
    }
}

} // namespace mh3

// ---- C-ABI ----------------------------------------------------------------------------------------------------------
namespace {

using namespace mh3;

int make_geo(const MH3CubeArgs* a, CubeGeo& g)
{
    if (!a)
        return MH3_ERR_POINTER;
    if (a->layout != MH3_CUBES_GRID && a->layout != MH3_CUBES_GATHERED)
        return MH3_ERR_PARAM;
    if (a->heads == 0 || a->grid_t == 0 || a->grid_h == 0 || a->grid_w == 0 || a->head_dim == 0)
        return MH3_ERR_SHAPE;
    if (a->head_dim != 128)
        return MH3_ERR_UNSUPPORTED;
    g.gt = a->grid_t, g.gh = a->grid_h, g.gw = a->grid_w;
    g.cth = (g.gt + 3u) / 4u, g.ch = (g.gh + 3u) / 4u, g.cw = (g.gw + 3u) / 4u;
    const uint64_t cubes = uint64_t(g.cth) * g.ch * g.cw;
    if (cubes * a->heads >= (uint64_t(1) << 31))
        return MH3_ERR_SHAPE;
    g.cubes = uint32_t(cubes), g.plane = g.ch * g.cw;
    g.heads = a->heads, g.layout = a->layout;
    g.row0 = a->row0, g.head_stride = a->head_stride, g.row_stride = a->row_stride;
    return MH3_OK;
}

int check_topk_args(const MH3CubeArgs* a, const CubeGeo& g)
{
    if (a->k == 0 || a->k > g.cubes)
        return MH3_ERR_PARAM;
    if (a->local != 0 && a->local != 1 && a->local != 3)
        return MH3_ERR_PARAM;
    if (a->out_stride < a->k + a->local)
        return MH3_ERR_SHAPE;
    if (g.cubes > 4096)
        return MH3_ERR_UNSUPPORTED;
    return MH3_OK;
}

int set_lds_limit(const void* kernel, size_t bytes)
{
    return hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, int(bytes)) == hipSuccess
               ? MH3_OK
               : MH3_ERR_HIP;
}

} // namespace

extern "C" {

int mh3_cube_pool(const MH3CubeArgs* args, const uint16_t* q, const uint16_t* k, float* qc, float* kc,
                  int32_t* counts, mh3_stream_t stream)
{
    CubeGeo g;
    int rc = make_geo(args, g);
    if (rc != MH3_OK)
        return rc;
    if (!q || !k || !qc || !kc)
        return MH3_ERR_POINTER;
    if (args->row_stride % 8 != 0 || args->head_stride % 8 != 0 || !host::aligned16(q) || !host::aligned16(k) ||
        !host::aligned16(qc) || !host::aligned16(kc))
        return MH3_ERR_ALIGN;
    const uint32_t items = g.heads * g.cubes;
    hipLaunchKernelGGL(cube_pool_kernel, dim3((items + 3u) / 4u), dim3(256), 0, static_cast<hipStream_t>(stream), g,
                       q, k, qc, kc, counts);
    return host::check_launch();
}

int mh3_cube_scores(const MH3CubeArgs* args, const float* qc, const float* kc, float* s, mh3_stream_t stream)
{
    CubeGeo g;
    int rc = make_geo(args, g);
    if (rc != MH3_OK)
        return rc;
    if (!qc || !kc || !s)
        return MH3_ERR_POINTER;
    if (!host::aligned16(qc) || !host::aligned16(kc))
        return MH3_ERR_ALIGN;
    hipLaunchKernelGGL(cube_scores_kernel, dim3((g.cubes + 15u) / 16u, g.heads), dim3(256), 0,
                       static_cast<hipStream_t>(stream), g, qc, kc, s);
    return host::check_launch();
}

int mh3_cube_topk(const MH3CubeArgs* args, const float* s, int32_t* idx, int32_t* cnt, mh3_stream_t stream)
{
    CubeGeo g;
    int rc = make_geo(args, g);
    if (rc != MH3_OK)
        return rc;
    if ((rc = check_topk_args(args, g)) != MH3_OK)
        return rc;
    if (!s || !idx || !cnt)
        return MH3_ERR_POINTER;
    const uint32_t items = g.heads * g.cubes;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (g.cubes <= 2048)
        hipLaunchKernelGGL(cube_topk_kernel<32>, dim3((items + 3u) / 4u), dim3(256), 0, st, g, s, args->k,
                           args->local, args->out_stride, idx, cnt);
    else
        hipLaunchKernelGGL(cube_topk_kernel<64>, dim3((items + 3u) / 4u), dim3(256), 0, st, g, s, args->k,
                           args->local, args->out_stride, idx, cnt);
    return host::check_launch();
}

int mh3_cube_select(const MH3CubeArgs* args, const float* qc, const float* kc, int32_t* idx, int32_t* cnt,
                    mh3_stream_t stream)
{
    CubeGeo g;
    int rc = make_geo(args, g);
    if (rc != MH3_OK)
        return rc;
    if ((rc = check_topk_args(args, g)) != MH3_OK)
        return rc;
    if (!qc || !kc || !idx || !cnt)
        return MH3_ERR_POINTER;
    if (!host::aligned16(qc) || !host::aligned16(kc))
        return MH3_ERR_ALIGN;
    const size_t lds = size_t(kSelectRows) * g.cubes * sizeof(float);
    if (lds > 160 * 1024)
        return MH3_ERR_UNSUPPORTED; // use cube_scores + cube_topk
    const dim3 grid((g.cubes + kSelectRows - 1) / kSelectRows, g.heads);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (g.cubes <= 2048) {
        if ((rc = set_lds_limit(reinterpret_cast<const void*>(&cube_select_kernel<32>), lds)) != MH3_OK)
            return rc;
        hipLaunchKernelGGL(cube_select_kernel<32>, grid, dim3(kSelectThreads), lds, st, g, qc, kc, args->k,
                           args->local, args->out_stride, idx, cnt);
    } else {
        if ((rc = set_lds_limit(reinterpret_cast<const void*>(&cube_select_kernel<64>), lds)) != MH3_OK)
            return rc;
        hipLaunchKernelGGL(cube_select_kernel<64>, grid, dim3(kSelectThreads), lds, st, g, qc, kc, args->k,
                           args->local, args->out_stride, idx, cnt);
    }
    return host::check_launch();
}

} // extern "C"
