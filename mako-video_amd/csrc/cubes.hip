// The `--sparse` block-sparse attention selector: cube_pool, cube_scores, cube_topk and the fused cube_select.
// Reference: H3::Cubes and the mako-common kernels cube_pool / cube_scores / cube_topk, described in
// docs/architecture.md:118-133, README.md:81-87 and docs/performance.md:162-181.
//
// Design (gfx950):
// - cube_pool: one wavefront per (head, cube) pools q and k together. Lane 16 x + p takes dimensions 8 p ... 8 p + 7
//   of the cube's x position x, so each load instruction reads four adjacent rows (1 KiB contiguous per head in the
//   grid layout) and each quad of lanes one aligned 64-byte piece of a row; all 32 loads of a lane are in flight at
//   once. Lane sums in float, then two lane exchanges across the 16-lane rows.
// - scores: float dot products on 16 x 16 blocks from the four bf16 MFMA products of operands split into bf16 high
//   and low parts (v_mfma_f32_16x16x32_bf16): a quarter of the matrix-core clocks of v_mfma_f32_16x16x4_f32, within
//   1e-5 of the row's largest score; each operand load of the wave reads 64 contiguous bytes of each of 16 rows.
// - top-k: one wavefront per (head, query cube) holds the row's scores as floats in VGPRs, lane l owning cubes
//   32 l ... 32 l + 31. A 128-bin histogram of the scores, linear in value between the row's minimum and maximum (LDS
//   atomics, one pass), brackets the k-th largest to one bin; a bin of more than 64 scores is binned again over its
//   own range, and at most 64 candidates, one to a lane, finish the search by ballots. Rows with an infinite or NaN
//   score are ranked as order-preserving 32-bit keys by a bisection of the key range.
//   The selection is a per-lane bit mask; wave prefix sums over lanes rank the ties (lowest index first) and place
//   each lane's indices, so the output is ascending with no per-element ballots.
// - cube_select keeps a 16 x C score tile in LDS between the two phases, so the scores never reach HBM. A first pass
//   splits the key cubes into the matrix cores' bf16 operands once (a workspace the caller gives), so its scoring
//   waves only load and multiply. Its workgroups are persistent (one a CU); scoring waves and ranking waves overlap
//   one tile's ranking with the next tile's scoring.
#include "mh3_common.hpp"

#include <algorithm>
#include <type_traits>

namespace mh3 {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

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
    // x slot of the cube (one 16-lane row of the wave each) and 8 of the 128 dimensions: each load of a 16-lane row
    // reads one token's 256 bytes, so every quad of lanes fetches one aligned 64-byte piece (a quad spread over four
    // rows would be four accesses for the address unit).
    const uint32_t dx = lane >> 4, part = lane & 15u;
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
    // The cube's 4 x positions are the wave's four 16-lane rows: (x0 + x1) + (x2 + x3) by two lane exchanges.
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        aq[e] += __shfl_xor(aq[e], 16, kWave);
        aq[e] += __shfl_xor(aq[e], 32, kWave);
        ak[e] += __shfl_xor(ak[e], 16, kWave);
        ak[e] += __shfl_xor(ak[e], 32, kWave);
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

// A 16-row block's operands for the bf16 MFMA (v_mfma_f32_16x16x32_bf16, four steps of k = 32). Lane l of a step
// holds row r0 + l % 16 (clamped to the last row) at 8 k-values; over the four steps, lane l's 32 operands are
// dimensions 16 v + 4 (l / 16) + u (operand 4 v + u, step s taking operands 8 s .. 8 s + 7), the same for q and k,
// so the contraction covers the 128 dimensions once. The loads take another lane order: lane l reads row r0 + l / 4,
// dimensions 16 v + 4 (l % 4) .. + 3, so each quad of lanes fetches one aligned 64-byte piece of a row (a quad spread
// over four rows costs the address unit four accesses and held these loads to about 16 bytes a clock a CU); a lane
// exchange (ds_bpermute, lane l from lane 4 (l % 16) + l / 16) then gives each lane its operands.
struct RawRows {
    float4 t[8]; // lane l: row r0 + l / 4, dimensions 16 i + 4 (l % 4) .. + 3
};

__device__ __forceinline__ void load_raw(const float* __restrict__ base, uint32_t r0, uint32_t rows, RawRows& raw)
{
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t r = r0 + (lane >> 2);
    r = r < rows ? r : rows - 1u;
    const float* p = base + uint64_t(r) * 128u + (lane & 3u) * 4u;
#pragma unroll
    for (int i = 0; i < 8; ++i)
        raw.t[i] = *reinterpret_cast<const float4*>(p + 16 * i);
}

// Each float operand x is split into two bf16 parts, x = hi + lo + r with hi = bf16(x) and lo = bf16(x - hi), both
// rounded to nearest even (x - hi is exact in float), so |r| <= 2^-18 |x|. The split is made before the lane
// exchange, on pairs of adjacent operands, so the exchange moves 32 packed words, as many as the floats would take.
struct SplitRow {
    bf16x8_t hi[4], lo[4];
};

__device__ __forceinline__ void split_exchange(const RawRows& raw, SplitRow& o)
{
    const uint32_t lane = threadIdx.x & 63u;
    const int src = int(4u * (4u * (lane & 15u) + (lane >> 4)));
    uint32_t h[16], l[16]; // h[2 i + j]: operands 4 i + 2 j and 4 i + 2 j + 1 of the lane
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float c[4] = {raw.t[i].x, raw.t[i].y, raw.t[i].z, raw.t[i].w};
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const float a = c[2 * j], b = c[2 * j + 1];
            const uint32_t hp = pack_bf16(a, b);
            const uint32_t lp = pack_bf16(a - bf16_lo(hp), b - bf16_hi(hp));
            h[2 * i + j] = uint32_t(__builtin_amdgcn_ds_bpermute(src, int(hp)));
            l[2 * i + j] = uint32_t(__builtin_amdgcn_ds_bpermute(src, int(lp)));
        }
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        o.hi[s] = __builtin_bit_cast(bf16x8_t, uint4{h[4 * s], h[4 * s + 1], h[4 * s + 2], h[4 * s + 3]});
        o.lo[s] = __builtin_bit_cast(bf16x8_t, uint4{l[4 * s], l[4 * s + 1], l[4 * s + 2], l[4 * s + 3]});
    }
}

// acc[v] = q[i0 + 4 (l / 16) + v] . k[j0 + l % 16] from the four bf16 products of the split operands, q.k =
// qlo.klo + qlo.khi + qhi.klo + qhi.khi, accumulated in float by the MFMA, the small products first. A product of
// bf16 values is exact in float, so a term's error is the split's remainders, at most about 2^-17 |q_d k_d|: over
// 2016 x 2016 scores of N(0, 1) rows the largest error is 6.3e-6 of the row's largest score (9.2e-6 without the
// qlo.klo product, 8.7e-7 for a float contraction), and it matters to the selection only where two scores tie to
// that order. The bf16 MFMAs (k = 32) take 256 clocks a block against 1024 for the 32 v_mfma_f32_16x16x4_f32 of a
// float contraction.
__device__ __forceinline__ floatx4 score_block(const SplitRow& q, const SplitRow& k)
{
    floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 4; ++s)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(q.lo[s], k.lo[s], acc, 0, 0, 0);
#pragma unroll
    for (int s = 0; s < 4; ++s)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(q.lo[s], k.hi[s], acc, 0, 0, 0);
#pragma unroll
    for (int s = 0; s < 4; ++s)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(q.hi[s], k.lo[s], acc, 0, 0, 0);
#pragma unroll
    for (int s = 0; s < 4; ++s)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(q.hi[s], k.hi[s], acc, 0, 0, 0);
    return acc;
}

// The same four scores by float FMAs in dimension order, straight from memory. An infinite or NaN operand, or one so
// large that bf16(x) overflows, makes the split's parts infinite or NaN, and with them the block's scores: a block
// with a non-finite score (the test is wave-uniform) is scored again here. Rare, so written for few registers.
__device__ __forceinline__ floatx4 score_block_direct(const float* __restrict__ qh, const float* __restrict__ kh,
                                                      uint32_t i0, uint32_t j0, uint32_t rows)
{
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t kr = min(j0 + (lane & 15u), rows - 1u);
    floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t d = 0; d < 128u; d += 4u) {
        const float4 kv = *reinterpret_cast<const float4*>(kh + uint64_t(kr) * 128u + d);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint32_t qr = min(i0 + 4u * (lane >> 4) + uint32_t(v), rows - 1u);
            const float4 qv = *reinterpret_cast<const float4*>(qh + uint64_t(qr) * 128u + d);
            acc[v] = fmaf(qv.w, kv.w, fmaf(qv.z, kv.z, fmaf(qv.y, kv.y, fmaf(qv.x, kv.x, acc[v]))));
        }
    }
    return acc;
}

constexpr float kScoreScale = 0.08838834764831845f; // 1 / sqrt(128)

// LDS rows for the top-k: cube j of a row sits at word (j / KPL) (KPL + 4) + j % KPL, so the KPL scores of lane l
// (cubes l KPL ...) are contiguous and 16-byte reads of 16 lanes at a stride of KPL + 4 words hit distinct banks.
template <int KPL>
__device__ __forceinline__ uint32_t pad_word(uint32_t j)
{
    return (j / KPL) * (KPL + 4) + j % KPL;
}
template <int KPL>
constexpr uint32_t kPaddedRow = 64u * (KPL + 4);

// The scores of one key block, stored. A block with a non-finite score (the test is wave-uniform) is scored again by
// float FMAs (score_block_direct); where `row_flags` is given, rows left with a non-finite score are flagged there.
// Scores s[r][j] (r < 16, j < cubes) go to `dst` at r * ld + j, or at r * ld + pad_word<32>(j) when PAD (rows past
// the last query cube skipped).
template <bool PAD>
__device__ __forceinline__ void store_block(const CubeGeo& g, const float* __restrict__ qh,
                                            const float* __restrict__ kh, uint32_t i0, uint32_t b, floatx4 acc,
                                            float* dst, uint64_t ld, uint32_t* row_flags)
{
    const uint32_t lane = threadIdx.x & 63u, j = b * 16u + (lane & 15u);
    const bool finite = __builtin_isfinite(acc[0]) && __builtin_isfinite(acc[1]) && __builtin_isfinite(acc[2]) &&
                        __builtin_isfinite(acc[3]);
    if (__ballot(!finite)) {
        acc = score_block_direct(qh, kh, i0, b * 16u, g.cubes);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint32_t r = (lane >> 4) * 4u + uint32_t(v);
            if (row_flags && j < g.cubes && i0 + r < g.cubes && !__builtin_isfinite(acc[v]))
                atomicOr(row_flags + r, 1u);
        }
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const uint32_t r = (lane >> 4) * 4u + uint32_t(v);
        if (j < g.cubes && i0 + r < g.cubes)
            dst[r * ld + (PAD ? pad_word<32>(j) : j)] = acc[v] * kScoreScale;
    }
}

// Scores of query block [i0, i0 + 16) of a head against every key cube, from qc and kc as they lie; the wave takes
// key blocks wave, wave + waves, ..., each split after its load, the next one's loads in flight while a block's MFMAs
// run (one block ahead: 0.467-0.469 ms at 768p against 0.478 ms for two). Rows go to `dst` at r * ld + j.
__device__ __forceinline__ void score_rows(const CubeGeo& g, const float* __restrict__ qh, const float* __restrict__ kh,
                                           uint32_t i0, float* dst, uint64_t ld, uint32_t wave, uint32_t waves)
{
    const uint32_t kblocks = (g.cubes + 15u) / 16u;
    SplitRow qs;
    {
        RawRows qraw;
        load_raw(qh, i0, g.cubes, qraw);
        split_exchange(qraw, qs);
    }
    RawRows kr;
    if (wave < kblocks)
        load_raw(kh, wave * 16u, g.cubes, kr);
    for (uint32_t b = wave; b < kblocks; b += waves) {
        SplitRow ks;
        split_exchange(kr, ks);
        if (b + waves < kblocks)
            load_raw(kh, (b + waves) * 16u, g.cubes, kr);
        store_block<false>(g, qh, kh, i0, b, score_block(qs, ks), dst, ld, nullptr);
    }
}

// The key operands split once for cube_select: block b (16 key cubes) of head h is 8 KiB at ks + (h kblocks + b) 512
// (16-byte units): unit (2 s + part) 64 + l holds lane l's operands of MFMA step s, part 0 the bf16 high parts and
// part 1 the low parts, exactly as split_exchange leaves them in the registers. A scoring wave then loads a block with
// eight 1 KiB contiguous reads and no VALU work, and the scores are the same bits as cube_scores'.
__global__ __launch_bounds__(256) void cube_split_kernel(CubeGeo g, const float* __restrict__ kc,
                                                         uint4* __restrict__ ks)
{
    const uint32_t kblocks = (g.cubes + 15u) / 16u;
    const uint32_t item = blockIdx.x * 4u + (threadIdx.x >> 6); // (head, key block), wave-uniform
    if (item >= g.heads * kblocks)
        return;
    const uint32_t h = item / kblocks, b = item - h * kblocks;
    RawRows raw;
    load_raw(kc + uint64_t(h) * g.cubes * 128u, b * 16u, g.cubes, raw);
    SplitRow s;
    split_exchange(raw, s);
    uint4* dst = ks + uint64_t(item) * 512u + (threadIdx.x & 63u);
#pragma unroll
    for (int st = 0; st < 4; ++st) {
        dst[(2 * st) * 64] = __builtin_bit_cast(uint4, s.hi[st]);
        dst[(2 * st + 1) * 64] = __builtin_bit_cast(uint4, s.lo[st]);
    }
}

__device__ __forceinline__ void load_split(const uint4* __restrict__ base, uint32_t b, SplitRow& o)
{
    const uint4* p = base + uint64_t(b) * 512u + (threadIdx.x & 63u);
#pragma unroll
    for (int st = 0; st < 4; ++st) {
        o.hi[st] = __builtin_bit_cast(bf16x8_t, p[(2 * st) * 64]);
        o.lo[st] = __builtin_bit_cast(bf16x8_t, p[(2 * st + 1) * 64]);
    }
}

// cube_select's scoring: as score_rows, with the key blocks' operands from cube_split_kernel (`ksh`: the head's
// blocks) and the scores into the padded LDS tile, rows with a non-finite score flagged in `row_flags`. One block in
// flight a wave: 0.525-0.532 ms at 768p against 0.535-0.551 ms for two (registers spilled) and 1.14 ms for three.
__device__ __forceinline__ void score_rows_split(const CubeGeo& g, const float* __restrict__ qh,
                                                 const float* __restrict__ kh, const uint4* __restrict__ ksh,
                                                 uint32_t i0, float* dst, uint64_t ld, uint32_t wave, uint32_t waves,
                                                 uint32_t* row_flags)
{
    const uint32_t kblocks = (g.cubes + 15u) / 16u;
    SplitRow qs;
    {
        RawRows qraw;
        load_raw(qh, i0, g.cubes, qraw);
        split_exchange(qraw, qs);
    }
    SplitRow kr;
    if (wave < kblocks)
        load_split(ksh, wave, kr);
    for (uint32_t b = wave; b < kblocks; b += waves) {
        const floatx4 acc = score_block(qs, kr);
        if (b + waves < kblocks)
            load_split(ksh, b + waves, kr);
        store_block<true>(g, qh, kh, i0, b, acc, dst, ld, row_flags);
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

// Keys >= t over the wave: per-lane counts in four independent chains, then one DPP wave sum.
template <int KPL>
__device__ __forceinline__ uint32_t count_ge(const uint32_t (&key)[KPL], uint32_t t)
{
    uint32_t c[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int m = 0; m < KPL; ++m)
        c[m & 3] += key[m] >= t ? 1u : 0u;
    return wave_sum_u32((c[0] + c[1]) + (c[2] + c[3]));
}

// Float value of a key (the inverse of score_key; key 0x80000000 is +0).
__device__ __forceinline__ float key_value(uint32_t key)
{
    return __uint_as_float((key & 0x80000000u) ? (key & 0x7fffffffu) : ~key);
}

constexpr uint32_t kHistBins = 128; // lanes 0 .. 31 hold four bins each

// Per-lane bit masks over a lane's KPL cubes.
template <int KPL>
using LaneMask = typename std::conditional<KPL == 32, uint32_t, uint64_t>::type;

// The selection from the threshold's masks, bit m for cube j0 + m of the lane: gt (scores above the k-th largest t)
// and eq (scores equal to t). The first k - #gt ties in cube order join gt (a prefix sum of per-lane tie counts ranks
// them; when there are exactly that many ties they all join), then the local cubes; a prefix sum of the per-lane
// counts gives each lane its output position, so the indices come out ascending.
template <int KPL>
__device__ __forceinline__ void select_emit(LaneMask<KPL> gt, LaneMask<KPL> eq, const CubeGeo& g, uint32_t i,
                                            uint32_t k, uint32_t local, int32_t* __restrict__ out, uint32_t out_stride,
                                            int32_t* __restrict__ cnt)
{
    typedef LaneMask<KPL> Mask;
    const uint32_t lane = threadIdx.x & 63u, j0 = lane * KPL;
    const uint32_t n_gt = uint32_t(__popcll(uint64_t(gt))), n_eq = uint32_t(__popcll(uint64_t(eq)));
    const uint32_t need_eq = k - wave_sum_u32(n_gt); // >= 1
    const uint32_t eq_before = wave_excl_scan_u32(n_eq);
    const uint32_t all_eq = uint32_t(__builtin_amdgcn_readlane(int(eq_before + n_eq), 63));
    Mask sel = gt;
    if (all_eq == need_eq) {
        sel |= eq;
    } else {
        uint32_t take = need_eq > eq_before ? min(need_eq - eq_before, n_eq) : 0u;
#pragma unroll
        for (int m = 0; m < KPL; ++m) {
            const bool tie = (eq >> m) & 1u;
            sel |= tie && take > 0u ? Mask(1) << m : Mask(0);
            take -= tie && take > 0u ? 1u : 0u;
        }
    }
    const uint32_t ct = i / g.plane;
    const uint32_t loc[3] = {local >= 1u ? i : 0xffffffffu, local == 3u && ct > 0u ? i - g.plane : 0xffffffffu,
                             local == 3u && ct + 1u < g.cth ? i + g.plane : 0xffffffffu};
#pragma unroll
    for (int e = 0; e < 3; ++e)
        sel |= loc[e] / KPL == lane ? Mask(1) << (loc[e] % KPL) : Mask(0);
    const uint32_t n_sel = uint32_t(__popcll(uint64_t(sel)));
    const uint32_t pos = wave_excl_scan_u32(n_sel);
    const uint32_t total = uint32_t(__builtin_amdgcn_readlane(int(pos + n_sel), 63));
    // Store r writes each lane's r-th selected index: as many store instructions as the fullest lane has indices,
    // not one per key slot.
    const uint32_t most = wave_max_u32(n_sel);
    uint64_t rest = uint64_t(sel);
    for (uint32_t r = 0; r < most; ++r) {
        if (rest) {
            out[pos + r] = int32_t(j0 + uint32_t(__builtin_ctzll(rest)));
            rest &= rest - 1u;
        }
    }
    for (uint32_t j = total + lane; j < out_stride; j += 64u)
        out[j] = -1;
    if (lane == 0)
        *cnt = int32_t(total);
}

// A row's scores as lane l holds them: cubes j = l KPL + m (m < KPL) as floats; slots with j >= cubes hold NaN.
template <int KPL>
struct RowVals {
    float f[KPL];
};

// Lane l's KPL scores of a row in the padded layout of pad_word.
template <int KPL>
__device__ __forceinline__ void load_vals(const float* row, RowVals<KPL>& r)
{
    const uint32_t lane = threadIdx.x & 63u;
    const float4* mine = reinterpret_cast<const float4*>(row + lane * (KPL + 4));
#pragma unroll
    for (int v = 0; v < KPL / 4; ++v) {
        const float4 x = mine[v];
        r.f[4 * v] = x.x, r.f[4 * v + 1] = x.y, r.f[4 * v + 2] = x.z, r.f[4 * v + 3] = x.w;
    }
}

constexpr int kMaxLevels = 32; // histogram levels of the float search

// Top-k plus local cubes of one (head, query cube i) row of `cubes` scores, by one wavefront. Lane l holds cubes
// j = l KPL + m (m < KPL) as floats (NaN past the last cube); `cand` (64 words) and `hist` (kHistBins words) are LDS
// private to the wave. The k-th largest score t is the largest t with #{score >= t} >= k. When every score is finite
// (`finite`, wave-uniform) it is found on the floats:
// - A 128-bin histogram, linear in value between the range's lowest and highest score (LDS atomics), brackets t to
//   one bin: bin(v) = min(127, (v - lo) * 128 / (hi - lo)) is non-decreasing in v (rounded subtraction,
//   multiplication, minimum and truncation all are), so every score of a higher bin exceeds every score of a lower
//   one. At the first level the NaN slots fall in the top bin and are taken off its count.
// - While t's bin holds more than 64 scores, the range narrows to that bin's scores and a new histogram spans them
//   (a range's lowest and highest scores fall in its bottom and top bins, so each level holds fewer scores); a range
//   of equal scores is t itself.
// - The bin's scores are compacted one to a lane and t is selected among them by ballots: the pivot is the lowest
//   remaining lane's score, and the scores above it, or those below it, remain, so the set shrinks every round.
// Rows with an infinite or NaN score, and ranges too narrow to scale, rank order-preserving keys (score_key) by a
// bisection of the key range. Float order is the key order on finite scores (-0 and +0 equal in both).
template <int KPL>
__device__ __forceinline__ void topk_vals(RowVals<KPL>& rv, bool finite, const CubeGeo& g, uint32_t i, uint32_t k,
                                          uint32_t local, int32_t* __restrict__ out, uint32_t out_stride,
                                          int32_t* __restrict__ cnt, uint32_t* cand, uint32_t* hist)
{
    typedef LaneMask<KPL> Mask;
    const uint32_t lane = threadIdx.x & 63u, C = g.cubes;
    float(&f)[KPL] = rv.f;
    bool found = false;
    float t = 0.0f;
    if (finite) {
        float mn = __builtin_inff(), mx = -__builtin_inff();
#pragma unroll
        for (int m = 0; m < KPL; ++m) {
            mn = fminf(mn, f[m]); // NaN slots are ignored
            mx = fmaxf(mx, f[m]);
        }
        float lo = key_value(wave_min_u32(score_key(mn))), hi = key_value(wave_max_u32(score_key(mx)));
        uint32_t bins[KPL / 4] = {};        // byte m % 4 of bins[m / 4]: score m's bin at the current level
        uint32_t b = 0u, n_hi = 0u, nb = C; // t's bin; scores above the range [lo, hi]; scores in it
        // One level: the histogram of the range's scores, then t's bin b, the scores above it and those in it. A score
        // is in the range when lo <= f <= hi (never a NaN slot).
        // At the first level only lanes holding a cube count (all of a lane's slots, its NaN slots in the top bin,
        // taken off afterwards): lanes of NaN slots alone would all add into the top bin at once, and conflicting LDS
        // atomics serialize (a 400-cube row: 51 of 64 lanes).
        const bool holds = lane * KPL < C;
        auto level = [&](auto first, float inv) {
            constexpr bool kFirst = decltype(first)::value;
#pragma unroll
            for (uint32_t e = lane; e < kHistBins; e += 64u)
                hist[e] = 0u;
            if (!kFirst || holds) {
#pragma unroll
                for (int m = 0; m < KPL; ++m) {
                    // NaN slots give the top bin; scores below the range (deeper levels, not counted) bin 0
                    const float x = fminf((f[m] - lo) * inv, float(kHistBins - 1u));
                    const uint32_t b_m = uint32_t(kFirst ? x : fmaxf(x, 0.0f));
                    if (kFirst || (f[m] >= lo && f[m] <= hi))
                        atomicAdd(hist + b_m, 1u);
                    bins[m / 4] = (m % 4 == 0 ? 0u : bins[m / 4]) | (b_m << (8 * (m % 4)));
                }
            }
            __builtin_amdgcn_s_waitcnt(0xC07F); // the wave's own LDS atomics are visible to its reads after lgkmcnt(0)
            const uint4 h4 =
                lane < kHistBins / 4u ? reinterpret_cast<const uint4*>(hist)[lane] : uint4{0u, 0u, 0u, 0u};
            uint32_t hs[4] = {h4.x, h4.y, h4.z, h4.w};
            if (kFirst && lane == kHistBins / 4u - 1u)
                hs[3] -= (C + KPL - 1u) / KPL * KPL - C; // the NaN slots of the lane holding the last cube
            const uint32_t s4 = hs[0] + hs[1] + hs[2] + hs[3];
            uint32_t above = nb - (wave_excl_scan_u32(s4) + s4); // range scores in bins above this lane's four
            const uint32_t need = k - n_hi;
            uint32_t bb = kHistBins, n_above = 0u, n_b = 0u;
#pragma unroll
            for (int e = 3; e >= 0; --e) {
                if (above < need && above + hs[e] >= need)
                    bb = 4u * lane + uint32_t(e), n_above = above, n_b = hs[e];
                above += hs[e];
            }
            const int src = int(__builtin_ctzll(__ballot(bb != kHistBins))); // the counts cross `need` once
            b = uint32_t(__builtin_amdgcn_readlane(int(bb), src));
            n_hi += uint32_t(__builtin_amdgcn_readlane(int(n_above), src));
            nb = uint32_t(__builtin_amdgcn_readlane(int(n_b), src));
        };
        // The range's scores in bin b (at most 64) compacted one to a lane, then t selected among them by ballots.
        auto in_bin = [&](int m) {
            return f[m] >= lo && f[m] <= hi && ((bins[m / 4] >> (8 * (m % 4))) & 0xffu) == b;
        };
        auto pick = [&]() {
            uint32_t mine_n = 0u;
#pragma unroll
            for (int m = 0; m < KPL; ++m)
                mine_n += in_bin(m) ? 1u : 0u;
            uint32_t slot = wave_excl_scan_u32(mine_n);
            // The bin's count from the histogram and from the scores agree; else the key path ranks the row.
            const bool agree = uint32_t(__builtin_amdgcn_readlane(int(slot + mine_n), 63)) == nb;
#pragma unroll
            for (int m = 0; m < KPL; ++m)
                if (agree && in_bin(m))
                    cand[slot++] = __float_as_uint(f[m]);
            __builtin_amdgcn_s_waitcnt(0xC07F); // the wave's own LDS writes are visible to its reads after lgkmcnt(0)
            const float c = lane < nb ? __uint_as_float(cand[lane]) : __builtin_nanf("");
            uint64_t rem = agree ? __ballot(lane < nb) : 0u;
            uint32_t need = k - n_hi; // 1 <= need <= #rem
            for (int it = 0; it < 64 && rem; ++it) { // at most 64 rounds: each removes a score
                const float p = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(c), int(__builtin_ctzll(rem))));
                const uint64_t above_p = __ballot(c > p) & rem, at_p = __ballot(c == p) & rem;
                const uint32_t n_above_p = uint32_t(__popcll(above_p)), n_at_p = uint32_t(__popcll(at_p));
                if (need <= n_above_p) {
                    rem = above_p;
                } else if (need <= n_above_p + n_at_p) {
                    t = p, found = true;
                    break;
                } else {
                    need -= n_above_p + n_at_p;
                    rem &= ~(above_p | at_p);
                }
            }
        };
        if (!(lo < hi)) {
            t = lo, found = true; // every score equal
        } else if (float inv = float(kHistBins) / (hi - lo); inv < __builtin_huge_valf()) {
            level(std::true_type{}, inv);
            for (int lv = 1; nb > 64u && lv < kMaxLevels; ++lv) { // beyond kMaxLevels: the key path
                // The new range: bin b's scores, from its lowest to its highest (monotone bins: exactly those).
                float mn2 = __builtin_inff(), mx2 = -__builtin_inff();
#pragma unroll
                for (int m = 0; m < KPL; ++m) {
                    const bool in = in_bin(m);
                    mn2 = in ? fminf(mn2, f[m]) : mn2;
                    mx2 = in ? fmaxf(mx2, f[m]) : mx2;
                }
                lo = key_value(wave_min_u32(score_key(mn2)));
                hi = key_value(wave_max_u32(score_key(mx2)));
                if (!(lo < hi)) {
                    t = lo, found = true; // bin b's scores are equal: t itself
                    break;
                }
                inv = float(kHistBins) / (hi - lo);
                if (!(inv < __builtin_huge_valf()))
                    break;
                level(std::false_type{}, inv);
            }
            if (!found && nb <= 64u)
                pick();
        }
    }
    Mask gt = 0, eq = 0;
    if (found) {
#pragma unroll
        for (int m = 0; m < KPL; ++m) {
            gt |= f[m] > t ? Mask(1) << m : Mask(0); // NaN slots compare false
            eq |= f[m] == t ? Mask(1) << m : Mask(0);
        }
    } else {
        const uint32_t j0 = lane * KPL, nv = C > j0 ? min(C - j0, uint32_t(KPL)) : 0u;
        uint32_t key[KPL];
        uint32_t kmn = 0xffffffffu, kmx = 0u;
#pragma unroll
        for (int m = 0; m < KPL; ++m) {
            key[m] = uint32_t(m) < nv ? score_key(f[m]) : 0u;
            kmn = uint32_t(m) < nv ? min(kmn, key[m]) : kmn;
            kmx = max(kmx, key[m]);
        }
        uint32_t klo = wave_min_u32(kmn), khi = wave_max_u32(kmx);
        while (klo < khi) { // slot keys (0) are never counted: mid > klo
            const uint32_t d = khi - klo, mid = klo + (d >> 1) + (d & 1u);
            if (count_ge(key, mid) >= k)
                klo = mid;
            else
                khi = mid - 1u;
        }
        const Mask valid = nv >= uint32_t(KPL) ? ~Mask(0) : (Mask(1) << nv) - Mask(1);
#pragma unroll
        for (int m = 0; m < KPL; ++m) {
            gt |= key[m] > klo ? Mask(1) << m : Mask(0);
            eq |= key[m] == klo ? Mask(1) << m : Mask(0);
        }
        gt &= valid;
        eq &= valid;
    }
    select_emit<KPL>(gt, eq, g, i, k, local, out, out_stride, cnt);
}

// One wavefront per (head, query cube) row of s: the row is staged into LDS in the padded layout (coalesced loads),
// then ranked.
template <int KPL>
__global__ __launch_bounds__(256) void cube_topk_kernel(CubeGeo g, const float* __restrict__ s, uint32_t k,
                                                        uint32_t local, uint32_t out_stride, int32_t* __restrict__ idx,
                                                        int32_t* __restrict__ cnt)
{
    extern __shared__ float rows[]; // 4 padded rows, then 64 candidate words and a histogram per wave
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    float* row = rows + wave * kPaddedRow<KPL>;
    uint32_t* cand = reinterpret_cast<uint32_t*>(rows + 4u * kPaddedRow<KPL>) + wave * (64u + kHistBins);
    const uint32_t item = blockIdx.x * 4u + wave;
    if (item >= g.heads * g.cubes)
        return;
    const float* src = s + uint64_t(item) * g.cubes;
    bool bad = false;
    for (int u0 = 0; u0 < KPL; u0 += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) // clamped indices: eight loads go out together, unconditionally
            v[u] = src[min(lane + 64u * uint32_t(u0 + u), g.cubes - 1u)];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const uint32_t j = lane + 64u * uint32_t(u0 + u);
            const float x = j < g.cubes ? v[u] : __builtin_nanf("");
            bad |= j < g.cubes && !__builtin_isfinite(x);
            row[pad_word<KPL>(j)] = x; // NaN in the slots past the last cube
        }
    }
    const bool finite = __ballot(bad) == 0u;
    __builtin_amdgcn_s_waitcnt(0xC07F); // the wave reads only what it wrote itself
    RowVals<KPL> rv;
    load_vals<KPL>(row, rv);
    topk_vals<KPL>(rv, finite, g, item % g.cubes, k, local, idx + uint64_t(item) * out_stride, out_stride, cnt + item,
                   cand, cand + 64);
}

// cube_select: a persistent workgroup of 12 waves loops over tiles (16 query cubes of a head, dealt round robin), in
// two roles: 4 scoring waves (one a SIMD) and 8 ranking waves (two a SIMD, rows r and r + 8 of a tile each).
// Iteration j: the scoring waves score the key blocks of tile t_j into the LDS tile (split bf16 MFMAs on the key
// operands cube_split_kernel prepared, the next key block's loads in flight while a block's MFMAs run) while the
// ranking waves rank their rows of t_(j-1) from registers (VALU work); barrier; the ranking waves copy their rows of
// t_j into registers, with the rows' non-finite flags; barrier (the tile is free again). The roles run side by side
// on every SIMD, one's loads and MFMAs beside the other's VALU work, and in separate loops with the same barriers, so
// neither holds the other's registers (168 a wave at 768 threads).
// Measured at 768p (alternated): 0.420-0.426 ms; scoring alone 0.28 ms. Before: the key blocks split by every tile
// that scores them (126 times a head at 768p), 0.525-0.548 ms with this ranking and 0.585-0.599 ms with the ranking on
// order-preserving keys; 16 waves that each score and then rank one row 0.611-0.629 ms; 8 scoring waves at 1024
// threads 0.62-0.64 ms (128 registers a wave, spills).
constexpr uint32_t kSelectScorers = 4, kSelectRankers = 8;
constexpr int kSelectThreads = int(64 * (kSelectScorers + kSelectRankers));
constexpr uint32_t kSelectRows = 16;
constexpr uint32_t kSelectMaxCubes = 2048;
static_assert(2 * kSelectRankers == kSelectRows, "two rows of a tile a ranking wave");
constexpr size_t kSelectLds =
    (size_t(kSelectRows) * kPaddedRow<32> + kSelectRankers * (64u + kHistBins) + kSelectRows) * sizeof(float);
static_assert(kSelectLds <= 160 * 1024, "the select tile, candidates, histograms and flags fit gfx950's LDS");

__global__ __launch_bounds__(kSelectThreads) void cube_select_kernel(CubeGeo g, const float* __restrict__ qc,
                                                                     const float* __restrict__ kc,
                                                                     const uint4* __restrict__ ks, uint32_t k,
                                                                     uint32_t local, uint32_t out_stride,
                                                                     int32_t* __restrict__ idx,
                                                                     int32_t* __restrict__ cnt)
{
    // [16][padded row], then 64 candidate words and a histogram per ranking wave, then a flag word per row (set: the
    // row has an infinite or NaN score)
    extern __shared__ float tile[];
    const uint32_t wave = threadIdx.x >> 6;
    const uint64_t plane = uint64_t(g.cubes) * 128u;
    const uint32_t row_tiles = (g.cubes + kSelectRows - 1u) / kSelectRows, tiles = row_tiles * g.heads;
    uint32_t* row_flags =
        reinterpret_cast<uint32_t*>(tile + kSelectRows * kPaddedRow<32> + kSelectRankers * (64u + kHistBins));
    {
        // NaN in each row's slots past the last cube (never scored: the ranking takes them as no score); flags clear.
        const uint32_t pad = 64u * 32u - g.cubes;
        for (uint32_t q = threadIdx.x; q < kSelectRows * pad; q += blockDim.x) {
            const uint32_t r = q / pad, j = g.cubes + (q - r * pad);
            tile[r * kPaddedRow<32> + pad_word<32>(j)] = __builtin_nanf("");
        }
        if (threadIdx.x < kSelectRows)
            row_flags[threadIdx.x] = 0u;
        __syncthreads();
    }
    if (wave < kSelectScorers) {
        const uint32_t kblocks = (g.cubes + 15u) / 16u;
        for (uint32_t t = blockIdx.x; t < tiles; t += gridDim.x) {
            const uint32_t h = t / row_tiles, i0 = (t - h * row_tiles) * kSelectRows;
            score_rows_split(g, qc + h * plane, kc + h * plane, ks + uint64_t(h) * kblocks * 512u, i0, tile,
                             kPaddedRow<32>, wave, kSelectScorers, row_flags);
            __syncthreads(); // tile t scored
            __syncthreads(); // the ranking waves hold every row of t: the tile is free
        }
        return;
    }
    const uint32_t r0 = wave - kSelectScorers; // rows r0 and r0 + 8 of each tile
    uint32_t* cand = reinterpret_cast<uint32_t*>(tile + kSelectRows * kPaddedRow<32>) + r0 * (64u + kHistBins);
    auto rank_row = [&](uint32_t t, uint32_t r, RowVals<32>& vals, bool finite) {
        const uint32_t h = t / row_tiles, i = (t - h * row_tiles) * kSelectRows + r;
        if (i < g.cubes) {
            const uint64_t item = uint64_t(h) * g.cubes + i;
            topk_vals<32>(vals, finite, g, i, k, local, idx + item * out_stride, out_stride, cnt + item, cand,
                          cand + 64);
        }
    };
    RowVals<32> rva, rvb;
    bool fa = true, fb = true;
    for (uint32_t j = 0;; ++j) {
        const uint32_t t = blockIdx.x + j * gridDim.x;
        if (j > 0u) {
            rank_row(t - gridDim.x, r0, rva, fa);
            rank_row(t - gridDim.x, r0 + kSelectRankers, rvb, fb);
        }
        if (t >= tiles)
            break;
        __syncthreads(); // tile t scored
        load_vals<32>(tile + r0 * kPaddedRow<32>, rva);
        load_vals<32>(tile + (r0 + kSelectRankers) * kPaddedRow<32>, rvb);
        fa = __builtin_amdgcn_readfirstlane(row_flags[r0]) == 0u;
        fb = __builtin_amdgcn_readfirstlane(row_flags[r0 + kSelectRankers]) == 0u;
        if ((threadIdx.x & 63u) == 0u)
            row_flags[r0] = row_flags[r0 + kSelectRankers] = 0u; // after the reads above (same wave, same words)
        __syncthreads(); // every row of t in registers: the tile is free
    }
}

// H3::Cubes' map (docs/architecture.md:120-125): attention row 64 c + l is cube c's slot l = (dt * 4 + dy) * 4 + dx,
// i.e. video token (4 ct + dt, 4 cy + dy, 4 cx + dx), whose model row is video_row0 + (t * grid_h + y) * grid_w + x,
// or -1 where the slot lies in the grid's padding; attention rows cubes * 64 + j are the dense rows
// dense_row0 + j. counts[c] is cube c's token count. A thread an attention row.
struct CubeMapParams {
    uint32_t gt, gh, gw, ch, cw, plane, cubes, n_dense;
    uint64_t video_row0, dense_row0;
};

__global__ __launch_bounds__(256) void cube_map_kernel(CubeMapParams p, int32_t* __restrict__ map,
                                                       int32_t* __restrict__ counts)
{
    const uint64_t r = uint64_t(blockIdx.x) * 256u + threadIdx.x;
    const uint64_t video = uint64_t(p.cubes) * 64u;
    if (r < video) {
        const uint32_t c = uint32_t(r >> 6), l = uint32_t(r & 63u);
        const uint32_t ct = c / p.plane, rem = c - ct * p.plane, cy = rem / p.cw, cx = rem - cy * p.cw;
        const uint32_t t = 4u * ct + (l >> 4), y = 4u * cy + ((l >> 2) & 3u), x = 4u * cx + (l & 3u);
        const bool ok = t < p.gt && y < p.gh && x < p.gw;
        map[r] = ok ? int32_t(p.video_row0 + (uint64_t(t) * p.gh + y) * p.gw + x) : -1;
        if (counts && l == 0) {
            const uint32_t nt = min(4u, p.gt - 4u * ct), ny = min(4u, p.gh - 4u * cy), nx = min(4u, p.gw - 4u * cx);
            counts[c] = int32_t(nt * ny * nx);
        }
    } else if (r < video + p.n_dense) {
        map[r] = int32_t(p.dense_row0 + (r - video));
    }
}

// The attention's query-cube order (flash_attn_sparse_128's ordered form): head h's cubes ranked by the key
// m(c) cubes + c, where m(c) is the middle entry idx[c][cnt[c] / 2] of cube c's pass list (the median of an ascending
// list; `cubes` for an empty list or an entry outside [0, cubes)), so the cubes sort by that entry and ties by index;
// order[h cubes + rank] = c. A workgroup stages one head's keys in LDS and ranks 256 of its cubes, a thread a cube:
// rank = #{keys below its own} (the keys are distinct), four keys an LDS read, the same for every lane (a broadcast).
constexpr uint32_t kOrderMaxCubes = 4096;

__global__ __launch_bounds__(256) void cube_order_kernel(uint32_t cubes, uint32_t out_stride,
                                                         const int32_t* __restrict__ idx,
                                                         const int32_t* __restrict__ cnt, int32_t* __restrict__ order)
{
    __shared__ uint4 keys4[kOrderMaxCubes / 4u];
    uint32_t* const keys = reinterpret_cast<uint32_t*>(keys4);
    const uint32_t slices = (cubes + 255u) / 256u, h = blockIdx.x / slices;
    const uint32_t mine_c = (blockIdx.x - h * slices) * 256u + threadIdx.x, n4 = (cubes + 3u) / 4u;
    const int32_t* hidx = idx + uint64_t(h) * cubes * out_stride;
    const int32_t* hcnt = cnt + uint64_t(h) * cubes;
    for (uint32_t c = threadIdx.x; c < 4u * n4; c += 256u) {
        uint32_t key = 0xffffffffu; // past the last cube: above every key
        if (c < cubes) {
            const int32_t n = min(max(hcnt[c], 0), int32_t(out_stride));
            const int32_t j = n > 0 ? hidx[uint64_t(c) * out_stride + uint32_t(n) / 2u] : -1;
            key = (j >= 0 && uint32_t(j) < cubes ? uint32_t(j) : cubes) * cubes + c;
        }
        keys[c] = key;
    }
    __syncthreads();
    if (mine_c >= cubes)
        return;
    const uint32_t mine = keys[mine_c];
    uint32_t rank[4] = {0u, 0u, 0u, 0u};
#pragma unroll 8
    for (uint32_t i = 0; i < n4; ++i) { // eight reads in flight: the loop is bound by the LDS latency otherwise
        const uint4 kq = keys4[i];
        rank[0] += kq.x < mine ? 1u : 0u;
        rank[1] += kq.y < mine ? 1u : 0u;
        rank[2] += kq.z < mine ? 1u : 0u;
        rank[3] += kq.w < mine ? 1u : 0u;
    }
    order[uint64_t(h) * cubes + (rank[0] + rank[1]) + (rank[2] + rank[3])] = int32_t(mine_c);
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

// Dynamic LDS above the default limit for `kernel`, once per device.
int set_lds_limit(const void* kernel, size_t bytes)
{
    const hipError_t e = host::allow_dynamic_lds(kernel, bytes);
    return e == hipSuccess ? MH3_OK : host::hip_error(e);
}

// Bytes from the start of a head-tile array (q or k) to the end of the last row the selector reads: its last head's
// last cube row (the grid's last token, or the last gathered cube's last slot).
uint64_t tile_span_bytes(const CubeGeo& g)
{
    const uint64_t last_row =
        g.row0 + (g.layout == MH3_CUBES_GRID ? uint64_t(g.gt) * g.gh * g.gw : uint64_t(g.cubes) * 64u) - 1u;
    return ((uint64_t(g.heads) - 1u) * g.head_stride + last_row * g.row_stride + 128u) * 2u;
}

} // namespace

extern "C" {

int mh3_cube_map(const MH3CubeMapArgs* args, int32_t* map, int32_t* counts, mh3_stream_t stream)
{
    if (!args)
        return MH3_ERR_POINTER;
    if (args->grid_t == 0 || args->grid_h == 0 || args->grid_w == 0)
        return MH3_ERR_SHAPE;
    const uint64_t cubes = uint64_t((args->grid_t + 3u) / 4u) * ((args->grid_h + 3u) / 4u) * ((args->grid_w + 3u) / 4u);
    const uint64_t tokens = uint64_t(args->grid_t) * args->grid_h * args->grid_w;
    const uint64_t rows = cubes * 64u + args->n_dense;
    const uint64_t lim = uint64_t(INT32_MAX);
    // Model rows are int32 in the map; the dense rows may not be video rows.
    if (rows > lim || args->video_row0 + tokens > lim + 1u || args->dense_row0 + args->n_dense > lim + 1u)
        return MH3_ERR_SHAPE;
    if (args->n_dense && args->dense_row0 < args->video_row0 + tokens &&
        args->video_row0 < args->dense_row0 + args->n_dense)
        return MH3_ERR_PARAM;
    if (!map)
        return MH3_ERR_POINTER;
    if (counts && host::overlaps(map, rows * 4u, counts, cubes * 4u))
        return MH3_ERR_PARAM;
    CubeMapParams p;
    p.gt = args->grid_t, p.gh = args->grid_h, p.gw = args->grid_w;
    p.ch = (p.gh + 3u) / 4u, p.cw = (p.gw + 3u) / 4u, p.plane = p.ch * p.cw, p.cubes = uint32_t(cubes);
    p.n_dense = args->n_dense, p.video_row0 = args->video_row0, p.dense_row0 = args->dense_row0;
    hipLaunchKernelGGL(cube_map_kernel, dim3(uint32_t((rows + 255u) / 256u)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), p, map, counts);
    return host::check_launch();
}

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
    const uint64_t pooled = uint64_t(g.heads) * g.cubes * 128u * 4u;
    const host::Span in[] = {{q, tile_span_bytes(g)}, {k, tile_span_bytes(g)}};
    const host::Span out[] = {{qc, pooled}, {kc, pooled}, {counts, uint64_t(g.cubes) * 4u}};
    if (host::any_overlap(in, out))
        return MH3_ERR_PARAM;
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
    const uint64_t pooled = uint64_t(g.heads) * g.cubes * 128u * 4u;
    const host::Span in[] = {{qc, pooled}, {kc, pooled}};
    const host::Span out[] = {{s, uint64_t(g.heads) * g.cubes * g.cubes * 4u}};
    if (host::any_overlap(in, out))
        return MH3_ERR_PARAM;
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
    {
        const host::Span in[] = {{s, uint64_t(g.heads) * g.cubes * g.cubes * 4u}};
        const host::Span out[] = {{idx, uint64_t(g.heads) * g.cubes * args->out_stride * 4u},
                            {cnt, uint64_t(g.heads) * g.cubes * 4u}};
        if (host::any_overlap(in, out))
            return MH3_ERR_PARAM;
    }
    const uint32_t items = g.heads * g.cubes;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (g.cubes <= 2048) {
        constexpr size_t lds = (4u * kPaddedRow<32> + 4u * (64u + kHistBins)) * sizeof(float);
        hipLaunchKernelGGL(cube_topk_kernel<32>, dim3((items + 3u) / 4u), dim3(256), lds, st, g, s, args->k,
                           args->local, args->out_stride, idx, cnt);
    } else {
        constexpr size_t lds = (4u * kPaddedRow<64> + 4u * (64u + kHistBins)) * sizeof(float);
        const int lds_ok = set_lds_limit(reinterpret_cast<const void*>(&cube_topk_kernel<64>), lds);
        if (lds_ok != MH3_OK)
            return lds_ok;
        hipLaunchKernelGGL(cube_topk_kernel<64>, dim3((items + 3u) / 4u), dim3(256), lds, st, g, s, args->k,
                           args->local, args->out_stride, idx, cnt);
    }
    return host::check_launch();
}

// cube_select's workspace: the key operands split into bf16 parts, 8 KiB a (head, 16-key-cube block).
uint64_t select_workspace(const CubeGeo& g) { return uint64_t(g.heads) * ((g.cubes + 15u) / 16u) * 8192u; }

int64_t mh3_cube_select_workspace_bytes(const MH3CubeArgs* args)
{
    CubeGeo g;
    const int rc = make_geo(args, g);
    return rc != MH3_OK ? int64_t(rc) : int64_t(select_workspace(g));
}

int mh3_cube_select(const MH3CubeArgs* args, const float* qc, const float* kc, void* workspace,
                    uint64_t workspace_bytes, int32_t* idx, int32_t* cnt, mh3_stream_t stream)
{
    CubeGeo g;
    int rc = make_geo(args, g);
    if (rc != MH3_OK)
        return rc;
    if ((rc = check_topk_args(args, g)) != MH3_OK)
        return rc;
    if (!qc || !kc || !idx || !cnt || !workspace)
        return MH3_ERR_POINTER;
    if (!host::aligned16(qc) || !host::aligned16(kc) || !host::aligned16(workspace))
        return MH3_ERR_ALIGN;
    if (workspace_bytes < select_workspace(g))
        return MH3_ERR_SHAPE;
    {
        const uint64_t pooled = uint64_t(g.heads) * g.cubes * 128u * 4u;
        const host::Span in[] = {{qc, pooled}, {kc, pooled}};
        const host::Span out[] = {{idx, uint64_t(g.heads) * g.cubes * args->out_stride * 4u},
                                  {cnt, uint64_t(g.heads) * g.cubes * 4u},
                                  {workspace, select_workspace(g)}};
        if (host::any_overlap(in, out))
            return MH3_ERR_PARAM;
    }
    if (g.cubes > kSelectMaxCubes)
        return MH3_ERR_UNSUPPORTED; // more cubes than the LDS tile holds: use cube_scores + cube_topk
    const int lds_ok = set_lds_limit(reinterpret_cast<const void*>(&cube_select_kernel), kSelectLds);
    if (lds_ok != MH3_OK)
        return lds_ok;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    uint4* ks = static_cast<uint4*>(workspace);
    const uint32_t blocks = g.heads * ((g.cubes + 15u) / 16u); // (head, key block) items, one a wave
    hipLaunchKernelGGL(cube_split_kernel, dim3((blocks + 3u) / 4u), dim3(256), 0, st, g, kc, ks);
    if ((rc = host::check_launch()) != MH3_OK)
        return rc;
    // Persistent: one workgroup a CU (the tile takes the LDS), at most one a tile.
    const uint32_t tiles = (g.cubes + kSelectRows - 1) / kSelectRows * g.heads;
    const dim3 grid(std::min<uint32_t>(tiles, uint32_t(host::cu_count())));
    hipLaunchKernelGGL(cube_select_kernel, grid, dim3(kSelectThreads), kSelectLds, st, g, qc, kc, ks, args->k,
                       args->local, args->out_stride, idx, cnt);
    return host::check_launch();
}

int mh3_cube_order(const MH3CubeArgs* args, const int32_t* idx, const int32_t* cnt, int32_t* order,
                   mh3_stream_t stream)
{
    CubeGeo g;
    const int rc = make_geo(args, g);
    if (rc != MH3_OK)
        return rc;
    if (args->out_stride == 0)
        return MH3_ERR_SHAPE;
    if (!idx || !cnt || !order)
        return MH3_ERR_POINTER;
    if ((reinterpret_cast<uintptr_t>(idx) | reinterpret_cast<uintptr_t>(cnt) | reinterpret_cast<uintptr_t>(order)) %
            4u !=
        0u)
        return MH3_ERR_ALIGN;
    {
        const uint64_t bytes = uint64_t(g.heads) * g.cubes * 4u; // cnt and order
        const host::Span in[] = {{idx, bytes * args->out_stride}, {cnt, bytes}};
        const host::Span out[] = {{order, bytes}};
        if (host::any_overlap(in, out))
            return MH3_ERR_PARAM;
    }
    if (g.cubes > kOrderMaxCubes)
        return MH3_ERR_UNSUPPORTED;
    const uint32_t slices = (g.cubes + 255u) / 256u;
    hipLaunchKernelGGL(cube_order_kernel, dim3(g.heads * slices), dim3(256), 0, static_cast<hipStream_t>(stream),
                       g.cubes, args->out_stride, idx, cnt, order);
    return host::check_launch();
}

} // extern "C"
