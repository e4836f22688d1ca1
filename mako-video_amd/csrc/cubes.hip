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
// - top-k: one wavefront per (head, query cube) holds the row's scores as order-preserving 32-bit keys in VGPRs, lane l
//   owning cubes 32 l ... 32 l + 31. A 128-bin histogram of the scores, linear in value between the row's minimum and
//   maximum (LDS atomics, one pass), brackets the k-th largest key to one bin's keys; where that bin holds more than
//   64 keys a binary search over the key range (per-lane counts, a DPP wave sum) narrows it further, and at most 64
//   candidates, one to a lane, finish the search.
//   The selection is a per-lane bit mask; wave prefix sums over lanes rank the ties (lowest index first) and place
//   each lane's indices, so the output is ascending with no per-element ballots.
// - cube_select keeps a 16 x C score tile in LDS between the two phases, so the scores never reach HBM. Its
//   workgroups are persistent (one a CU); scoring waves and ranking waves overlap one tile's ranking with the next
//   tile's scoring.
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

// Scores of query block [i0, i0 + 16) of head h against every key cube; the wave takes key blocks wave, wave + waves...
// Writes s[r][j] for r < 16, j < cubes into `dst` at r * ld + j, or at r * ld + pad_word<32>(j) when PAD (rows past
// the last query cube skipped). With DEPTH > 0 the key blocks stream through a DEPTH-deep register ring (block
// b + DEPTH waves loads while block b's MFMAs run); with DEPTH 0 each block is loaded when it is scored.
template <bool PAD, int DEPTH>
__device__ __forceinline__ void score_rows(const CubeGeo& g, const float* __restrict__ qh, const float* __restrict__ kh,
                                           uint32_t i0, float* dst, uint64_t ld, uint32_t wave, uint32_t waves)
{
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t kblocks = (g.cubes + 15u) / 16u;
    SplitRow qs;
    {
        RawRows qraw;
        load_raw(qh, i0, g.cubes, qraw);
        split_exchange(qraw, qs);
    }
    auto finish = [&](uint32_t b, floatx4 acc) {
        const bool finite = __builtin_isfinite(acc[0]) && __builtin_isfinite(acc[1]) && __builtin_isfinite(acc[2]) &&
                            __builtin_isfinite(acc[3]);
        if (__ballot(!finite))
            acc = score_block_direct(qh, kh, i0, b * 16u, g.cubes);
        const uint32_t j = b * 16u + (lane & 15u);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint32_t r = (lane >> 4) * 4u + uint32_t(v);
            if (j < g.cubes && i0 + r < g.cubes)
                dst[r * ld + (PAD ? pad_word<32>(j) : j)] = acc[v] * kScoreScale;
        }
    };
    if constexpr (DEPTH == 0) {
        for (uint32_t b = wave; b < kblocks; b += waves) {
            SplitRow ks;
            {
                RawRows raw;
                load_raw(kh, b * 16u, g.cubes, raw);
                split_exchange(raw, ks);
            }
            finish(b, score_block(qs, ks));
        }
    } else {
        RawRows kr[DEPTH];
#pragma unroll
        for (int d = 0; d < DEPTH; ++d)
            if (wave + uint32_t(d) * waves < kblocks)
                load_raw(kh, (wave + uint32_t(d) * waves) * 16u, g.cubes, kr[d]);
        for (uint32_t b0 = wave; b0 < kblocks; b0 += DEPTH * waves) {
#pragma unroll
            for (int d = 0; d < DEPTH; ++d) {
                const uint32_t b = b0 + uint32_t(d) * waves;
                if (b >= kblocks)
                    break;
                SplitRow ks;
                split_exchange(kr[d], ks);
                if (b + DEPTH * waves < kblocks)
                    load_raw(kh, (b + DEPTH * waves) * 16u, g.cubes, kr[d]);
                finish(b, score_block(qs, ks));
            }
        }
    }
}

// Key blocks in flight a wave in cube_scores: one (0.467-0.469 ms at 768p against 0.478 for two, alternated).
constexpr int kScoreDepth = 1;

__global__ __launch_bounds__(256) void cube_scores_kernel(CubeGeo g, const float* __restrict__ qc,
                                                          const float* __restrict__ kc, float* __restrict__ s)
{
    const uint32_t h = blockIdx.y, i0 = blockIdx.x * 16u;
    const uint64_t plane = uint64_t(g.cubes) * 128u;
    score_rows<false, kScoreDepth>(g, qc + h * plane, kc + h * plane, i0, s + (uint64_t(h) * g.cubes + i0) * g.cubes,
                                   g.cubes, threadIdx.x >> 6, blockDim.x >> 6);
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

// Top-k plus local cubes of one (head, query cube i) row of `cubes` scores, by one wavefront. Lane l holds cubes
// j = l KPL + m (m < KPL), read from `row` in the padded layout of pad_word; entries with j >= cubes are ignored.
// `cand` (64 words) and `hist` (kHistBins words) are LDS private to the wave.
// The k-th largest key t is the largest t with #{key >= t} >= k. The search keeps lo (#{key >= lo} = n_lo >= k) and
// hi (#{key > hi} = n_hi < k), t in [lo, hi]. When the row's scores are finite and not all equal, a histogram sets
// the first bracket: bin(v) = min(127, (v - vmin) * 128 / (vmax - vmin)) is non-decreasing in v (rounded
// subtraction, multiplication, minimum and truncation all are), so every key of a higher bin exceeds every key of a
// lower one. With b the bin where the count from the top first reaches k, lo and hi are the smallest and largest keys
// of bin b, n_hi the keys above it and n_lo that plus its own. A binary search over the key range then narrows
// [lo, hi] while more than 64 keys lie in it; the rest are compacted one to a lane and the search finishes over them
// alone (#{key >= m} = n_hi + #{candidates >= m}).
// The selection is then a per-lane bit mask: keys above t, the first k - #{key > t} keys equal to t in cube order
// (ranked by a wave prefix sum of per-lane tie counts) and the local cubes; a prefix sum of the per-lane counts gives
// each lane its output position, so the indices come out ascending.
// A row's scores as lane l holds them: keys of cubes j = l KPL + m (m < KPL); bit m of `valid` set when j < cubes
// (other keys 0).
template <int KPL>
struct RowKeys {
    typedef typename std::conditional<KPL == 32, uint32_t, uint64_t>::type Mask;
    uint32_t key[KPL];
    Mask valid;
};

// Lane l's KPL scores of a row in the padded layout of pad_word, as keys.
template <int KPL>
__device__ __forceinline__ void load_keys(const float* row, uint32_t C, RowKeys<KPL>& r)
{
    typedef typename RowKeys<KPL>::Mask Mask;
    const uint32_t lane = threadIdx.x & 63u, j0 = lane * KPL;
    const float4* mine = reinterpret_cast<const float4*>(row + lane * (KPL + 4));
    const uint32_t nv = C > j0 ? min(C - j0, uint32_t(KPL)) : 0u; // the lane's cubes: keys 0 .. nv - 1
    r.valid = nv >= uint32_t(KPL) ? ~Mask(0) : (Mask(1) << nv) - Mask(1);
#pragma unroll
    for (int v = 0; v < KPL / 4; ++v) {
        const float4 f = mine[v];
        const float fv[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int m = 4 * v + c;
            r.key[m] = uint32_t(m) < nv ? score_key(fv[c]) : 0u;
        }
    }
}

template <int KPL>
__device__ __forceinline__ void topk_keys(const RowKeys<KPL>& rk, const CubeGeo& g, uint32_t i, uint32_t k,
                                          uint32_t local, int32_t* __restrict__ out, uint32_t out_stride,
                                          int32_t* __restrict__ cnt, uint32_t* cand, uint32_t* hist)
{
    typedef typename RowKeys<KPL>::Mask Mask;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t C = g.cubes, j0 = lane * KPL;
    const uint32_t(&key)[KPL] = rk.key;
    const Mask valid = rk.valid;
    uint32_t mn = 0xffffffffu, mx = 0u;
#pragma unroll
    for (int m = 0; m < KPL; ++m) {
        const bool ok = (valid >> m) & 1u;
        mn = ok && key[m] < mn ? key[m] : mn;
        mx = ok && key[m] > mx ? key[m] : mx;
    }
    uint32_t lo = wave_min_u32(mn), hi = wave_max_u32(mx);
    uint32_t n_lo = C, n_hi = 0u; // every valid key is >= the minimum; padding keys (0) are never counted (mid > 0)
    constexpr uint32_t kKeyNegInf = 0x007fffffu, kKeyPosInf = 0xff800000u; // score_key(-inf), score_key(+inf)
    const float vmin = key_value(lo), vmax = key_value(hi);
    const float inv = float(kHistBins) / (vmax - vmin);
    if (lo > kKeyNegInf && hi < kKeyPosInf && lo < hi && inv < __builtin_huge_valf()) {
#pragma unroll
        for (uint32_t e = lane; e < kHistBins; e += 64u)
            hist[e] = 0u; // 32-bit stores: a hoisted 16-byte zero vector was spilled under 1024 threads
        // NaN (padding keys) gives the top bin; padding is never counted or compared.
        auto bin_of = [&](uint32_t key_m) {
            return uint32_t(fminf((key_value(key_m) - vmin) * inv, float(kHistBins - 1u)));
        };
        // Each key's bin, kept four to a register (byte m % 4 of bins[m / 4]; 0xff for a padding key, which no bin
        // index equals) for the bracket's pass below.
        uint32_t bins[KPL / 4];
#pragma unroll
        for (int m = 0; m < KPL; ++m) {
            const bool ok = (valid >> m) & 1u;
            const uint32_t b_m = ok ? bin_of(key[m]) : 0xffu;
            if (ok)
                atomicAdd(hist + b_m, 1u);
            bins[m / 4] = (m % 4 == 0 ? 0u : bins[m / 4]) | (b_m << (8 * (m % 4)));
        }
        __builtin_amdgcn_s_waitcnt(0xC07F); // the wave's own LDS atomics are visible to its reads after lgkmcnt(0)
        const uint4 h4 = lane < kHistBins / 4u ? reinterpret_cast<const uint4*>(hist)[lane] // bins 4 lane ... + 3
                                               : uint4{0u, 0u, 0u, 0u};
        const uint32_t hs[4] = {h4.x, h4.y, h4.z, h4.w};
        const uint32_t s4 = hs[0] + hs[1] + hs[2] + hs[3];
        uint32_t above = C - (wave_excl_scan_u32(s4) + s4); // keys in bins above this lane's four
        uint32_t b = kHistBins, n_above = 0u, n_b = 0u;
#pragma unroll
        for (int e = 3; e >= 0; --e) {
            if (above < k && above + hs[e] >= k)
                b = 4u * lane + uint32_t(e), n_above = above, n_b = hs[e];
            above += hs[e];
        }
        const uint64_t owner = __ballot(b != kHistBins); // exactly one lane: the counts from the top cross k once
        const int src = int(__builtin_ctzll(owner));
        b = uint32_t(__builtin_amdgcn_readlane(int(b), src));
        n_hi = uint32_t(__builtin_amdgcn_readlane(int(n_above), src));
        n_lo = n_hi + uint32_t(__builtin_amdgcn_readlane(int(n_b), src));
        uint32_t bmn = 0xffffffffu, bmx = 0u;
#pragma unroll
        for (int m = 0; m < KPL; ++m) {
            const bool in_b = ((bins[m / 4] >> (8 * (m % 4))) & 0xffu) == b;
            bmn = in_b && key[m] < bmn ? key[m] : bmn;
            bmx = in_b && key[m] > bmx ? key[m] : bmx;
        }
        lo = wave_min_u32(bmn), hi = wave_max_u32(bmx);
    }
    while (lo < hi && n_lo - n_hi > 64u) {
        const uint32_t d = hi - lo;
        const uint32_t mid = lo + (d >> 1) + (d & 1u);
        const uint32_t n = count_ge(key, mid);
        if (n >= k)
            lo = mid, n_lo = n;
        else
            hi = mid - 1u, n_hi = n;
    }
    if (lo < hi) {
        uint32_t mine_n = 0;
#pragma unroll
        for (int m = 0; m < KPL; ++m)
            mine_n += ((valid >> m) & 1u) && key[m] >= lo && key[m] <= hi ? 1u : 0u;
        uint32_t slot = wave_excl_scan_u32(mine_n); // the candidates number n_lo - n_hi <= 64
#pragma unroll
        for (int m = 0; m < KPL; ++m)
            if (((valid >> m) & 1u) && key[m] >= lo && key[m] <= hi)
                cand[slot++] = key[m];
        __builtin_amdgcn_s_waitcnt(0xC07F); // the wave's own LDS writes are visible to its reads after lgkmcnt(0)
        const uint32_t c = lane < n_lo - n_hi ? cand[lane] : 0u;
        const uint32_t need = k - n_hi;
        while (lo < hi) {
            const uint32_t d = hi - lo;
            const uint32_t mid = lo + (d >> 1) + (d & 1u);
            if (uint32_t(__popcll(__ballot(c >= mid))) >= need)
                lo = mid;
            else
                hi = mid - 1u;
        }
    }
    const uint32_t t = lo;
    Mask gt = 0, eq = 0;
#pragma unroll
    for (int m = 0; m < KPL; ++m) {
        gt |= key[m] > t ? Mask(1) << m : Mask(0);
        eq |= key[m] == t ? Mask(1) << m : Mask(0);
    }
    gt &= valid;
    eq &= valid;
    const uint32_t n_gt = uint32_t(__popcll(uint64_t(gt))), n_eq = uint32_t(__popcll(uint64_t(eq)));
    const uint32_t need_eq = k - wave_sum_u32(n_gt); // >= 1
    const uint32_t eq_before = wave_excl_scan_u32(n_eq);
    uint32_t take = need_eq > eq_before ? min(need_eq - eq_before, n_eq) : 0u;
    Mask sel = gt;
#pragma unroll
    for (int m = 0; m < KPL; ++m) {
        const bool tie = (eq >> m) & 1u;
        sel |= tie && take > 0u ? Mask(1) << m : Mask(0);
        take -= tie && take > 0u ? 1u : 0u;
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

template <int KPL>
__device__ __forceinline__ void topk_row(const float* row, const CubeGeo& g, uint32_t i, uint32_t k, uint32_t local,
                                         int32_t* __restrict__ out, uint32_t out_stride, int32_t* __restrict__ cnt,
                                         uint32_t* cand, uint32_t* hist)
{
    RowKeys<KPL> rk;
    load_keys<KPL>(row, g.cubes, rk);
    topk_keys<KPL>(rk, g, i, k, local, out, out_stride, cnt, cand, hist);
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
#pragma unroll 8
    for (uint32_t j = lane; j < g.cubes; j += 64u)
        row[pad_word<KPL>(j)] = src[j];
    __builtin_amdgcn_s_waitcnt(0xC07F); // the wave reads only what it wrote itself
    topk_row<KPL>(row, g, item % g.cubes, k, local, idx + uint64_t(item) * out_stride, out_stride, cnt + item, cand,
                  cand + 64);
}

// cube_select: a persistent workgroup of 12 waves loops over tiles (16 query cubes of a head, dealt round robin), in
// two roles: 4 scoring waves (one a SIMD) and 8 ranking waves (two a SIMD, rows r and r + 8 of a tile each).
// Iteration j: the scoring waves score the key blocks of tile t_j into the LDS tile (split bf16 MFMAs, the next key
// block's loads in flight while a block's MFMAs run) while the ranking waves rank their rows of t_(j-1) from
// registers (VALU work); barrier; the ranking waves copy their rows of t_j into registers as keys; barrier (the tile
// is free again). The roles run side by side on every SIMD, one's loads and MFMAs beside the other's VALU work, and
// in separate loops with the same barriers, so neither holds the other's registers (168 a wave at 768 threads).
// Measured at 768p (alternated): 0.585-0.607 ms against 0.611-0.629 for 16 waves that each score and then rank one
// row (there scoring and ranking barely overlap: the split's VALU work competes with the ranking's); scoring alone
// 0.51 ms, ranking alone 0.43 ms. Slower: 8 scoring waves at 1024 threads (0.62-0.64 ms, 128 registers a wave with
// spills), scoring without the one-block ring (0.66-0.68 ms), a two-block ring (0.87 ms: 17 registers spilled in the
// loop). A timing copy without the split's VALU work and lane exchange (its outputs wrong) ran 0.51-0.56 ms: split
// copies of qc and kc prepared ahead would gain at most that, less the pass that writes them.
constexpr uint32_t kSelectScorers = 4, kSelectRankers = 8;
constexpr int kSelectThreads = int(64 * (kSelectScorers + kSelectRankers));
constexpr uint32_t kSelectRows = 16;
constexpr uint32_t kSelectMaxCubes = 2048;
static_assert(2 * kSelectRankers == kSelectRows, "two rows of a tile a ranking wave");
constexpr size_t kSelectLds =
    (size_t(kSelectRows) * kPaddedRow<32> + kSelectRankers * (64u + kHistBins)) * sizeof(float);
static_assert(kSelectLds <= 160 * 1024, "the select tile, candidates and histograms fit gfx950's LDS");

__global__ __launch_bounds__(kSelectThreads) void cube_select_kernel(CubeGeo g, const float* __restrict__ qc,
                                                                     const float* __restrict__ kc, uint32_t k,
                                                                     uint32_t local, uint32_t out_stride,
                                                                     int32_t* __restrict__ idx,
                                                                     int32_t* __restrict__ cnt)
{
    extern __shared__ float tile[]; // [16][padded row], then 64 candidate words and a histogram per ranking wave
    const uint32_t wave = threadIdx.x >> 6;
    const uint64_t plane = uint64_t(g.cubes) * 128u;
    const uint32_t row_tiles = (g.cubes + kSelectRows - 1u) / kSelectRows, tiles = row_tiles * g.heads;
    if (wave < kSelectScorers) {
        for (uint32_t t = blockIdx.x; t < tiles; t += gridDim.x) {
            const uint32_t h = t / row_tiles, i0 = (t - h * row_tiles) * kSelectRows;
            score_rows<true, 1>(g, qc + h * plane, kc + h * plane, i0, tile, kPaddedRow<32>, wave, kSelectScorers);
            __syncthreads(); // tile t scored
            __syncthreads(); // the ranking waves hold every row of t: the tile is free
        }
        return;
    }
    const uint32_t r0 = wave - kSelectScorers; // rows r0 and r0 + 8 of each tile
    uint32_t* cand = reinterpret_cast<uint32_t*>(tile + kSelectRows * kPaddedRow<32>) + r0 * (64u + kHistBins);
    auto rank_row = [&](uint32_t t, uint32_t r, const RowKeys<32>& keys) {
        const uint32_t h = t / row_tiles, i = (t - h * row_tiles) * kSelectRows + r;
        if (i < g.cubes) {
            const uint64_t item = uint64_t(h) * g.cubes + i;
            topk_keys<32>(keys, g, i, k, local, idx + item * out_stride, out_stride, cnt + item, cand, cand + 64);
        }
    };
    RowKeys<32> rka, rkb;
    for (uint32_t j = 0;; ++j) {
        const uint32_t t = blockIdx.x + j * gridDim.x;
        if (j > 0u) {
            rank_row(t - gridDim.x, r0, rka);
            rank_row(t - gridDim.x, r0 + kSelectRankers, rkb);
        }
        if (t >= tiles)
            break;
        __syncthreads(); // tile t scored
        load_keys<32>(tile + r0 * kPaddedRow<32>, g.cubes, rka);
        load_keys<32>(tile + (r0 + kSelectRankers) * kPaddedRow<32>, g.cubes, rkb);
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
    {
        const uint64_t pooled = uint64_t(g.heads) * g.cubes * 128u * 4u;
        const host::Span in[] = {{qc, pooled}, {kc, pooled}};
        const host::Span out[] = {{idx, uint64_t(g.heads) * g.cubes * args->out_stride * 4u},
                            {cnt, uint64_t(g.heads) * g.cubes * 4u}};
        if (host::any_overlap(in, out))
            return MH3_ERR_PARAM;
    }
    if (g.cubes > kSelectMaxCubes)
        return MH3_ERR_UNSUPPORTED; // more cubes than the LDS tile holds: use cube_scores + cube_topk
    const int lds_ok = set_lds_limit(reinterpret_cast<const void*>(&cube_select_kernel), kSelectLds);
    if (lds_ok != MH3_OK)
        return lds_ok;
    // Persistent: one workgroup a CU (the tile takes the LDS), at most one a tile.
    const uint32_t tiles = (g.cubes + kSelectRows - 1) / kSelectRows * g.heads;
    const dim3 grid(std::min<uint32_t>(tiles, uint32_t(host::cu_count())));
    hipLaunchKernelGGL(cube_select_kernel, grid, dim3(kSelectThreads), kSelectLds, static_cast<hipStream_t>(stream), g,
                       qc, kc, args->k, args->local, args->out_stride, idx, cnt);
    return host::check_launch();
}

} // extern "C"
