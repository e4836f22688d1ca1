// `flash_attn_sparse_128`: flash attention over the sparse selector's pass lists, head_dim 128, bf16 in and out.
// Reference semantics: the mako-common kernel of this name, described in docs/architecture.md:123-130 and
// docs/performance.md:162-181. The queries of cube i (head h) attend the tokens of the cubes idx[h][i][0 .. cnt) and
// every dense row (text, keyframe, audio); a dense row's query attends every token; padding slots of cubes at the
// grid's edge are neither keys nor outputs.
//
// Design (gfx950, v_mfma_f32_32x32x16_bf16):
// - The reference gathers each head's rows into cube order (heads_partial with the cube map), attends, and writes the
//   outputs back to the model's rows. Here the kernel reads q, k, v where they lie, in the model's order (the grid
//   layout) or already gathered, through the same cube arithmetic as the selector, and writes the output rows in
//   place: no gather or scatter pass.
// - A workgroup is one (head, 64-row query tile): two waves of 32 queries. Tiles are numbered dense runs of 64 first,
//   then one per cube; the dense query tiles of every head come first in the grid (they attend every token, ten
//   times a cube tile's work), then the cube tiles head by head, so one head's K and V stay hot in the MALL.
// - Scores are computed transposed, S^T = K Q^T (keys as the MFMA's M, queries as N): the accumulator puts all of
//   a query's keys in one lane and its lane + 32 twin, so the softmax's row maximum and sum are in-lane plus one
//   cross-half exchange, and the rescale of a query's output is one factor per lane.
// - The output is also transposed, O^T += V^T P^T. P^T is the B operand as the score accumulator leaves it in
//   registers; the contraction order over keys is free, so V^T is staged in LDS with its key positions in that
//   order: position p of 16-key chunk c holds key 32 (c / 2) + 16 (c % 2) + 8 (p % 8 / 4) + 4 (p / 8) + p % 4.
// - Each key tile (64 rows of K and V, 32 KB) is loaded by the 128 threads into registers, then written to LDS: K
//   row-major with its 16-byte chunks XOR-swizzled by the row (conflict-free fragment reads), V as 8 x 8 blocks
//   transposed in registers (v_perm) into V^T rows, chunks swizzled by d / 2. The loads' registers are free again
//   during the MFMAs, which keeps a wave within 256 registers: two waves a SIMD, four workgroups a CU, and one
//   workgroup's loads overlap the others' MFMAs.
#include "mh3_common.hpp"

namespace mh3 {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr uint32_t kAttnThreads = 128;
constexpr uint32_t kNoTile = 0xffffffffu;

struct AttnParams {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    uint16_t* out;
    const int32_t* idx;
    const int32_t* cnt;
    uint64_t row0, dense_row0, head_stride, row_stride;
    uint32_t gt, gh, gw, ch, cw, plane; // plane = ch * cw cubes a frame group
    uint32_t cubes, heads, n_dense, nd; // nd: dense tiles of 64 rows
    uint32_t layout, out_stride;
    float scale_log2; // score scale times log2(e): softmax in base 2
};

// A tile of 64 slots. kind 0: dense run (slot l is row base + l, a token while l < lim_t); 1: cube in the grid layout
// (slot (dt, dy, dx) is row base + (dt gh + dy) gw + dx); 2: cube gathered (row base + l); a cube slot is a token while
// dt < lim_t, dy < lim_y, dx < lim_x. kind 3: no tile (an index outside the cubes): no tokens.
struct Tile {
    uint64_t base;
    uint32_t kind, lim_t, lim_y, lim_x;
};

__device__ __forceinline__ Tile make_tile(const AttnParams& p, uint32_t t)
{
    Tile r{0, 3u, 0, 0, 0};
    if (t == kNoTile)
        return r;
    if (t < p.nd) {
        r.kind = 0;
        r.base = p.dense_row0 + 64ull * t;
        r.lim_t = min(64u, p.n_dense - 64u * t);
        return r;
    }
    const uint32_t c = t - p.nd;
    const uint32_t ct = c / p.plane, cy = c / p.cw % p.ch, cx = c % p.cw;
    r.lim_t = min(4u, p.gt - 4u * ct);
    r.lim_y = min(4u, p.gh - 4u * cy);
    r.lim_x = min(4u, p.gw - 4u * cx);
    if (p.layout == MH3_CUBES_GRID) {
        r.kind = 1;
        r.base = p.row0 + (uint64_t(4u * ct) * p.gh + 4u * cy) * p.gw + 4u * cx;
    } else {
        r.kind = 2;
        r.base = p.row0 + 64ull * c;
    }
    return r;
}

__device__ __forceinline__ bool slot_token(const Tile& r, uint32_t l)
{
    if (r.kind == 0)
        return l < r.lim_t;
    if (r.kind == 3)
        return false;
    return (l >> 4) < r.lim_t && ((l >> 2) & 3u) < r.lim_y && (l & 3u) < r.lim_x;
}

// The slot's grid-layout offset (dt gh + dy) gw + dx; below 2^32 (the host checks 4 gh gw < 2^32).
__device__ __forceinline__ uint32_t grid_offset(const AttnParams& p, uint32_t l)
{
    return ((l >> 4) * p.gh + ((l >> 2) & 3u)) * p.gw + (l & 3u);
}

__device__ __forceinline__ uint64_t slot_row(const AttnParams& p, const Tile& r, uint32_t l)
{
    return r.base + (r.kind == 1 ? uint64_t(grid_offset(p, l)) : uint64_t(l));
}

__device__ __forceinline__ uint4 load16(const uint16_t* p)
{
    return *reinterpret_cast<const uint4*>(p);
}

// The key whose V column sits at position j (0..7) of position group pg (0..7: 16-key chunk pg / 2, half pg % 2).
__device__ __forceinline__ uint32_t vt_key(uint32_t pg, uint32_t j)
{
    return 32u * (pg >> 2) + 16u * ((pg >> 1) & 1u) + 8u * (j >> 2) + 4u * (pg & 1u) + (j & 3u);
}

__global__ __launch_bounds__(kAttnThreads, 2) void attn_sparse_kernel(AttnParams p)
{
    __shared__ uint4 lds_k[64 * 16]; // [key][16-byte chunk]; chunk c of key r at c ^ (r & 15)
    __shared__ uint4 lds_vt[128 * 8]; // [d][8 chunks of 8 key positions]; chunk c of row d at c ^ ((d >> 1) & 7)

    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6, n = lane & 31u, hh = lane >> 5;

    // This workgroup's head and query tile.
    uint32_t h, qt;
    {
        const uint32_t b = blockIdx.x, dense_blocks = p.nd * p.heads;
        if (b < dense_blocks) {
            h = b / p.nd;
            qt = b - h * p.nd;
        } else {
            const uint32_t r = b - dense_blocks;
            h = r / p.cubes;
            qt = p.nd + (r - h * p.cubes);
        }
    }
    const uint64_t hoff = uint64_t(h) * p.head_stride;
    const uint16_t* qh = p.q + hoff;
    const uint16_t* kh = p.k + hoff;
    const uint16_t* vh = p.v + hoff;

    // The key tiles: a dense query tile takes every cube then the dense runs; cube i its pass list then the dense runs.
    const bool dense_q = qt < p.nd;
    uint32_t n_sel = p.cubes;
    const int32_t* list = nullptr;
    if (!dense_q) {
        const uint64_t item = uint64_t(h) * p.cubes + (qt - p.nd);
        list = p.idx + item * p.out_stride;
        n_sel = uint32_t(min(max(p.cnt[item], 0), int32_t(p.out_stride)));
    }
    const uint32_t n_tiles = n_sel + p.nd;
    auto key_tile = [&](uint32_t e) -> uint32_t {
        if (e >= n_sel)
            return e - n_sel;
        if (dense_q)
            return p.nd + e;
        const int32_t j = list[e];
        return j >= 0 && uint32_t(j) < p.cubes ? p.nd + uint32_t(j) : kNoTile;
    };

    // Loader slots, fixed for the whole kernel: K chunk kc of rows kr(jj) = tid / 16 + 8 jj; V columns 8 dg .. + 7 of
    // the keys vt_key(pg, j).
    const uint32_t kc = tid & 15u, pg = tid >> 4, dg = tid & 15u;
    uint4 kreg[8], vreg[8];
    uint64_t mask_next = 0;
    auto load_tile = [&](uint32_t t) {
        const Tile tl = make_tile(p, t);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t ks = (tid >> 4) + 8u * j, vs = vt_key(pg, j);
            kreg[j] = slot_token(tl, ks) ? load16(kh + slot_row(p, tl, ks) * p.row_stride + kc * 8u)
                                         : uint4{0u, 0u, 0u, 0u};
            vreg[j] = slot_token(tl, vs) ? load16(vh + slot_row(p, tl, vs) * p.row_stride + dg * 8u)
                                         : uint4{0u, 0u, 0u, 0u};
        }
        mask_next = __ballot(slot_token(tl, lane));
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t r = (tid >> 4) + 8u * j;
            lds_k[r * 16u + (kc ^ (r & 15u))] = kreg[j];
        }
        // 8 keys x 8 d to 8 d x 8 keys: output dword m of d i pairs keys 2m (low half) and 2m + 1 (high half).
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t sel = (i & 1) ? 0x07060302u : 0x05040100u;
            uint32_t w[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const uint4 a = vreg[2 * m], b = vreg[2 * m + 1];
                const uint32_t wa = (i >> 1) == 0 ? a.x : (i >> 1) == 1 ? a.y : (i >> 1) == 2 ? a.z : a.w;
                const uint32_t wb = (i >> 1) == 0 ? b.x : (i >> 1) == 1 ? b.y : (i >> 1) == 2 ? b.z : b.w;
                w[m] = __builtin_amdgcn_perm(wb, wa, sel);
            }
            const uint32_t d = 8u * dg + uint32_t(i);
            lds_vt[d * 8u + (pg ^ ((d >> 1) & 7u))] = uint4{w[0], w[1], w[2], w[3]};
        }
    };

    // This wave's 32 queries as the B operand of S^T = K Q^T: lane (n, hh) holds d 16 dc + 8 hh .. + 7 of query n.
    const Tile qtile = make_tile(p, qt);
    const uint32_t qslot = 32u * wave + n;
    const bool q_token = slot_token(qtile, qslot);
    const uint64_t qrow = slot_row(p, qtile, qslot);
    bf16x8_t qf[8];
#pragma unroll
    for (int dc = 0; dc < 8; ++dc) {
        const uint4 t = q_token ? load16(qh + qrow * p.row_stride + 16u * dc + 8u * hh) : uint4{0u, 0u, 0u, 0u};
        qf[dc] = __builtin_bit_cast(bf16x8_t, t);
    }

    floatx16 o[4];
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int e = 0; e < 16; ++e)
            o[b][e] = 0.0f;
    float m_run = -__builtin_inff(), l_run = 0.0f;

    for (uint32_t e = 0; e < n_tiles; ++e) {
        load_tile(key_tile(e));
        __syncthreads(); // every wave is done with the previous tile's LDS
        store_tile();
        const uint64_t mask = mask_next;
        __syncthreads();

        // The tile's two 32-key blocks in turn, each an online-softmax step (fewer live registers than one step of
        // 64 keys). S^T block b: lane (n, hh), element i is key 32 b + 8 (i / 4) + 4 hh + i % 4 of query n.
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            floatx16 s;
#pragma unroll
            for (int i = 0; i < 16; ++i)
                s[i] = 0.0f;
            const uint32_t r = 32u * b + n;
#pragma unroll
            for (int dc = 0; dc < 8; ++dc) {
                const uint4 a = lds_k[r * 16u + ((2u * dc + hh) ^ (r & 15u))];
                s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), qf[dc], s, 0, 0, 0);
            }
            // Softmax in base 2; padding keys score -inf.
            float mt = -__builtin_inff();
            const uint32_t bmask = uint32_t(mask >> (32 * b));
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float x = s[i] * p.scale_log2;
                if (bmask != ~0u)
                    x = (bmask >> (8u * (i >> 2) + 4u * hh + (i & 3))) & 1u ? x : -__builtin_inff();
                s[i] = x;
                mt = fmaxf(mt, x);
            }
            mt = fmaxf(mt, __shfl_xor(mt, 32, kWave));
            const float m_new = fmaxf(m_run, mt);
            const float m_ref = m_new == -__builtin_inff() ? 0.0f : m_new;
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_ref);
            m_run = m_new;
            float ps = 0.0f;
            uint32_t pw[8];
#pragma unroll
            for (int i = 0; i < 16; i += 2) {
                const float p0 = __builtin_amdgcn_exp2f(s[i] - m_ref);
                const float p1 = __builtin_amdgcn_exp2f(s[i + 1] - m_ref);
                ps += p0 + p1;
                pw[i >> 1] = pack_bf16(p0, p1);
            }
            l_run = l_run * alpha + ps;
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    o[db][i] *= alpha;
            // P^T chunk c = 2 b + g holds accumulator elements 8 g .. 8 g + 7 of this block.
            const bf16x8_t pf0 = __builtin_bit_cast(bf16x8_t, uint4{pw[0], pw[1], pw[2], pw[3]});
            const bf16x8_t pf1 = __builtin_bit_cast(bf16x8_t, uint4{pw[4], pw[5], pw[6], pw[7]});
            // O^T (d 32 db + 8 (i / 4) + 4 hh + i % 4 of query n) += V^T P^T over the block's two 16-key chunks.
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const uint32_t d = 32u * db + n, sw = (d >> 1) & 7u;
                const uint4 a0 = lds_vt[d * 8u + ((4u * b + hh) ^ sw)];
                const uint4 a1 = lds_vt[d * 8u + ((4u * b + 2u + hh) ^ sw)];
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a0), pf0, o[db], 0, 0, 0);
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a1), pf1, o[db], 0, 0, 0);
            }
        }
    }

    // Normalize and write the query rows (a gathered cube's padding slots get zeros; other non-tokens nothing).
    const float l_tot = l_run + __shfl_xor(l_run, 32, kWave);
    const float inv = q_token && l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    if (q_token || qtile.kind == 2) {
        uint16_t* orow = p.out + hoff + qrow * p.row_stride;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const uint32_t d0 = 32u * db + 8u * g + 4u * hh;
                const uint2 w = q_token ? uint2{pack_bf16(o[db][4 * g] * inv, o[db][4 * g + 1] * inv),
                                                pack_bf16(o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv)}
                                        : uint2{0u, 0u}; // +0, not the sign of 0 * o
                *reinterpret_cast<uint2*>(orow + d0) = w;
            }
    }
}

} // namespace
} // namespace mh3

extern "C" int mh3_flash_attn_sparse_128(const MH3AttnArgs* args, const uint16_t* q, const uint16_t* k,
                                         const uint16_t* v, const int32_t* idx, const int32_t* cnt, uint16_t* out,
                                         mh3_stream_t stream)
{
    using namespace mh3;
    if (!args)
        return MH3_ERR_POINTER;
    const MH3CubeArgs& c = args->cubes;
    if (c.layout != MH3_CUBES_GRID && c.layout != MH3_CUBES_GATHERED)
        return MH3_ERR_PARAM;
    if (c.heads == 0 || c.grid_t == 0 || c.grid_h == 0 || c.grid_w == 0 || c.head_dim == 0 || c.out_stride == 0)
        return MH3_ERR_SHAPE;
    if (c.head_dim != 128)
        return MH3_ERR_UNSUPPORTED;
    if (!(args->scale >= 0.0f) || args->scale == __builtin_inff())
        return MH3_ERR_PARAM;
    if (!q || !k || !v || !idx || !cnt || !out)
        return MH3_ERR_POINTER;
    if (out == q || out == k || out == v)
        return MH3_ERR_PARAM;
    if (c.row_stride % 8 != 0 || c.head_stride % 8 != 0 || c.row_stride < 128 || !host::aligned16(q) ||
        !host::aligned16(k) || !host::aligned16(v) || !host::aligned16(out))
        return MH3_ERR_ALIGN;
    AttnParams p{};
    p.gt = c.grid_t, p.gh = c.grid_h, p.gw = c.grid_w;
    p.ch = (p.gh + 3u) / 4u, p.cw = (p.gw + 3u) / 4u;
    const uint64_t cth = (p.gt + 3u) / 4u, plane = uint64_t(p.ch) * p.cw, cubes = cth * plane;
    const uint64_t nd = (uint64_t(args->n_dense) + 63u) / 64u;
    if (cubes * c.heads >= (1ull << 31) || (cubes + nd) * c.heads >= (1ull << 31) ||
        4ull * p.gh * p.gw >= (1ull << 32))
        return MH3_ERR_SHAPE;
    // The dense rows may not overlap the video rows.
    const uint64_t video = c.layout == MH3_CUBES_GRID ? uint64_t(p.gt) * p.gh * p.gw : 64ull * cubes;
    if (args->n_dense && args->dense_row0 < c.row0 + video && c.row0 < args->dense_row0 + args->n_dense)
        return MH3_ERR_PARAM;
    p.q = q, p.k = k, p.v = v, p.out = out, p.idx = idx, p.cnt = cnt;
    p.row0 = c.row0, p.dense_row0 = args->dense_row0, p.head_stride = c.head_stride, p.row_stride = c.row_stride;
    p.plane = uint32_t(plane), p.cubes = uint32_t(cubes), p.heads = c.heads, p.n_dense = args->n_dense;
    p.nd = uint32_t(nd), p.layout = c.layout, p.out_stride = c.out_stride;
    const float scale = args->scale > 0.0f ? args->scale : 0.08838834764831845f; // 1 / sqrt(128)
    p.scale_log2 = scale * 1.4426950408889634f;
    const uint64_t blocks = (cubes + nd) * c.heads;
    hipLaunchKernelGGL(attn_sparse_kernel, dim3(uint32_t(blocks)), dim3(kAttnThreads), 0,
                       static_cast<hipStream_t>(stream), p);
    return host::check_launch();
}
