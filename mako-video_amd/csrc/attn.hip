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
//   registers; the contraction order over keys is free, so the V^T fragment's key positions follow it: position p of
//   16-key chunk c is key 32 (c / 2) + 16 (c % 2) + 8 (p % 8 / 4) + 4 (p / 8) + p % 4.
// - K and V tiles (64 rows each, 32 KB) go from global memory straight into LDS (buffer_load ... lds), one tile
//   ahead of the MFMAs when two stages fit. Each lane fetches whichever source chunk its LDS slot holds, so the
//   layouts are free, with one constraint from the address unit: the four lanes of a quad must fetch one aligned
//   64-byte piece (a quad spread over four rows is four accesses, and held the K/V stream to about 16 bytes a clock a
//   CU). K is 256-byte rows whose 16-byte chunks are XOR-swizzled by the row (operand reads of 16 rows hit distinct
//   banks); V is 1 KB blocks of 4 keys whose 64-byte pieces are interleaved, read with ds_read_b64_tr_b16. That
//   instruction hands lane i of a 16-lane group element i & 3 of the 8-byte rows named by lanes (i >> 2) + 4 j,
//   j = 0..3: with lane L naming key (L >> 2)'s columns d0 + 4 (L & 3) .. + 3, lane i receives column d0 + i of four
//   keys, a V^T fragment, with no transpose in registers. Padding slots are fetched from past the buffer's end, which
//   reads zeros.
// - Each cube tile walks its pass list from a rotated start (position rank mod S of S, S the cube workgroups an XCD
//   holds at once, rank the tile's place in its XCD's sequence), wrapping round. The XCD's resident tiles then sweep
//   the key cubes together, so a K/V tile one of them fetches is still in L2 when the others that selected it reach
//   it: the L2 hit rate at 768p went from 11-15% to 29-35% and the L2 misses fell by a fifth, for 2.4% less time
//   (the DMA latency of each tile also bounds the kernel). The first 4 S tiles of an XCD walk from the start of their
//   lists instead: they start in step (the whole first round at once, and the next rounds nearly so), and tiles in
//   step share their K/V tiles by walking together. 5 heads at 768p: 7.37-7.40 ms against 7.96-7.98 rotated from
//   the first tile and 7.73-7.75 never rotated; 40 heads: 54.0-54.4 against 54.2-54.6 (68.1 never rotated).
// - Softmax in base 2 with the scale folded into the exponent. A query's running maximum moves only when a tile
//   raises it by more than 8 (in log2 units): P stays below 2^8, and most tiles skip the rescale of O.
#include "mh3_common.hpp"

#include <algorithm>

namespace mh3 {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr uint32_t kAttnThreads = 128;
constexpr bool kAttnXcd = true;   // map each XCD to a contiguous eighth of every head's query cubes
constexpr bool kAttnSweep = true; // rotate each cube tile's pass list so an XCD's resident tiles sweep the keys together
constexpr uint32_t kAttnInStep = 4; // rounds of an XCD's cube tiles that walk their lists unrotated (1, 2, 8: slower;
                                    // 3, 5, 6: within 1%)
constexpr int kAttnStages = 1;    // K/V stages in LDS (2 overlaps a tile's loads with the previous tile's MFMAs but
                                  // halves the workgroups a CU holds; one stage and two waves a SIMD measured faster)
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
    uint32_t xcd_slices; // cube tiles mapped to XCDs in eighths of each head (needs 8 | cubes and 8 | nd heads)
    uint32_t sweep;      // with xcd_slices: cube workgroups an XCD runs at once (0: pass lists in plain order)
    FastDiv div_plane, div_cw; // c / plane and c / cw by multiply-high: a key tile's cube coordinates cost a few
                               // scalar instructions instead of integer divisions
    float scale_log2;    // score scale times log2(e): softmax in base 2
    const int32_t* order; // or null: head h's j-th cube tile takes query cube order[h cubes + j] (clamped)
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
    const uint32_t ct = p.div_plane.div(c), rem = c - ct * p.plane, cy = p.div_cw.div(rem), cx = rem - cy * p.cw;
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

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef short v4i16 __attribute__((ext_vector_type(4)));

// s_waitcnt that waits for vmcnt == 0 only (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8),
// between scheduling barriers so the compiler moves no memory access across it.
__device__ __forceinline__ void wait_vm0()
{
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0x0070 | 0x0F00);
    __builtin_amdgcn_sched_barrier(0);
}

__device__ __forceinline__ void lds_barrier()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F); // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

constexpr uint32_t kStageBytes = 32768; // K 16 KB, then V 16 KB
constexpr uint32_t kPastEnd = 0x80000000u; // a buffer offset past num_records: the load reads zeros
constexpr uint32_t kRecords = 0x7fffffffu;

__device__ __forceinline__ bool tile_full(const Tile& r)
{
    return r.kind == 0 ? r.lim_t == 64u : (r.kind != 3 && r.lim_t == 4u && r.lim_y == 4u && r.lim_x == 4u);
}

template <int STAGES>
__global__ __launch_bounds__(kAttnThreads, STAGES == 2 ? 1 : 2) void attn_sparse_kernel(AttnParams p)
{
    extern __shared__ __attribute__((aligned(16))) char lds[]; // STAGES x (K stage, V stage)

    const uint32_t tid = threadIdx.x, lane = tid & 63u, n = lane & 31u, hh = lane >> 5;
    // The wave index is uniform: held in a scalar register, the DMA's per-instruction row offsets (soffset) are
    // scalar arithmetic and take no vector registers (which otherwise spill).
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // This workgroup's head and query tile: the dense query tiles of every head first, then the cube tiles. Blocks
    // go to the 8 XCDs round-robin (block b to XCD b % 8); when the counts allow, XCD x takes the x-th eighth of each
    // head's cubes in raster order (or in p.order's), so the workgroups resident on one XCD are query cubes whose
    // pass lists overlap and meet in that XCD's L2, while all XCDs stay on the same head.
    uint32_t h, qt, rank = 0; // rank: the workgroup's place in its XCD's sequence of cube tiles
    {
        const uint32_t b = blockIdx.x, dense_blocks = p.nd * p.heads;
        if (b < dense_blocks) {
            // With the XCD slices, XCD x takes the dense tiles of whole heads (the x-th eighth of them in order), so
            // a head's dense tiles, which walk the same keys in the same order, share each K/V tile in one L2 (5
            // heads at 768p: 7.29-7.32 ms against 7.47-7.48 with a head's tiles dealt over the 8 XCDs).
            const uint32_t l = p.xcd_slices ? (b % 8u) * (dense_blocks / 8u) + b / 8u : b;
            h = l / p.nd;
            qt = l - h * p.nd;
        } else {
            const uint32_t r = b - dense_blocks;
            uint32_t j; // the cube tile's place among its head's
            if (p.xcd_slices) {
                const uint32_t per = p.cubes / 8u, k = r / 8u;
                h = k / per;
                j = (r % 8u) * per + (k - h * per);
                rank = k;
            } else {
                h = r / p.cubes;
                j = r - h * p.cubes;
            }
            qt = p.nd + (p.order ? min(uint32_t(p.order[uint64_t(h) * p.cubes + j]), p.cubes - 1u) : j);
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
    // The pass list is walked from position rot, wrapping round: a workgroup that starts when the XCD's resident ones
    // are a fraction f into their lists starts a fraction f into its own, so the resident tiles sweep the key cubes
    // together and a K/V tile fetched for one is still in that XCD's L2 when the others that selected it reach it.
    // The first kAttnInStep rounds of an XCD's sequence start (nearly) together and walk from position 0 in step.
    // The order only changes the softmax's summation order.
    const bool rotated = !dense_q && p.sweep && rank >= kAttnInStep * p.sweep;
    const uint32_t rot = rotated ? uint32_t(uint64_t(rank % p.sweep) * n_sel / p.sweep) : 0u;
    auto key_tile = [&](uint32_t e) -> uint32_t {
        if (e >= n_sel)
            return e - n_sel;
        if (dense_q)
            return p.nd + e;
        const uint32_t ee = e + rot < n_sel ? e + rot : e + rot - n_sel;
        const int32_t j = list[ee];
        return j >= 0 && uint32_t(j) < p.cubes ? p.nd + uint32_t(j) : kNoTile;
    };

    // DMA source offsets of this wave's 8 K and 8 V instructions. Instruction i = 8 wave + u of the workgroup's 16
    // fills the LDS kilobyte 1024 i with slots 4 i .. 4 i + 3 (K rows, and V's keys); the hardware puts lane L's
    // 16 bytes at position 16 L of it, and each lane fetches whichever source chunk that position holds:
    //   K: position L holds chunk (L % 16) ^ (r % 16) of tile row r = 4 i + L / 16 (256-byte rows whose 16-byte
    //      chunks are XOR-swizzled by the row, so that the MFMA operand reads of 16 rows hit distinct banks);
    //   V: position L holds chunk 4 (L / 16) + L % 4 of key 4 i + (L / 4) % 4 (the four keys' 64-byte pieces
    //      interleaved, so that a transposed read of four keys' 8-byte rows hits distinct banks).
    // Either way every four consecutive lanes fetch one aligned 64-byte piece of one row, which the address unit
    // takes as one access. (Lanes of a quad on four different rows, the layout this replaced, cost four accesses and
    // capped the K/V stream at about 16 bytes a clock a CU.) Slots 4 i .. 4 i + 3 are four consecutive rows in both
    // layouts (in the grid dt = i / 4, dy = i % 4, dx = 0 .. 3), so each offset is a lane constant (voffset) plus a
    // term of i alone (soffset).
    const uint32_t rs2 = uint32_t(p.row_stride) * 2u, gw_rs2 = p.gw * rs2;
    const uint32_t k_row = lane >> 4, k_pos = lane & 15u, v_key = (lane >> 2) & 3u;
    const uint32_t v_lane_off = v_key * rs2 + 16u * (4u * (lane >> 4) + (lane & 3u));
    // Starts tile t's loads into stage st; returns its key mask (bit l: slot l is a token).
    auto dma_tile = [&](uint32_t t, uint32_t st) -> uint64_t {
        const Tile tl = make_tile(p, t);
        const uint64_t row_bytes = (tl.kind == 3 ? 0ull : tl.base) * p.row_stride * 2ull;
        const __amdgpu_buffer_rsrc_t rk =
            __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<char*>(const_cast<uint16_t*>(kh)) + row_bytes, 0,
                                              int(kRecords), kRsrcFlags);
        const __amdgpu_buffer_rsrc_t rv =
            __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<char*>(const_cast<uint16_t*>(vh)) + row_bytes, 0,
                                              int(kRecords), kRsrcFlags);
        char* ks = lds + st * kStageBytes;
        char* vs = ks + 16384;
        const bool full = tile_full(tl), grid = tl.kind == 1;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const uint32_t i = 8u * wave + uint32_t(u);
            const uint32_t s_i = grid ? ((i >> 2) * p.gh + (i & 3u)) * gw_rs2 : 4u * i * rs2; // slot 4 i's row
            // K chunk (L % 16) ^ (r % 16), r % 16 = 4 (i % 4) + L / 16
            uint32_t ko = k_row * rs2 + 16u * (k_pos ^ (4u * (i & 3u) + k_row)), vo = v_lane_off;
            if (!full) {
                ko = slot_token(tl, 4u * i + k_row) ? ko : kPastEnd;
                vo = slot_token(tl, 4u * i + v_key) ? vo : kPastEnd;
            }
            const int so = int(__builtin_amdgcn_readfirstlane(s_i));
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_ptr_t)(ks + 1024u * i), 16, ko, so, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_ptr_t)(vs + 1024u * i), 16, vo, so, 0, 0);
        }
        return full ? ~0ull : __ballot(slot_token(tl, lane));
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
    // Fragment addresses: lane constants, and immediates or (K's swizzle) an XOR with 32 dc.
    //   K: row 32 b + n, chunk 2 dc + hh at 8192 b + 256 n + 16 ((2 dc + hh) ^ (n % 16)) = 8192 b + (k_lane ^ 32 dc).
    //   V: key k, column d of a 4-key block at 256 (d / 32) + 64 k + 2 (d % 32); lane L of 16-lane group grp names
    //      key L / 4's columns d0 + 4 (L % 4) .. + 3, d0 = 32 db + 16 (grp % 2), of the block 2 (8 b + 4 g) + grp / 2.
    const uint32_t k_lane = 256u * n + 16u * (hh ^ (n & 15u));
    const uint32_t L = lane & 15u, grp = lane >> 4;
    const uint32_t v_lane = 1024u * (grp >> 1) + 32u * (grp & 1u) + 64u * (L >> 2) + 8u * (L & 3u);

    uint64_t mask = n_tiles ? dma_tile(key_tile(0), 0) : 0ull;
    for (uint32_t e = 0; e < n_tiles; ++e) {
        const uint32_t st = STAGES == 2 ? (e & 1u) : 0u;
        wait_vm0();
        lds_barrier(); // tile e is in LDS for every wave; every wave is done with tile e - 1
        uint64_t mask_next = 0;
        if (STAGES == 2 && e + 1 < n_tiles)
            mask_next = dma_tile(key_tile(e + 1), st ^ 1u);
        const char* ks = lds + st * kStageBytes;
        const char* vs = lds + st * kStageBytes + 16384u + v_lane;

        // S^T: lane (n, hh), element i of block b is key 32 b + 8 (i / 4) + 4 hh + i % 4 of query n.
        floatx16 s[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
#pragma unroll
            for (int i = 0; i < 16; ++i)
                s[b][i] = 0.0f;
#pragma unroll
            for (int dc = 0; dc < 8; ++dc) {
                const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(ks + 8192u * b + (k_lane ^ (32u * dc)));
                s[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[dc], s[b], 0, 0, 0);
            }
        }
        // Online softmax in base 2: padding keys score -inf; the maximum moves only when it rises by more than 8.
        float mt = -__builtin_inff();
        if (mask != ~0ull) {
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const uint32_t key = 32u * b + 8u * (i >> 2) + 4u * hh + (i & 3);
                    s[b][i] = (mask >> key) & 1ull ? s[b][i] : -__builtin_inff();
                }
        }
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int i = 0; i < 16; ++i)
                mt = fmaxf(mt, s[b][i]);
        mt = fmaxf(mt, __shfl_xor(mt, 32, kWave)) * p.scale_log2;
        if (__ballot(mt > m_run + 8.0f)) {
            const float m_new = fmaxf(m_run, mt);
            const float alpha = m_run == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (int b = 0; b < 4; ++b)
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    o[b][i] *= alpha;
        }
        const float m_ref = m_run == -__builtin_inff() ? 0.0f : m_run;
        float ps = 0.0f;
        uint32_t pw[2][8];
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int i = 0; i < 16; i += 2) {
                const float p0 = __builtin_amdgcn_exp2f(fmaf(s[b][i], p.scale_log2, -m_ref));
                const float p1 = __builtin_amdgcn_exp2f(fmaf(s[b][i + 1], p.scale_log2, -m_ref));
                ps += p0 + p1;
                pw[b][i >> 1] = pack_bf16(p0, p1);
            }
        l_run += ps;
        // O^T (d 32 db + 8 (i / 4) + 4 hh + i % 4 of query n) += V^T P^T; P^T chunk c = 2 b + g is accumulator
        // elements 8 g .. + 7 of block b; its V^T fragment is two transposed reads (positions 0-3, 4-7 of the half).
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int b = c >> 1, g = c & 1;
            const bf16x8_t pf = __builtin_bit_cast(bf16x8_t, uint4{pw[b][4 * g], pw[b][4 * g + 1], pw[b][4 * g + 2],
                                                                   pw[b][4 * g + 3]});
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const uint32_t off = 1024u * (8u * b + 4u * g) + 256u * db;
                const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((v4i16 __attribute__((address_space(3)))*)(
                    const_cast<char*>(vs) + off));
                const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((v4i16 __attribute__((address_space(3)))*)(
                    const_cast<char*>(vs) + off + 2048u));
                const bf16x8_t a = __builtin_bit_cast(
                    bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pf, o[db], 0, 0, 0);
            }
        }
        if (STAGES == 1) {
            lds_barrier(); // every wave is done with the stage before it is refilled
            if (e + 1 < n_tiles)
                mask_next = dma_tile(key_tile(e + 1), 0);
        }
        mask = mask_next;
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

namespace {

// order: null for the plain entry point; `ordered`: the ordered one, which needs it.
int launch_attn(const MH3AttnArgs* args, const uint16_t* q, const uint16_t* k, const uint16_t* v, const int32_t* idx,
                const int32_t* cnt, const int32_t* order, bool ordered, uint16_t* out, mh3_stream_t stream)
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
    if (!q || !k || !v || !idx || !cnt || !out || (ordered && !order))
        return MH3_ERR_POINTER;
    if (out == q || out == k || out == v)
        return MH3_ERR_PARAM;
    if (c.row_stride % 8 != 0 || c.head_stride % 8 != 0 || c.row_stride < 128 || !host::aligned16(q) ||
        !host::aligned16(k) || !host::aligned16(v) || !host::aligned16(out) ||
        reinterpret_cast<uintptr_t>(order) % 4u != 0u)
        return MH3_ERR_ALIGN;
    AttnParams p{};
    p.gt = c.grid_t, p.gh = c.grid_h, p.gw = c.grid_w;
    p.ch = (p.gh + 3u) / 4u, p.cw = (p.gw + 3u) / 4u;
    const uint64_t cth = (p.gt + 3u) / 4u, plane = uint64_t(p.ch) * p.cw, cubes = cth * plane;
    const uint64_t nd = (uint64_t(args->n_dense) + 63u) / 64u;
    // Row offsets within a tile, in bytes, stay below 2^31 (the DMA's 32-bit buffer offsets).
    const uint64_t tile_rows = c.layout == MH3_CUBES_GRID ? (3ull * p.gh + 4u) * p.gw : 64u;
    if (cubes * c.heads >= (1ull << 31) || (cubes + nd) * c.heads >= (1ull << 31) ||
        std::max<uint64_t>(tile_rows, 64u) * c.row_stride * 2u >= (1ull << 31))
        return MH3_ERR_SHAPE;
    // The dense rows may not overlap the video rows.
    const uint64_t video = c.layout == MH3_CUBES_GRID ? uint64_t(p.gt) * p.gh * p.gw : 64ull * cubes;
    if (args->n_dense && args->dense_row0 < c.row0 + video && c.row0 < args->dense_row0 + args->n_dense)
        return MH3_ERR_PARAM;
    // Nor may out overlap q, k, v or the pass lists, which other workgroups are still reading (each starts by reading
    // its own query tile and list): q, k, v and out each span from the array's start to the last head's last row
    // (video or dense) that the call reads or writes.
    const uint64_t last_row =
        std::max<uint64_t>(c.row0 + video, args->n_dense ? args->dense_row0 + args->n_dense : 0u) - 1u;
    const uint64_t span = ((uint64_t(c.heads) - 1u) * c.head_stride + last_row * c.row_stride + 128u) * 2u;
    {
        const host::Span in[] = {{q, span},
                                 {k, span},
                                 {v, span},
                                 {idx, uint64_t(c.heads) * cubes * c.out_stride * 4u},
                                 {cnt, uint64_t(c.heads) * cubes * 4u},
                                 {order, uint64_t(c.heads) * cubes * 4u}};
        const host::Span o[] = {{out, span}};
        if (host::any_overlap(in, o))
            return MH3_ERR_PARAM;
    }
    p.q = q, p.k = k, p.v = v, p.out = out, p.idx = idx, p.cnt = cnt, p.order = order;
    p.row0 = c.row0, p.dense_row0 = args->dense_row0, p.head_stride = c.head_stride, p.row_stride = c.row_stride;
    p.plane = uint32_t(plane), p.cubes = uint32_t(cubes), p.heads = c.heads, p.n_dense = args->n_dense;
    p.div_plane = FastDiv::make(p.plane);
    p.div_cw = FastDiv::make(p.cw);
    p.nd = uint32_t(nd), p.layout = c.layout, p.out_stride = c.out_stride;
    p.xcd_slices = kAttnXcd && cubes % 8u == 0 && (nd * c.heads) % 8u == 0 ? 1u : 0u;
    const float scale = args->scale > 0.0f ? args->scale : 0.08838834764831845f; // 1 / sqrt(128)
    p.scale_log2 = scale * 1.4426950408889634f;
    const uint64_t blocks = (cubes + nd) * c.heads;
    constexpr int kStages = kAttnStages;
    const void* kern = reinterpret_cast<const void*>(&attn_sparse_kernel<kStages>);
    const size_t lds = size_t(kStages) * kStageBytes;
    if (const hipError_t e = host::allow_dynamic_lds(kern, lds); e != hipSuccess)
        return host::hip_error(e);
    if (kAttnSweep && p.xcd_slices) {
        int per_cu = 0;
        if (const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, int(kAttnThreads), lds);
            e != hipSuccess)
            return host::hip_error(e);
        // The sweep period: the cube workgroups an XCD holds at once (half or twice that measured slower).
        p.sweep = uint32_t(uint64_t(std::max(per_cu, 1)) * uint32_t(host::cu_count()) / 8u);
    }
    hipLaunchKernelGGL(attn_sparse_kernel<kStages>, dim3(uint32_t(blocks)), dim3(kAttnThreads), lds,
                       static_cast<hipStream_t>(stream), p);
    return host::check_launch();
}

} // namespace

extern "C" int mh3_flash_attn_sparse_128(const MH3AttnArgs* args, const uint16_t* q, const uint16_t* k,
                                         const uint16_t* v, const int32_t* idx, const int32_t* cnt, uint16_t* out,
                                         mh3_stream_t stream)
{
    return launch_attn(args, q, k, v, idx, cnt, nullptr, false, out, stream);
}

extern "C" int mh3_flash_attn_sparse_128_ordered(const MH3AttnArgs* args, const uint16_t* q, const uint16_t* k,
                                                 const uint16_t* v, const int32_t* idx, const int32_t* cnt,
                                                 const int32_t* order, uint16_t* out, mh3_stream_t stream)
{
    return launch_attn(args, q, k, v, idx, cnt, order, true, out, stream);
}
