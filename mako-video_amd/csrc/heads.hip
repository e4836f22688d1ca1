// `heads_partial`: the step between the QKV GEMM and attention. Per model row and head, q and k get an RMS norm over
// the head's 128 values and the rotary positions on the first `rot` of them; v is copied; the results go out as head
// tiles, optionally gathered through the cube map into the order the sparse selector and flash_attn_sparse_128 read.
// Reference semantics: the mako-common kernel of this name, described in docs/architecture.md:35-38,61-63,123-125
// ("RMS norms per head, rotary positions"; "the head tiles are gathered through that map ... padding rows zero").
//
// Design (gfx950): the op reads every element of q, k and v once and writes it once (4 bytes an element), so it is
// HBM-bound. A head vector (128 bf16 = 256 bytes) belongs to one 16-lane DPP row, 16 bytes a lane, so the sum of
// squares is a DPP row reduction with no LDS and no barrier.
// - A workgroup of 512 threads is 32 such groups. It takes whole rows, enough that their head vectors fill about 96
//   slots and at least two rows, and each group has up to 3 head vectors in flight (loads first, then the arithmetic
//   and the stores).
//   Consecutive groups take consecutive head vectors of a row, so a wave's load covers 1 KB of contiguous qkv.
// - The rotary pairs value i with i + rot / 2: lane p (values 8 p .. 8 p + 7) pairs with lane p +- rot / 16 of the
//   same group; the partner's raw bf16 words come over by ds_bpermute, and each lane normalizes both halves itself
//   (the norm factor is the group's).
// - The workgroup stages the two norm weight vectors and its rows' cos / sin tables in LDS once.
// - A padding slot of the cube map writes zeros and reads nothing.
// mh3_heads_partial_pool adds cube_pool to the same pass (heads_pool_kernel, a workgroup per cube): the selector's
// cube means come from the values as they are stored, so q and k are not read back from HBM.
#include "mh3_common.hpp"

namespace mh3 {
namespace {

constexpr uint32_t kHeadsThreads = 512;
constexpr uint32_t kGroups = kHeadsThreads / 16u; // one head vector a 16-lane group
constexpr int kHeadsU = 3;                        // head vectors a group has in flight
constexpr uint32_t kSlots = kGroups * kHeadsU;    // head vectors a workgroup pass
// Dynamic LDS of at least this much, so three workgroups (24 waves, three rows of qkv at 40 heads) share a CU: that
// streamed 1-3% faster than the 4 to 6 the registers allow, and two or one were slower (at 768p, alternating runs).
constexpr size_t kHeadsLdsFloor = 41 * 1024;

struct HeadsParams {
    const uint16_t* qkv;
    const float* qw;
    const float* kw;
    const float* cos_t;
    const float* sin_t;
    const int32_t* map;
    uint16_t* out[3];
    uint64_t qkv_stride, ohs, ors;
    uint32_t rows, model_rows, heads, half, per_row, rows_per_block;
    uint32_t row_begin; // first output row of the launch; it covers rows row_begin .. rows - 1
    FastDiv div_row, div_heads;
    float eps;
};

// A lane's part in the rotary: lane p of a 16-lane group (values 8 p .. 8 p + 7) pairs with lane p +- rot / 16; pd is
// the partner's first value and ci the cos / sin column of the lane's first value.
struct RotLane {
    uint32_t partner, pd, ci;
    bool rotating, first_half;
};
__device__ __forceinline__ RotLane rot_lane(uint32_t lane, uint32_t half)
{
    const uint32_t part = lane & 15u, hv = half / 8u; // lanes a half of the rotating values spans
    RotLane r;
    r.rotating = part < 2u * hv;
    r.first_half = part < hv;
    const uint32_t pp = r.rotating ? (r.first_half ? part + hv : part - hv) : part;
    r.partner = (lane & ~15u) | pp;
    r.pd = 8u * pp;
    r.ci = r.rotating ? 8u * part - (r.first_half ? 0u : half) : 0u;
    return r;
}

// One head vector of a 16-lane group, 16 bytes a lane: q or k (kind 0 or 1) normalized with its weights wk[128] and
// rotated with the row's tables c[] and s[] (already offset by the lane's column), or v (kind 2) passed through. Every
// lane of the wave must call it (the partner exchange is a wave-wide ds_bpermute). wk, c and s are 16-byte aligned
// LDS; the tables are read by every lane (a lane that does not rotate reads column 0 and keeps its values).
__device__ __forceinline__ uint4 head_vector(const uint4 raw, uint32_t kind, const float* wk, const float* c,
                                             const float* s, const RotLane& rl, uint32_t part, float eps)
{
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
    // The partner's words (every lane takes part in the exchange; lanes without a partner get their own).
    uint32_t pw[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
        pw[e] = uint32_t(__builtin_amdgcn_ds_bpermute(int(rl.partner << 2), int(w[e])));
    float x[8], xp[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        x[2 * e] = bf16_lo(w[e]), x[2 * e + 1] = bf16_hi(w[e]);
        xp[2 * e] = bf16_lo(pw[e]), xp[2 * e + 1] = bf16_hi(pw[e]);
    }
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e)
        ss = fmaf(x[e], x[e], ss);
    ss = row16_sum(ss);
    if (kind >= 2u)
        return raw;
    // The hardware reciprocal square root (within 1 ulp; one instruction where 1 / sqrtf is some 25).
    const float inv = __builtin_amdgcn_rsqf(fmaf(ss, 1.0f / 128.0f, eps));
    float wm[8], wp[8], cv[8], sv[8];
    auto ld8 = [](const float* src, float (&dst)[8]) {
        const float4 lo = reinterpret_cast<const float4*>(src)[0], hi = reinterpret_cast<const float4*>(src)[1];
        dst[0] = lo.x, dst[1] = lo.y, dst[2] = lo.z, dst[3] = lo.w, dst[4] = hi.x, dst[5] = hi.y, dst[6] = hi.z,
        dst[7] = hi.w;
    };
    ld8(wk + 8u * part, wm);
    ld8(wk + rl.pd, wp);
    ld8(c, cv);
    ld8(s, sv);
    // (a, b) -> (a cos - b sin, b cos + a sin): the first half's partner term enters negated.
    const float sg = rl.first_half ? -1.0f : 1.0f;
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float a = x[e] * inv * wm[e];
        const float b = xp[e] * inv * wp[e];
        y[e] = rl.rotating ? fmaf(a, cv[e], sg * b * sv[e]) : a;
    }
    return uint4{pack_bf16(y[0], y[1]), pack_bf16(y[2], y[3]), pack_bf16(y[4], y[5]), pack_bf16(y[6], y[7])};
}

// The workgroup's norm weights into LDS wt[256] (q, then k; NULL weights are 1).
__device__ __forceinline__ void stage_weights(float* wt, const float* qw, const float* kw, uint32_t tid,
                                              uint32_t threads)
{
    for (uint32_t i = tid; i < 256u; i += threads) {
        const float* w = i < 128u ? qw : kw;
        wt[i] = w ? w[i & 127u] : 1.0f;
    }
}

__global__ __launch_bounds__(kHeadsThreads) void heads_kernel(HeadsParams p)
{
    // LDS: the norm weights w [2][128] (q, then k); the rows' model rows src [rows_per_block] (-1: padding); their
    // cos and sin tables [rows_per_block][half] each.
    extern __shared__ float lds[];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, part = lane & 15u, group = tid >> 4;
    const uint32_t r0 = p.row_begin + blockIdx.x * p.rows_per_block;
    const uint32_t nr = min(p.rows_per_block, p.rows - r0);
    float* wt = lds;
    int32_t* srcs = reinterpret_cast<int32_t*>(lds + 256);
    float* ct = lds + 256 + ((p.rows_per_block + 3u) & ~3u); // 16-byte aligned
    float* st = ct + p.rows_per_block * p.half;
    stage_weights(wt, p.qw, p.kw, tid, kHeadsThreads);
    // A map entry outside [0, model_rows) is a padding slot.
    auto src_of = [&](uint32_t r) -> int32_t {
        const int32_t m = p.map ? p.map[r0 + r] : int32_t(r0 + r);
        return m >= 0 && uint32_t(m) < p.model_rows ? m : -1;
    };
    for (uint32_t i = tid; i < nr; i += kHeadsThreads)
        srcs[i] = src_of(i);
    for (uint32_t i = tid; i < nr * p.half; i += kHeadsThreads) {
        const uint32_t r = i / p.half, c = i - r * p.half;
        const int32_t src = src_of(r);
        ct[i] = src >= 0 ? p.cos_t[uint64_t(src) * p.half + c] : 0.0f;
        st[i] = src >= 0 ? p.sin_t[uint64_t(src) * p.half + c] : 0.0f;
    }
    __syncthreads();

    const uint32_t items = nr * p.per_row;
    const RotLane rl = rot_lane(lane, p.half);
    for (uint32_t base = 0; base < items; base += kSlots) {
        uint4 raw[kHeadsU];
        uint32_t row_l[kHeadsU], kind_h[kHeadsU];
        int32_t src_r[kHeadsU];
#pragma unroll
        for (int u = 0; u < kHeadsU; ++u) {
            const uint32_t it = base + group + kGroups * uint32_t(u);
            const bool live = it < items;
            const uint32_t r = live ? p.div_row.div(it) : 0u;
            const uint32_t j = live ? it - r * p.per_row : 0u;
            const int32_t src = live ? srcs[r] : -1;
            row_l[u] = r;
            kind_h[u] = j;
            src_r[u] = src;
            raw[u] = src >= 0 ? ld_stream(reinterpret_cast<const uint4*>(p.qkv + uint64_t(src) * p.qkv_stride +
                                                                          128u * j + 8u * part))
                              : uint4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < kHeadsU; ++u) {
            const uint32_t it = base + group + kGroups * uint32_t(u);
            const uint32_t kind = p.div_heads.div(kind_h[u]), h = kind_h[u] - kind * p.heads;
            const uint4 o = head_vector(raw[u], kind, wt + 128u * min(kind, 1u), ct + row_l[u] * p.half + rl.ci,
                                        st + row_l[u] * p.half + rl.ci, rl, part, p.eps);
            uint16_t* const out = kind == 0u ? p.out[0] : kind == 1u ? p.out[1] : p.out[2];
            if (it < items) {
                uint16_t* dst = out + uint64_t(h) * p.ohs + uint64_t(r0 + row_l[u]) * p.ors + 8u * part;
                st_stream(reinterpret_cast<uint4*>(dst), src_r[u] >= 0 ? o : uint4{0u, 0u, 0u, 0u});
            }
        }
    }
}

// heads_partial fused with cube_pool over its output: a workgroup per cube (512 threads). Output rows row0 + 64 c + l
// (slot l = 4 s + dx, s = dt * 4 + dy) are produced as heads_kernel produces them, and the cube's q and k means are
// summed from the rounded values as they are stored, in cube_pool_kernel's order: for each dx, slots s = 0 .. 15 in
// turn from zero (a slot outside the grid adds zero), then (dx 0 + dx 1) + (dx 2 + dx 3), divided by the token count.
// The outputs are therefore bit-identical to heads_partial followed by cube_pool in the gathered layout.
// A wave takes four consecutive head vectors of a row (one a 16-lane group), so each of its loads reads 1 KB of a
// row; a group sums its head vector over dx 0..3 in turn, each over s = 0 .. 15, and combines the four partial sums
// in its own registers. Taking one head vector a wave instead (the four groups the four dx, combined by lane
// exchanges) read four 256-byte pieces of four rows a load and measured 3-4% slower.
struct HeadsPoolParams {
    HeadsParams hp;
    float* qc;
    float* kc;
    int32_t* counts;
    uint64_t row0; // gathered: output row of cube 0's slot 0; grid: the model row of grid position (0, 0, 0)
    uint32_t gt, gh, gw, cw, plane, cubes;
    uint32_t grid; // nonzero: no map, each token's row read and written at its model row (the grid layout)
};
constexpr uint32_t kPoolThreads = 512;
constexpr int kPoolU = 8;                           // slots a group has in flight

// At most 128 registers (two workgroups a CU): left to itself the compiler takes more than that.
__global__ __launch_bounds__(kPoolThreads) __attribute__((amdgpu_waves_per_eu(4))) void
heads_pool_kernel(HeadsPoolParams pp)
{
    const HeadsParams& p = pp.hp;
    extern __shared__ float lds[];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, part = lane & 15u, grp = lane >> 4, wave = tid >> 6;
    const uint32_t c = blockIdx.x;
    const uint64_t orow0 = pp.row0 + uint64_t(c) * 64u;
    float* wt = lds;
    int32_t* srcs = reinterpret_cast<int32_t*>(lds + 256);
    // The cos and sin tables, at least 8 floats each: head_vector reads 8 values of them on every lane, rotating or
    // not, so with no rotary (half 0) they still lie inside the allocation.
    float* ct = lds + 256 + 64;
    float* st = ct + max(64u * p.half, 8u);
    stage_weights(wt, p.qw, p.kw, tid, kPoolThreads);
    const uint32_t cube_t = c / pp.plane, rem = c - cube_t * pp.plane, cube_y = rem / pp.cw, cube_x = rem - cube_y * pp.cw;
    // Slot l's model row (-1: none). Gathered: through the map (or l's own output row); grid: the token at the slot's
    // grid position, if it lies in the grid.
    auto src_of = [&](uint32_t l) -> int32_t {
        if (pp.grid) {
            const uint32_t tt = cube_t * 4u + (l >> 4), yy = cube_y * 4u + ((l >> 2) & 3u), xx = cube_x * 4u + (l & 3u);
            return tt < pp.gt && yy < pp.gh && xx < pp.gw
                       ? int32_t(pp.row0 + (uint64_t(tt) * pp.gh + yy) * pp.gw + xx)
                       : -1;
        }
        const int32_t m = p.map ? p.map[orow0 + l] : int32_t(orow0 + l);
        return m >= 0 && uint32_t(m) < p.model_rows ? m : -1;
    };
    if (tid < 64u)
        srcs[tid] = src_of(tid);
    for (uint32_t i = tid; i < 64u * p.half; i += kPoolThreads) {
        const uint32_t l = i / p.half, col = i - l * p.half;
        const int32_t src = src_of(l);
        ct[i] = src >= 0 ? p.cos_t[uint64_t(src) * p.half + col] : 0.0f;
        st[i] = src >= 0 ? p.sin_t[uint64_t(src) * p.half + col] : 0.0f;
    }
    const uint32_t nt = min(4u, pp.gt - cube_t * 4u), ny = min(4u, pp.gh - cube_y * 4u), nx = min(4u, pp.gw - cube_x * 4u);
    if (pp.counts && tid == 0)
        pp.counts[c] = int32_t(nt * ny * nx);
    __syncthreads();

    const RotLane rl = rot_lane(lane, p.half);
    const float n = float(nt * ny * nx);
    const uint32_t blocks = (p.per_row + 3u) / 4u;
    for (uint32_t b = wave; b < blocks; b += kPoolThreads / 64u) {
        const uint32_t j = b * 4u + grp;
        const bool live = j < p.per_row;
        const uint32_t jj = live ? j : 0u;
        const uint32_t kind = p.div_heads.div(jj), h = jj - kind * p.heads;
        const float* wk = wt + 128u * min(kind, 1u);
        uint16_t* const out = (kind == 0u ? p.out[0] : kind == 1u ? p.out[1] : p.out[2]) + uint64_t(h) * p.ohs;
        float p01[8], p2[8];
#pragma unroll 1
        for (uint32_t dx = 0; dx < 4u; ++dx) {
            const bool x_ok = cube_x * 4u + dx < pp.gw;
            float acc[8];
#pragma unroll
            for (int e = 0; e < 8; ++e)
                acc[e] = 0.0f;
#pragma unroll 1
            for (uint32_t s0 = 0; s0 < 16u; s0 += kPoolU) {
                uint4 raw[kPoolU];
                int32_t src_r[kPoolU];
#pragma unroll
                for (int u = 0; u < kPoolU; ++u) {
                    const int32_t src = live ? srcs[(s0 + uint32_t(u)) * 4u + dx] : -1;
                    src_r[u] = src;
                    raw[u] = src >= 0 ? ld_stream(reinterpret_cast<const uint4*>(
                                            p.qkv + uint64_t(src) * p.qkv_stride + 128u * jj + 8u * part))
                                      : uint4{0u, 0u, 0u, 0u};
                }
#pragma unroll
                for (int u = 0; u < kPoolU; ++u) {
                    const uint32_t s = s0 + uint32_t(u), l = s * 4u + dx;
                    uint4 o = head_vector(raw[u], kind, wk, ct + l * p.half + rl.ci, st + l * p.half + rl.ci, rl,
                                          part, p.eps);
                    o = src_r[u] >= 0 ? o : uint4{0u, 0u, 0u, 0u};
                    // Gathered: every slot's row is written (a padding slot's zeros); grid: a token's own row only.
                    const uint64_t orow = pp.grid ? uint64_t(src_r[u] >= 0 ? src_r[u] : 0) : orow0 + l;
                    if (live && (!pp.grid || src_r[u] >= 0))
                        st_stream(reinterpret_cast<uint4*>(out + orow * p.ors + 8u * part), o);
                    const bool ok = x_ok && cube_t * 4u + (s >> 2) < pp.gt && cube_y * 4u + (s & 3u) < pp.gh;
                    const uint32_t w[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        acc[2 * e] += ok ? bf16_lo(w[e]) : 0.0f;
                        acc[2 * e + 1] += ok ? bf16_hi(w[e]) : 0.0f;
                    }
                }
            }
            // (dx 0 + dx 1) + (dx 2 + dx 3), as cube_pool_kernel's two lane exchanges combine them.
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                if (dx == 0u)
                    p01[e] = acc[e];
                else if (dx == 1u)
                    p01[e] += acc[e];
                else if (dx == 2u)
                    p2[e] = acc[e];
                else
                    p01[e] += p2[e] + acc[e];
            }
        }
        if (live && kind < 2u) {
            float4* o = reinterpret_cast<float4*>((kind == 0u ? pp.qc : pp.kc) + (uint64_t(h) * pp.cubes + c) * 128u +
                                                  part * 8u);
            o[0] = float4{p01[0] / n, p01[1] / n, p01[2] / n, p01[3] / n};
            o[1] = float4{p01[4] / n, p01[5] / n, p01[6] / n, p01[7] / n};
        }
    }
}

} // namespace
} // namespace mh3

namespace {

using namespace mh3;

// The checks of mh3_heads_partial and the kernel parameters they give (row_begin 0, rows_per_block unset).
int heads_setup(const MH3HeadsArgs* args, const uint16_t* qkv, const float* q_w, const float* k_w,
                const float* cos_t, const float* sin_t, const int32_t* map, uint16_t* q, uint16_t* k, uint16_t* v,
                HeadsParams& p)
{
    if (!args)
        return MH3_ERR_POINTER;
    const MH3HeadsArgs& a = *args;
    if (a.heads == 0 || a.head_dim == 0)
        return MH3_ERR_SHAPE;
    if (a.head_dim != 128)
        return MH3_ERR_UNSUPPORTED;
    if (a.rot % 16u != 0 || a.rot > a.head_dim || !(a.eps > 0.0f))
        return MH3_ERR_PARAM;
    if (a.heads > 4096u || a.qkv_stride < 3ull * a.heads * a.head_dim)
        return MH3_ERR_SHAPE;
    if (a.rows == 0)
        return MH3_OK;
    if (a.rows >= (1u << 31) || a.model_rows == 0 || a.model_rows >= (1u << 31) || (!map && a.model_rows < a.rows))
        return MH3_ERR_SHAPE;
    if (!qkv || !q || !k || (a.rot && (!cos_t || !sin_t)))
        return MH3_ERR_POINTER;
    if (a.qkv_stride % 8 != 0 || a.out_head_stride % 8 != 0 || a.out_row_stride % 8 != 0 || !host::aligned16(qkv) ||
        !host::aligned16(q) || !host::aligned16(k) || (v && !host::aligned16(v)) ||
        (q_w && !host::aligned16(q_w)) || (k_w && !host::aligned16(k_w)))
        return MH3_ERR_ALIGN;
    // Outputs over qkv only in place: each output at its own input's position.
    const uint64_t qkv_bytes = ((uint64_t(a.model_rows) - 1) * a.qkv_stride + 3ull * a.heads * 128u) * 2u;
    const uint64_t out_bytes =
        ((uint64_t(a.heads) - 1) * a.out_head_stride + (uint64_t(a.rows) - 1) * a.out_row_stride + 128u) * 2u;
    uint16_t* outs[3] = {q, k, v};
    for (int t = 0; t < 3; ++t) {
        if (!outs[t] || !host::overlaps(outs[t], out_bytes, qkv, qkv_bytes))
            continue;
        const bool in_place = !map && outs[t] == qkv + uint64_t(t) * a.heads * 128u && a.out_head_stride == 128u &&
                              a.out_row_stride == a.qkv_stride;
        if (!in_place)
            return MH3_ERR_PARAM;
    }
    // Nor may an output overlap the norm weights, the rotary tables or the map.
    const uint64_t tab = a.rot ? uint64_t(a.model_rows) * (a.rot / 2u) * 4u : 0u;
    const host::Span small_in[] = {
        {q_w, 512u}, {k_w, 512u}, {cos_t, tab}, {sin_t, tab}, {map, map ? uint64_t(a.rows) * 4u : 0u}};
    for (int t = 0; t < 3; ++t) {
        const host::Span o[] = {{outs[t], out_bytes}};
        if (host::any_overlap(small_in, o))
            return MH3_ERR_PARAM;
    }
    p = HeadsParams{};
    p.qkv = qkv, p.qw = q_w, p.kw = k_w, p.cos_t = cos_t, p.sin_t = sin_t, p.map = map;
    p.out[0] = q, p.out[1] = k, p.out[2] = v;
    p.qkv_stride = a.qkv_stride, p.ohs = a.out_head_stride, p.ors = a.out_row_stride;
    p.rows = a.rows, p.model_rows = a.model_rows, p.heads = a.heads, p.half = a.rot / 2u, p.eps = a.eps;
    p.per_row = (v ? 3u : 2u) * a.heads;
    // At least two rows a workgroup: at 40 heads (120 head vectors a row, two passes) that measured 3-4% faster than
    // one row, and four rows slower again.
    p.rows_per_block = std::max(2u, kSlots / p.per_row);
    p.div_row = FastDiv::make(p.per_row);
    p.div_heads = FastDiv::make(a.heads);
    return MH3_OK;
}

// heads_kernel over output rows [row_begin, row_end).
int launch_heads(HeadsParams p, uint32_t row_begin, uint32_t row_end, hipStream_t stream)
{
    if (row_end <= row_begin)
        return MH3_OK;
    p.row_begin = row_begin, p.rows = row_end;
    const uint64_t blocks = (uint64_t(row_end - row_begin) + p.rows_per_block - 1) / p.rows_per_block;
    size_t lds = (256u + ((p.rows_per_block + 3u) & ~3u) + 2u * size_t(p.rows_per_block) * p.half) * sizeof(float);
    if (lds < kHeadsLdsFloor)
        lds = kHeadsLdsFloor;
    if (const hipError_t e = host::allow_dynamic_lds(reinterpret_cast<const void*>(&heads_kernel), lds); e != hipSuccess)
        return host::hip_error(e);
    hipLaunchKernelGGL(heads_kernel, dim3(uint32_t(blocks)), dim3(kHeadsThreads), lds, stream, p);
    return host::check_launch();
}

} // namespace

extern "C" int mh3_heads_partial(const MH3HeadsArgs* args, const uint16_t* qkv, const float* q_w, const float* k_w,
                                 const float* cos_t, const float* sin_t, const int32_t* map, uint16_t* q, uint16_t* k,
                                 uint16_t* v, mh3_stream_t stream)
{
    HeadsParams p;
    const int rc = heads_setup(args, qkv, q_w, k_w, cos_t, sin_t, map, q, k, v, p);
    if (rc != MH3_OK || args->rows == 0)
        return rc;
    return launch_heads(p, 0u, args->rows, static_cast<hipStream_t>(stream));
}

extern "C" int mh3_heads_partial_pool(const MH3HeadsArgs* args, const MH3CubeArgs* cubes, const uint16_t* qkv,
                                      const float* q_w, const float* k_w, const float* cos_t, const float* sin_t,
                                      const int32_t* map, uint16_t* q, uint16_t* k, uint16_t* v, float* qc, float* kc,
                                      int32_t* counts, mh3_stream_t stream)
{
    if (!args || !cubes)
        return MH3_ERR_POINTER;
    const MH3CubeArgs& cb = *cubes;
    const bool grid = cb.layout == MH3_CUBES_GRID;
    if ((cb.layout != MH3_CUBES_GATHERED && !grid) || cb.heads != args->heads || cb.head_dim != args->head_dim ||
        cb.head_stride != args->out_head_stride || cb.row_stride != args->out_row_stride || (grid && map))
        return MH3_ERR_PARAM; // the pool must read the head tiles this call writes
    if (cb.grid_t == 0 || cb.grid_h == 0 || cb.grid_w == 0)
        return MH3_ERR_SHAPE;
    const uint64_t ncubes = uint64_t((cb.grid_t + 3u) / 4u) * ((cb.grid_h + 3u) / 4u) * ((cb.grid_w + 3u) / 4u);
    // The rows the cubes cover: 64 a cube in the gathered layout, the grid's tokens in the model's order.
    const uint64_t span = grid ? uint64_t(cb.grid_t) * cb.grid_h * cb.grid_w : ncubes * 64u;
    if (ncubes * cb.heads >= (uint64_t(1) << 31) || cb.row0 + span > args->rows)
        return MH3_ERR_SHAPE;
    HeadsParams p;
    const int rc = heads_setup(args, qkv, q_w, k_w, cos_t, sin_t, map, q, k, v, p);
    if (rc != MH3_OK)
        return rc;
    if (!qc || !kc)
        return MH3_ERR_POINTER;
    if (!host::aligned16(qc) || !host::aligned16(kc))
        return MH3_ERR_ALIGN;
    {
        // The pooled outputs may not overlap any input, the head tiles this call writes, or each other: one
        // workgroup a cube writes them while the others still read qkv and write their own rows.
        const uint64_t qkv_bytes = ((uint64_t(args->model_rows) - 1) * args->qkv_stride + 3ull * args->heads * 128u) * 2u;
        const uint64_t out_bytes = ((uint64_t(args->heads) - 1) * args->out_head_stride +
                                    (uint64_t(args->rows) - 1) * args->out_row_stride + 128u) * 2u;
        const uint64_t tab = args->rot ? uint64_t(args->model_rows) * (args->rot / 2u) * 4u : 0u;
        const uint64_t pooled = ncubes * args->heads * 128u * 4u;
        const host::Span in[] = {{qkv, qkv_bytes}, {q, out_bytes},   {k, out_bytes},
                                 {v, out_bytes},   {q_w, 512u},      {k_w, 512u},
                                 {cos_t, tab},     {sin_t, tab},     {map, map ? uint64_t(args->rows) * 4u : 0u}};
        const host::Span out[] = {{qc, pooled}, {kc, pooled}, {counts, ncubes * 4u}};
        if (host::any_overlap(in, out))
            return MH3_ERR_PARAM;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    const uint32_t video0 = uint32_t(cb.row0), video1 = uint32_t(cb.row0 + span);
    int r = launch_heads(p, 0u, video0, st); // rows before the cubes, and after them (the dense rows)
    if (r == MH3_OK)
        r = launch_heads(p, video1, args->rows, st);
    if (r != MH3_OK)
        return r;
    HeadsPoolParams pp{};
    pp.hp = p, pp.qc = qc, pp.kc = kc, pp.counts = counts, pp.row0 = cb.row0;
    pp.gt = cb.grid_t, pp.gh = cb.grid_h, pp.gw = cb.grid_w, pp.cw = (cb.grid_w + 3u) / 4u;
    pp.plane = ((cb.grid_h + 3u) / 4u) * pp.cw, pp.cubes = uint32_t(ncubes), pp.grid = grid ? 1u : 0u;
    const size_t lds = (256u + 64u + 2u * std::max(64u * p.half, 8u)) * sizeof(float); // 26 KB at rot 96
    if (const hipError_t e = host::allow_dynamic_lds(reinterpret_cast<const void*>(&heads_pool_kernel), lds);
        e != hipSuccess)
        return host::hip_error(e);
    hipLaunchKernelGGL(heads_pool_kernel, dim3(uint32_t(ncubes)), dim3(kPoolThreads), lds, st, pp);
    return host::check_launch();
}
