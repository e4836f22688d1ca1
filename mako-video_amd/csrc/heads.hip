// `heads_partial`: the step between the QKV GEMM and attention. Per model row and head, q and k get an RMS norm over
// the head's 128 values and the rotary positions on the first `rot` of them; v is copied; the results go out as head
// tiles, optionally gathered through the cube map into the order the sparse selector and flash_attn_sparse_128 read.
// Reference semantics: the mako-common kernel of this name, described in docs/architecture.md:35-38,61-63,123-125
// ("RMS norms per head, rotary positions"; "the head tiles are gathered through that map ... padding rows zero").
//
// Design (gfx950): the op reads every element of q, k and v once and writes it once (4 bytes an element), so it is
// HBM-bound. A head vector (128 bf16 = 256 bytes) belongs to one 16-lane DPP row, 16 bytes a lane, so the sum of
// squares is a DPP row reduction with no LDS and no barrier.
// - A workgroup of 512 threads is 32 such groups. It takes whole rows, enough that their head vectors fill about 128
//   slots and at least two rows, and each group has up to 4 head vectors in flight (loads first, then the arithmetic
//   and the stores).
//   Consecutive groups take consecutive head vectors of a row, so a wave's load covers 1 KB of contiguous qkv.
// - The rotary pairs value i with i + rot / 2: lane p (values 8 p .. 8 p + 7) pairs with lane p +- rot / 16 of the
//   same group; the partner's raw bf16 words come over by ds_bpermute, and each lane normalizes both halves itself
//   (the norm factor is the group's).
// - The workgroup stages the two norm weight vectors and its rows' cos / sin tables in LDS once.
// - A padding slot of the cube map writes zeros and reads nothing.
#include "mh3_common.hpp"

namespace mh3 {
namespace {

constexpr uint32_t kHeadsThreads = 512;
constexpr uint32_t kGroups = kHeadsThreads / 16u; // one head vector a 16-lane group
constexpr int kHeadsU = 4;                        // head vectors a group has in flight
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
    FastDiv div_row, div_heads;
    float eps;
};

__global__ __launch_bounds__(kHeadsThreads) void heads_kernel(HeadsParams p)
{
    // LDS: the norm weights w [2][128] (q, then k); the rows' model rows src [rows_per_block] (-1: padding); their
    // cos and sin tables [rows_per_block][half] each.
    extern __shared__ float lds[];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, part = lane & 15u, group = tid >> 4;
    const uint32_t r0 = blockIdx.x * p.rows_per_block;
    const uint32_t nr = min(p.rows_per_block, p.rows - r0);
    float* wt = lds;
    int32_t* srcs = reinterpret_cast<int32_t*>(lds + 256);
    float* ct = lds + 256 + p.rows_per_block;
    float* st = ct + p.rows_per_block * p.half;
    for (uint32_t i = tid; i < 256u; i += kHeadsThreads) {
        const float* w = i < 128u ? p.qw : p.kw;
        wt[i] = w ? w[i & 127u] : 1.0f;
    }
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
    // The rotary partner lane of this one within its group, and the sign its sine term takes.
    const uint32_t hv = p.half / 8u; // lanes a half of the rotating values spans
    const bool rotating = part < 2u * hv;
    const bool first_half = part < hv;
    const uint32_t partner = (lane & ~15u) | (rotating ? (first_half ? part + hv : part - hv) : part);
    const uint32_t pd = 8u * (rotating ? (first_half ? part + hv : part - hv) : part); // the partner's first value
    const uint32_t ci = rotating ? 8u * part - (first_half ? 0u : p.half) : 0u;          // cos / sin column
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
            const uint32_t w[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
            // The partner's words (every lane takes part in the exchange; lanes without a partner get their own).
            uint32_t pw[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                pw[e] = uint32_t(__builtin_amdgcn_ds_bpermute(int(partner << 2), int(w[e])));
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
            uint4 o = raw[u];
            if (kind < 2u) {
                const float inv = 1.0f / sqrtf(fmaf(ss, 1.0f / 128.0f, p.eps));
                const float* wk = wt + 128u * kind;
                float y[8];
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    y[e] = x[e] * inv * wk[8u * part + e];
                if (rotating) {
                    const float* c = ct + row_l[u] * p.half + ci;
                    const float* s = st + row_l[u] * p.half + ci;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float b = xp[e] * inv * wk[pd + e];
                        y[e] = first_half ? fmaf(y[e], c[e], -b * s[e]) : fmaf(y[e], c[e], b * s[e]);
                    }
                }
                o = uint4{pack_bf16(y[0], y[1]), pack_bf16(y[2], y[3]), pack_bf16(y[4], y[5]), pack_bf16(y[6], y[7])};
            }
            uint16_t* const out = kind == 0u ? p.out[0] : kind == 1u ? p.out[1] : p.out[2];
            if (it < items) {
                uint16_t* dst = out + uint64_t(h) * p.ohs + uint64_t(r0 + row_l[u]) * p.ors + 8u * part;
                st_stream(reinterpret_cast<uint4*>(dst), src_r[u] >= 0 ? o : uint4{0u, 0u, 0u, 0u});
            }
        }
    }
}

} // namespace
} // namespace mh3

extern "C" int mh3_heads_partial(const MH3HeadsArgs* args, const uint16_t* qkv, const float* q_w, const float* k_w,
                                 const float* cos_t, const float* sin_t, const int32_t* map, uint16_t* q, uint16_t* k,
                                 uint16_t* v, mh3_stream_t stream)
{
    using namespace mh3;
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
    HeadsParams p{};
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
    const uint64_t blocks = (uint64_t(a.rows) + p.rows_per_block - 1) / p.rows_per_block;
    size_t lds = (256u + p.rows_per_block + 2u * size_t(p.rows_per_block) * p.half) * sizeof(float);
    if (lds < kHeadsLdsFloor)
        lds = kHeadsLdsFloor;
    if (host::allow_dynamic_lds(reinterpret_cast<const void*>(&heads_kernel), lds) != hipSuccess)
        return MH3_ERR_HIP;
    hipLaunchKernelGGL(heads_kernel, dim3(uint32_t(blocks)), dim3(kHeadsThreads), lds,
                       static_cast<hipStream_t>(stream), p);
    return host::check_launch();
}
