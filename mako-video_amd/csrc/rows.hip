// Row kernels of the H3 block: the adaLN-modulated RMS norm (`rms_mod_rows`), the gated residual add
// (`gate_add_rows`), the two fused into one HBM pass, and `swiglu_rows`. Reference semantics: the mako-common
// kernels of these names, described in docs/architecture.md:49-52,61-66 and docs/performance.md:44.
//
// Design (gfx950): a workgroup owns one row at a time and streams through rows (a persistent grid). Each thread keeps
// a fixed slice of VPT 16-byte vectors of the row (8 bf16 or 4 float each), so the row is read from HBM once and held
// in registers; the sum of squares is a lane-local sum, a 6-step wave butterfly and one exchange of per-wave partials
// through LDS (double-buffered by row parity: one barrier a row). The next row's loads are issued before the current
// row is reduced and written, so every wave keeps a row's worth of loads in flight. The per-column coefficients of a
// modulation set (a = w (1 + scale) gate, b = shift gate) are folded once per workgroup: into registers when there is
// one set (the thread's columns never change), into an LDS table when several sets fit in 64 KiB, else recomputed
// from the parameter vectors per row. Streaming data uses non-temporal loads and stores.
#include "mh3_common.hpp"

namespace mh3 {

// kGateAddMod is the block's own order: x += gate * y, then h = the modulated norm of the updated (stored) x.
enum RowOp { kRmsMod = 0, kGateAdd = 1, kFused = 2, kGateAddMod = 3 };
// Coefficient planes of an op: a and b; kGateAddMod adds c (the gate).
template <int OP>
constexpr uint32_t kPlanes = OP == kGateAddMod ? 3u : 2u;

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
    __device__ static void unpack(const u32x4_t& r, float (&f)[8])
    {
        f[0] = bf16_lo(r[0]), f[1] = bf16_hi(r[0]), f[2] = bf16_lo(r[1]), f[3] = bf16_hi(r[1]);
        f[4] = bf16_lo(r[2]), f[5] = bf16_hi(r[2]), f[6] = bf16_lo(r[3]), f[7] = bf16_hi(r[3]);
    }
    // acc + the sum of squares of the 8 elements.
    __device__ static float sumsq(const u32x4_t& r, float acc)
    {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc = fmaf(bf16_lo(r[i]), bf16_lo(r[i]), acc);
            acc = fmaf(bf16_hi(r[i]), bf16_hi(r[i]), acc);
        }
        return acc;
    }
    __device__ static u32x4_t pack4(const float (&f)[8])
    {
        return u32x4_t{pack_bf16(f[0], f[1]), pack_bf16(f[2], f[3]), pack_bf16(f[4], f[5]), pack_bf16(f[6], f[7])};
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
    __device__ static void unpack(const u32x4_t& r, float (&f)[4])
    {
        f[0] = __uint_as_float(r[0]), f[1] = __uint_as_float(r[1]), f[2] = __uint_as_float(r[2]);
        f[3] = __uint_as_float(r[3]);
    }
    __device__ static float sumsq(const u32x4_t& r, float acc)
    {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            acc = fmaf(__uint_as_float(r[i]), __uint_as_float(r[i]), acc);
        return acc;
    }
    __device__ static u32x4_t pack4(const float (&f)[4])
    {
        return u32x4_t{__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3])};
    }
    __device__ static uint4 pack(const float (&f)[4])
    {
        return uint4{__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3])};
    }
};

struct RowsParams {
    const u32x4_t* x;   // rms_mod / fused: the normed input; gate_add, gate_add_mod: the addend y
    const u32x4_t* res; // fused: the residual; gate_add, gate_add_mod: x (in/out)
    u32x4_t* out;       // gate_add_mod: h
    u32x4_t* out2;      // gate_add_mod: the updated x
    const float* w;
    const float* shift;
    const float* scale;
    const float* gate;
    const uint8_t* set_of_row;
    uint32_t rows, dim, nvec, n_sets;
    uint32_t set_stride; // floats from one set's shift / scale / gate vector to the next set's
    float eps, inv_dim;
    uint32_t rows_per_wave; // wave kernel: 0 = persistent grid
};

enum CoefSrc { kCoefReg = 0, kCoefLds = 1, kCoefGlobal = 2 };

// The per-column coefficients of set s: y = (x * inv) * a + b (rms_mod), out = res + (x * inv) * a + b (fused),
// out = res + a * y (gate_add), x' = x + c * y and h = (x' * inv) * a + b (gate_add_mod), for the E columns
// c0 .. c0 + E - 1 (c0 a multiple of 4), through 16-byte loads.
template <int OP, int E>
__device__ __forceinline__ void coef_vec(const RowsParams& p, uint32_t s, uint32_t c0, float (&a)[E], float (&b)[E],
                                         float (&c)[E])
{
    const uint64_t i = uint64_t(s) * p.set_stride + c0;
#pragma unroll
    for (int q = 0; q < E / 4; ++q) {
        float g[4], w[4], sc[4], sh[4];
        if constexpr (OP != kRmsMod) {
            const float4 t = *reinterpret_cast<const float4*>(p.gate + i + 4 * q);
            g[0] = t.x, g[1] = t.y, g[2] = t.z, g[3] = t.w;
        }
        if constexpr (OP != kGateAdd) {
            const float4 ts = *reinterpret_cast<const float4*>(p.scale + i + 4 * q);
            const float4 th = *reinterpret_cast<const float4*>(p.shift + i + 4 * q);
            sc[0] = ts.x, sc[1] = ts.y, sc[2] = ts.z, sc[3] = ts.w;
            sh[0] = th.x, sh[1] = th.y, sh[2] = th.z, sh[3] = th.w;
            if (p.w) {
                const float4 tw = *reinterpret_cast<const float4*>(p.w + c0 + 4 * q);
                w[0] = tw.x, w[1] = tw.y, w[2] = tw.z, w[3] = tw.w;
            } else {
                w[0] = w[1] = w[2] = w[3] = 1.0f;
            }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if constexpr (OP == kGateAdd) {
                a[4 * q + e] = g[e];
                b[4 * q + e] = 0.0f;
            } else {
                const float m = w[e] * (1.0f + sc[e]);
                if constexpr (OP == kFused) {
                    a[4 * q + e] = m * g[e];
                    b[4 * q + e] = sh[e] * g[e];
                } else {
                    a[4 * q + e] = m;
                    b[4 * q + e] = sh[e];
                }
                if constexpr (OP == kGateAddMod)
                    c[4 * q + e] = g[e];
            }
        }
    }
}

template <int DT, int VPT, int OP, int SRC>
__global__ __launch_bounds__(1024) void rows_kernel(RowsParams p)
{
    using V = RowVec<DT>;
    constexpr int E = V::N;
    // LDS: [2][64] partial sums of squares (4 a wave: one per 16-lane row), by row parity; then, for kCoefLds,
    // a[n_sets][dim] and b[n_sets][dim].
    extern __shared__ float smem[];
    float* ctab = smem + 128;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6, nparts = (blockDim.x >> 6) * 4u;
    const uint32_t nthr = blockDim.x;

    float ca[VPT][E], cb[VPT][E], cc[VPT][E];
    if constexpr (SRC == kCoefReg) {
#pragma unroll
        for (int j = 0; j < VPT; ++j)
            coef_vec<OP, E>(p, 0, min(tid + j * nthr, p.nvec - 1u) * E, ca[j], cb[j], cc[j]);
    }
    const uint32_t coef_total = p.n_sets * p.dim;
    if constexpr (SRC == kCoefLds) {
        for (uint32_t i = tid; i < p.n_sets * p.nvec; i += nthr) {
            const uint32_t s = i / p.nvec, v = i - s * p.nvec;
            float a[E], b[E], c[E];
            coef_vec<OP, E>(p, s, v * E, a, b, c);
#pragma unroll
            for (int e = 0; e < E; ++e) {
                ctab[s * p.dim + v * E + e] = a[e];
                ctab[coef_total + s * p.dim + v * E + e] = b[e];
                if constexpr (OP == kGateAddMod)
                    ctab[2 * coef_total + s * p.dim + v * E + e] = c[e];
            }
        }
        __syncthreads();
    }

    // Row r's vectors of this thread, through a descriptor over the row alone: lanes past the row's last vector and
    // rows past the last row read zero (no memory traffic), so the loads need no branches.
    auto load = [&](uint32_t r, u32x4_t (&xv)[VPT], u32x4_t (&rv)[VPT]) {
        const uint32_t rr = min(r, p.rows - 1u), bytes = r < p.rows ? p.nvec * 16u : 0u;
        const __amdgpu_buffer_rsrc_t sx = buffer_rsrc(p.x + uint64_t(rr) * p.nvec, bytes);
        const __amdgpu_buffer_rsrc_t sr = buffer_rsrc(p.res + uint64_t(rr) * p.nvec, bytes);
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const uint32_t off = (tid + j * nthr) * 16u;
            xv[j] = __builtin_amdgcn_raw_buffer_load_b128(sx, off, 0, kNonTemporal);
            if constexpr (OP != kRmsMod)
                rv[j] = __builtin_amdgcn_raw_buffer_load_b128(sr, off, 0, kNonTemporal);
        }
    };
    // Reduces, modulates and writes row r from registers; `parity` picks the LDS partial-sum slot.
    auto process = [&](uint32_t r, const u32x4_t (&xin)[VPT], const u32x4_t (&rv)[VPT], uint32_t parity) {
        const uint32_t set = p.set_of_row ? min(uint32_t(p.set_of_row[r]), p.n_sets - 1u) : 0u;
        // gate_add_mod: the updated x, rounded and stored first; the norm is of the stored values.
        u32x4_t xn[VPT];
        if constexpr (OP == kGateAddMod) {
            const __amdgpu_buffer_rsrc_t sx = buffer_rsrc(p.out2 + uint64_t(r) * p.nvec, p.nvec * 16u);
#pragma unroll
            for (int j = 0; j < VPT; ++j) {
                const uint32_t v = min(tid + j * nthr, p.nvec - 1u);
                float f[E], rr[E], o[E], gc[E];
                V::unpack(xin[j], f);
                V::unpack(rv[j], rr);
                if constexpr (SRC == kCoefGlobal) {
                    float ga[E], gb[E];
                    coef_vec<OP, E>(p, set, v * E, ga, gb, gc);
                }
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    const float g = SRC == kCoefReg ? cc[j][e]
                                    : SRC == kCoefLds ? ctab[2 * coef_total + set * p.dim + v * E + e]
                                                      : gc[e];
                    o[e] = fmaf(g, f[e], rr[e]);
                }
                xn[j] = V::pack4(o);
                __builtin_amdgcn_raw_buffer_store_b128(xn[j], sx, (tid + j * nthr) * 16u, 0, kNonTemporal);
            }
        }
        const u32x4_t(&xv)[VPT] = OP == kGateAddMod ? xn : xin;
        float inv = 1.0f;
        if constexpr (OP != kGateAdd) {
            float ss = 0.0f;
#pragma unroll
            for (int j = 0; j < VPT; ++j)
                ss = V::sumsq(xv[j], ss);
            ss = row16_sum(ss);
            float* part = smem + parity * 64u;
            if ((lane & 15u) == 0)
                part[wave * 4u + (lane >> 4)] = ss;
            __syncthreads();
            float total = 0.0f;
            for (uint32_t w = 0; w < nparts; ++w)
                total += part[w];
            inv = 1.0f / sqrtf(fmaf(total, p.inv_dim, p.eps));
        }
        // Stores past the row's last vector are dropped by the descriptor.
        const __amdgpu_buffer_rsrc_t so = buffer_rsrc(p.out + uint64_t(r) * p.nvec, p.nvec * 16u);
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const uint32_t v = min(tid + j * nthr, p.nvec - 1u); // clamped for the coefficient reads only
            float f[E], rr[E], o[E];
            V::unpack(xv[j], f);
            if constexpr (OP == kGateAdd || OP == kFused)
                V::unpack(rv[j], rr);
            float ga[E], gb[E], gc[E];
            if constexpr (SRC == kCoefGlobal)
                coef_vec<OP, E>(p, set, v * E, ga, gb, gc);
#pragma unroll
            for (int e = 0; e < E; ++e) {
                float a, b;
                if constexpr (SRC == kCoefReg) {
                    a = ca[j][e];
                    b = cb[j][e];
                } else if constexpr (SRC == kCoefLds) {
                    a = ctab[set * p.dim + v * E + e];
                    b = ctab[coef_total + set * p.dim + v * E + e];
                } else {
                    a = ga[e];
                    b = gb[e];
                }
                if constexpr (OP == kRmsMod || OP == kGateAddMod)
                    o[e] = fmaf(f[e] * inv, a, b);
                else if constexpr (OP == kFused)
                    o[e] = rr[e] + fmaf(f[e] * inv, a, b);
                else
                    o[e] = fmaf(a, f[e], rr[e]);
            }
            __builtin_amdgcn_raw_buffer_store_b128(V::pack4(o), so, (tid + j * nthr) * 16u, 0, kNonTemporal);
        }
    };

    // Two register sets take turns: one row is reduced and written while the next one's loads are in flight. The
    // loop is unrolled by two so no in-flight load is ever copied between registers (a copy would wait for it).
    const uint32_t G = gridDim.x;
    uint32_t row = blockIdx.x;
    if (row >= p.rows)
        return;
    u32x4_t xa[VPT], ra[VPT], xb[VPT], rb[VPT];
    load(row, xa, ra);
    while (true) {
        const uint32_t r1 = row + G;
        load(r1, xb, rb);
        process(row, xa, ra, 0u);
        if (r1 >= p.rows)
            break;
        const uint32_t r2 = r1 + G;
        load(r2, xa, ra);
        process(r1, xb, rb, 1u);
        if (r2 >= p.rows)
            break;
        row = r2;
    }
}

// One wavefront per row (no cross-wave reduction, so no barrier a row). The workgroup folds the coefficient table
// of every set into LDS once; each wave holds a whole row (NV 16-byte vectors a lane of x, and of the residual) in
// registers, reduces it with DPP and three cross-row reads, and streams the outputs one vector at a time, reading
// that vector's coefficients from LDS just before use.
constexpr uint32_t kWaveBlock = 512; // wave-kernel workgroup threads: 8 waves, two workgroups a CU

template <int DT, int NV, int OP, int SRC>
__global__ __launch_bounds__(kWaveBlock) void rows_wave_kernel(RowsParams p)
{
    using V = RowVec<DT>;
    constexpr int E = V::N;
    extern __shared__ float ctab[]; // a[n_sets][dim], then b[n_sets][dim]
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    // Rows: with rows_per_wave = 0 the grid is persistent and strides over all rows; otherwise workgroup b takes the
    // contiguous rows [b * waves * rows_per_wave, ...), its waves interleaved over them so they read neighbours.
    const uint32_t waves = blockDim.x >> 6;
    const uint32_t first = p.rows_per_wave ? blockIdx.x * waves * p.rows_per_wave + wave : blockIdx.x * waves + wave;
    const uint32_t step = p.rows_per_wave ? waves : gridDim.x * waves;
    const uint32_t last = p.rows_per_wave ? min(p.rows, (blockIdx.x + 1) * waves * p.rows_per_wave) : p.rows;
    // A row's loads go through a descriptor over that row alone; a row past `last` reads zero without traffic.
    u32x4_t xv[NV], rv[NV];
    auto load = [&](uint32_t row) {
        const uint32_t bytes = row < last ? p.nvec * 16u : 0u;
        const uint32_t rr = min(row, p.rows - 1u);
        const __amdgpu_buffer_rsrc_t sx = buffer_rsrc(p.x + uint64_t(rr) * p.nvec, bytes);
        const __amdgpu_buffer_rsrc_t sr = buffer_rsrc(p.res + uint64_t(rr) * p.nvec, bytes);
        // All of x first, then the residual: loads complete in order, so the sum of squares waits for x alone and
        // runs while the residual is still in flight (2-3% faster than interleaving the two at 129,536 x 5120).
#pragma unroll
        for (int j = 0; j < NV; ++j)
            xv[j] = __builtin_amdgcn_raw_buffer_load_b128(sx, (lane + 64u * j) * 16u, 0, kNonTemporal);
#pragma unroll
        for (int j = 0; j < NV; ++j)
            if constexpr (OP != kRmsMod)
                rv[j] = __builtin_amdgcn_raw_buffer_load_b128(sr, (lane + 64u * j) * 16u, 0, kNonTemporal);
    };
    const uint32_t coef_total = p.n_sets * p.dim;
    for (uint32_t i = tid; SRC == kCoefLds && i < p.n_sets * p.nvec; i += blockDim.x) {
        const uint32_t s = i / p.nvec, v = i - s * p.nvec;
        float a[E], b[E], c[E];
        coef_vec<OP, E>(p, s, v * E, a, b, c);
#pragma unroll
        for (int e = 0; e < E; ++e) {
            ctab[s * p.dim + v * E + e] = a[e];
            ctab[coef_total + s * p.dim + v * E + e] = b[e];
            if constexpr (OP == kGateAddMod)
                ctab[2 * coef_total + s * p.dim + v * E + e] = c[e];
        }
    }
    if constexpr (SRC == kCoefLds)
        __syncthreads();

    // (Issuing the first row's loads before the table is built is slower: the table's parameter loads would then
    // complete in order behind them.)
    for (uint32_t row = first; row < last; row += step) {
        load(row);
        const __amdgpu_buffer_rsrc_t so = buffer_rsrc(p.out + uint64_t(row) * p.nvec, p.nvec * 16u);
        const uint32_t set = p.set_of_row ? min(uint32_t(p.set_of_row[row]), p.n_sets - 1u) : 0u;
        if constexpr (OP == kGateAddMod) {
            // x' = x + gate * y, rounded and stored; it replaces y in xv, and the norm below is of the stored values.
            const __amdgpu_buffer_rsrc_t sx = buffer_rsrc(p.out2 + uint64_t(row) * p.nvec, p.nvec * 16u);
            const float* tc = ctab + 2 * coef_total + set * p.dim;
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const uint32_t v = min(lane + 64u * j, p.nvec - 1u);
                float f[E], rr[E], o[E], g[E];
                if constexpr (SRC == kCoefLds) {
#pragma unroll
                    for (int q = 0; q < E / 4; ++q) {
                        const float4 t4 = *reinterpret_cast<const float4*>(tc + v * E + 4 * q);
                        g[4 * q] = t4.x, g[4 * q + 1] = t4.y, g[4 * q + 2] = t4.z, g[4 * q + 3] = t4.w;
                    }
                } else {
                    float ga[E], gb[E];
                    coef_vec<OP, E>(p, set, v * E, ga, gb, g);
                }
                V::unpack(xv[j], f);
                V::unpack(rv[j], rr);
#pragma unroll
                for (int e = 0; e < E; ++e)
                    o[e] = fmaf(g[e], f[e], rr[e]);
                xv[j] = V::pack4(o);
                __builtin_amdgcn_raw_buffer_store_b128(xv[j], sx, (lane + 64u * j) * 16u, 0, kNonTemporal);
            }
        }
        float inv = 1.0f;
        if constexpr (OP != kGateAdd) {
            float ss = 0.0f;
#pragma unroll
            for (int j = 0; j < NV; ++j)
                ss = V::sumsq(xv[j], ss);
            ss = row16_sum(ss);
            // The output pass unpacks x again rather than keeping the sum pass's unpacked values live.
#pragma unroll
            for (int j = 0; j < NV; ++j)
                asm volatile("" : "+v"(xv[j]));
            const float total = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ss), 0)) +
                                __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ss), 16)) +
                                __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ss), 32)) +
                                __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ss), 48));
            inv = 1.0f / sqrtf(fmaf(total, p.inv_dim, p.eps));
        }
        const float* ta = ctab + set * p.dim;
        const float* tb = ctab + coef_total + set * p.dim;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const uint32_t v = min(lane + 64u * j, p.nvec - 1u);
            float f[E], rr[E], o[E], a[E], b[E];
            if constexpr (SRC == kCoefLds) {
#pragma unroll
                for (int q = 0; q < E / 4; ++q) {
                    const float4 ta4 = *reinterpret_cast<const float4*>(ta + v * E + 4 * q);
                    const float4 tb4 = *reinterpret_cast<const float4*>(tb + v * E + 4 * q);
                    a[4 * q] = ta4.x, a[4 * q + 1] = ta4.y, a[4 * q + 2] = ta4.z, a[4 * q + 3] = ta4.w;
                    b[4 * q] = tb4.x, b[4 * q + 1] = tb4.y, b[4 * q + 2] = tb4.z, b[4 * q + 3] = tb4.w;
                }
            } else {
                float c[E];
                coef_vec<OP, E>(p, set, v * E, a, b, c);
            }
            V::unpack(xv[j], f);
            if constexpr (OP == kGateAdd || OP == kFused)
                V::unpack(rv[j], rr);
#pragma unroll
            for (int e = 0; e < E; ++e) {
                if constexpr (OP == kRmsMod || OP == kGateAddMod)
                    o[e] = fmaf(f[e] * inv, a[e], b[e]);
                else if constexpr (OP == kFused)
                    o[e] = rr[e] + fmaf(f[e] * inv, a[e], b[e]);
                else
                    o[e] = fmaf(a[e], f[e], rr[e]);
            }
            __builtin_amdgcn_raw_buffer_store_b128(V::pack4(o), so, (lane + 64u * j) * 16u, 0, kNonTemporal);
            __builtin_amdgcn_sched_barrier(0); // one vector's coefficients live at a time
        }
    }
}

// ---- the float residual stream with bf16 GEMM operands ------------------------------------------------------------
// The reference keeps the block's residual stream x in float and rounds the GEMMs' inputs to bf16
// (docs/architecture.md:69-70). These kernels read and write float x and give or take the GEMMs' bf16 rows: the
// modulated norm's output (the next GEMM's input, rounded once) and, with YB, the gated addend y (a GEMM's bf16
// output). One wavefront a row, as in rows_wave_kernel; a lane's unit is 4 columns, 16 bytes of a float row and 8 of a
// bf16 row: unit lane + 64 j, j < NU, so every load and store instruction covers one contiguous stretch of its row.
// The coefficient table is rows_wave_kernel's, and so are the reduction (DPP row sums, four readlanes) and the
// arithmetic, so each op gives the same bits whether fused (kGateAddMod) or run as its two parts.
template <int OP, int YB, int NU, int SRC>
__global__ __launch_bounds__(kWaveBlock) void rows_f32_stream_kernel(RowsParams p)
{
    using F = RowVec<MH3_F32>;
    extern __shared__ float ctab[]; // kCoefLds: a[n_sets][dim], b[n_sets][dim] (and c for kGateAddMod)
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t units = p.nvec; // 4-column units a row
    const uint32_t coef_total = p.n_sets * p.dim;
    for (uint32_t i = tid; SRC == kCoefLds && i < p.n_sets * units; i += blockDim.x) {
        const uint32_t s = i / units, v = i - s * units;
        float a[4], b[4], c[4];
        coef_vec<OP, 4>(p, s, v * 4u, a, b, c);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            ctab[s * p.dim + v * 4u + e] = a[e];
            ctab[coef_total + s * p.dim + v * 4u + e] = b[e];
            if constexpr (OP == kGateAddMod)
                ctab[2 * coef_total + s * p.dim + v * 4u + e] = c[e];
        }
    }
    __syncthreads();
    const uint32_t row = blockIdx.x * (blockDim.x >> 6) + wave;
    if (row >= p.rows)
        return;
    const uint32_t set = p.set_of_row ? min(uint32_t(p.set_of_row[row]), p.n_sets - 1u) : 0u;
    // The float row x (rms_mod: the input; the gate-add ops: the stream updated in place).
    const u32x4_t* xsrc = OP == kRmsMod ? p.x : p.res;
    const __amdgpu_buffer_rsrc_t sx = buffer_rsrc(xsrc + uint64_t(row) * units, units * 16u);
    u32x4_t xv[NU];
#pragma unroll
    for (int j = 0; j < NU; ++j)
        xv[j] = __builtin_amdgcn_raw_buffer_load_b128(sx, (lane + 64u * j) * 16u, 0, kNonTemporal);
    if constexpr (OP == kGateAdd || OP == kGateAddMod) {
        // x' = x + gate * y in float, stored; the norm below is of these values.
        u32x4_t yv[NU];
        u32x2_t yh[NU];
        const char* ybase = reinterpret_cast<const char*>(p.x) + uint64_t(row) * units * (YB ? 8u : 16u);
        const __amdgpu_buffer_rsrc_t sy = buffer_rsrc(ybase, units * (YB ? 8u : 16u));
#pragma unroll
        for (int j = 0; j < NU; ++j) {
            if constexpr (YB)
                yh[j] = __builtin_amdgcn_raw_buffer_load_b64(sy, (lane + 64u * j) * 8u, 0, kNonTemporal);
            else
                yv[j] = __builtin_amdgcn_raw_buffer_load_b128(sy, (lane + 64u * j) * 16u, 0, kNonTemporal);
        }
        const __amdgpu_buffer_rsrc_t so2 = buffer_rsrc(p.out2 + uint64_t(row) * units, units * 16u);
        const float* tg = ctab + (OP == kGateAdd ? 0u : 2u * coef_total) + set * p.dim;
#pragma unroll
        for (int j = 0; j < NU; ++j) {
            const uint32_t v = min(lane + 64u * j, units - 1u);
            float g[4], f[4], y[4], o[4];
            if constexpr (SRC == kCoefLds) {
                const float4 g4 = *reinterpret_cast<const float4*>(tg + v * 4u);
                g[0] = g4.x, g[1] = g4.y, g[2] = g4.z, g[3] = g4.w;
            } else {
                float ga[4], gb[4], gc[4];
                coef_vec<OP, 4>(p, set, v * 4u, ga, gb, gc);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    g[e] = OP == kGateAdd ? ga[e] : gc[e];
            }
            F::unpack(xv[j], f);
            if constexpr (YB) {
                y[0] = bf16_lo(yh[j][0]), y[1] = bf16_hi(yh[j][0]), y[2] = bf16_lo(yh[j][1]), y[3] = bf16_hi(yh[j][1]);
            } else {
                F::unpack(yv[j], y);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e)
                o[e] = fmaf(g[e], y[e], f[e]);
            xv[j] = F::pack4(o);
            __builtin_amdgcn_raw_buffer_store_b128(xv[j], so2, (lane + 64u * j) * 16u, 0, kNonTemporal);
        }
    }
    if constexpr (OP == kRmsMod || OP == kGateAddMod) {
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < NU; ++j)
            ss = F::sumsq(xv[j], ss);
        ss = row16_sum(ss);
        const float total = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ss), 0)) +
                            __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ss), 16)) +
                            __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ss), 32)) +
                            __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ss), 48));
        const float inv = 1.0f / sqrtf(fmaf(total, p.inv_dim, p.eps));
        const __amdgpu_buffer_rsrc_t so = buffer_rsrc(reinterpret_cast<const char*>(p.out) + uint64_t(row) * units * 8u,
                                                      units * 8u);
        const float* ta = ctab + set * p.dim;
        const float* tb = ctab + coef_total + set * p.dim;
#pragma unroll
        for (int j = 0; j < NU; ++j) {
            const uint32_t v = min(lane + 64u * j, units - 1u);
            float f[4], o[4], a[4], b[4];
            if constexpr (SRC == kCoefLds) {
                const float4 a4 = *reinterpret_cast<const float4*>(ta + v * 4u);
                const float4 b4 = *reinterpret_cast<const float4*>(tb + v * 4u);
                a[0] = a4.x, a[1] = a4.y, a[2] = a4.z, a[3] = a4.w;
                b[0] = b4.x, b[1] = b4.y, b[2] = b4.z, b[3] = b4.w;
            } else {
                float c[4];
                coef_vec<OP, 4>(p, set, v * 4u, a, b, c);
            }
            F::unpack(xv[j], f);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                o[e] = fmaf(f[e] * inv, a[e], b[e]);
            const u32x2_t h = {pack_bf16(o[0], o[1]), pack_bf16(o[2], o[3])};
            __builtin_amdgcn_raw_buffer_store_b64(h, so, (lane + 64u * j) * 8u, 0, kNonTemporal);
        }
    }
}

// ---- swiglu ---------------------------------------------------------------------------------------------------------

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

constexpr size_t kCoefLdsMax = 64 * 1024;
constexpr size_t kWaveLdsFloor = 54 * 1024; // above a third of gfx950's 160 KiB: two wave-kernel workgroups a CU
constexpr size_t kOrderLdsFloor = 81 * 1024; // above half of it: one workgroup a CU (the block's own order)
constexpr size_t kSwigluFusedLds = 40 * 1024; // four SwiGLU workgroups a CU (fused-row layout)
constexpr int kSwigluVecs = 1; // 16-byte vectors of gate (and of up) a thread has in flight

template <int DT, int VPT, int OP>
const void* pick_rows_kernel(int src)
{
    if (src == kCoefReg)
        return reinterpret_cast<const void*>(&rows_kernel<DT, VPT, OP, kCoefReg>);
    if (src == kCoefLds)
        return reinterpret_cast<const void*>(&rows_kernel<DT, VPT, OP, kCoefLds>);
    return reinterpret_cast<const void*>(&rows_kernel<DT, VPT, OP, kCoefGlobal>);
}

template <int DT, int NV, int OP>
const void* pick_wave_kernel(int src)
{
    if (src == kCoefLds)
        return reinterpret_cast<const void*>(&rows_wave_kernel<DT, NV, OP, kCoefLds>);
    return reinterpret_cast<const void*>(&rows_wave_kernel<DT, NV, OP, kCoefGlobal>);
}

template <int DT, int OP>
int launch_rows_wave(const RowsParams& p, hipStream_t stream)
{
    const uint32_t need = (p.nvec + 63u) / 64u;
    // The coefficients come from an LDS table the workgroup builds when it fits, else from the parameter vectors.
    const int src = size_t(p.n_sets) * p.dim * kPlanes<OP> * sizeof(float) <= kCoefLdsMax ? kCoefLds : kCoefGlobal;
    const void* k = nullptr;
    if (need <= 2)
        k = pick_wave_kernel<DT, 2, OP>(src);
    else if (need <= 4)
        k = pick_wave_kernel<DT, 4, OP>(src);
    else if (need <= 8)
        k = pick_wave_kernel<DT, 8, OP>(src);
    else if (need <= 10)
        k = pick_wave_kernel<DT, 10, OP>(src);
    else
        k = pick_wave_kernel<DT, 12, OP>(src);
    const uint32_t threads = kWaveBlock, waves = threads / 64u;
    // The dynamic LDS is at least kWaveLdsFloor, so two workgroups (16 waves, 16 rows in flight) share a CU. Fewer
    // rows in flight streamed faster than the registers would allow (at three or four 8-wave workgroups a CU: 5.79 to
    // 5.91 TB/s for the fused op at 768p), as fewer open streams contend for the DRAM banks; of one workgroup of 10 to
    // 16 waves, or two of 5 to 9, two of 7 or 8 were fastest, 0.5-1.6% ahead of one of 11 (alternating runs on one
    // GPU), since while one workgroup drains its last rows the other keeps the CU's loads going. A grid of persistent
    // workgroups, whose waves stride through far-apart rows, was 9-15% slower.
    // The block's own order (two read and two write streams) streams faster still with 8 rows in flight a CU: one
    // workgroup a CU measured 1.3% faster than two at 129,536 x 5120 (0.922-0.926 against 0.934-0.940 ms, alternated
    // on one GPU), while the fused op (one write stream) was 3% slower that way.
    const size_t table = src == kCoefLds ? size_t(p.n_sets) * p.dim * kPlanes<OP> * sizeof(float) : 0;
    const size_t floor = OP == kGateAddMod ? kOrderLdsFloor : kWaveLdsFloor;
    const size_t lds = table > floor ? table : floor;
    if (const hipError_t e = host::allow_dynamic_lds(k, lds); e != hipSuccess)
        return host::hip_error(e);
    // A row a wave; a persistent grid (rows_per_wave 0) measured slower.
    RowsParams arg = p;
    arg.rows_per_wave = 1;
    const uint64_t blocks = (uint64_t(p.rows) + waves - 1) / waves;
    void* args[] = {&arg};
    if (const hipError_t e = hipLaunchKernel(k, dim3(uint32_t(blocks)), dim3(threads), args, lds, stream);
        e != hipSuccess) {
        (void)hipGetLastError(); // the launch's error is reported here; clear it for the next call
        return host::hip_error(e);
    }
    return host::check_launch();
}

// The float stream with bf16 GEMM rows (flags): one wavefront a row, NU 4-column units a lane.
template <int OP, int YB, int SRC>
const void* pick_f32_stream_kernel(uint32_t units)
{
    const uint32_t need = (units + 63u) / 64u;
    if (need <= 4)
        return reinterpret_cast<const void*>(&rows_f32_stream_kernel<OP, YB, 4, SRC>);
    if (need <= 8)
        return reinterpret_cast<const void*>(&rows_f32_stream_kernel<OP, YB, 8, SRC>);
    if (need <= 16)
        return reinterpret_cast<const void*>(&rows_f32_stream_kernel<OP, YB, 16, SRC>);
    if (need <= 20)
        return reinterpret_cast<const void*>(&rows_f32_stream_kernel<OP, YB, 20, SRC>);
    return reinterpret_cast<const void*>(&rows_f32_stream_kernel<OP, YB, 24, SRC>);
}

template <int OP>
int launch_rows_f32_stream(const RowsParams& p, uint32_t flags, hipStream_t stream)
{
    // The coefficients come from an LDS table the workgroup builds when it fits, else from the parameter vectors.
    const bool in_lds = size_t(p.n_sets) * p.dim * kPlanes<OP> * sizeof(float) <= kCoefLdsMax;
    const bool yb = (flags & MH3_ROWS_Y_BF16) != 0;
    const void* k = in_lds ? (yb ? pick_f32_stream_kernel<OP, 1, kCoefLds>(p.nvec)
                                 : pick_f32_stream_kernel<OP, 0, kCoefLds>(p.nvec))
                           : (yb ? pick_f32_stream_kernel<OP, 1, kCoefGlobal>(p.nvec)
                                 : pick_f32_stream_kernel<OP, 0, kCoefGlobal>(p.nvec));
    const size_t table = in_lds ? size_t(p.n_sets) * p.dim * kPlanes<OP> * sizeof(float) : 0;
    const size_t floor = OP == kGateAddMod ? kOrderLdsFloor : kWaveLdsFloor;
    const size_t lds = table > floor ? table : floor;
    if (const hipError_t e = host::allow_dynamic_lds(k, lds); e != hipSuccess)
        return host::hip_error(e);
    RowsParams arg = p;
    const uint32_t waves = kWaveBlock / 64u;
    const uint64_t blocks = (uint64_t(p.rows) + waves - 1) / waves;
    void* args[] = {&arg};
    if (const hipError_t e = hipLaunchKernel(k, dim3(uint32_t(blocks)), dim3(kWaveBlock), args, lds, stream);
        e != hipSuccess) {
        (void)hipGetLastError();
        return host::hip_error(e);
    }
    return host::check_launch();
}

template <int DT, int OP>
int launch_rows_dt(const RowsParams& p, hipStream_t stream)
{
    // One wavefront a row when the row fits 12 vectors a lane and the two-plane coefficient table fits in LDS.
    if (p.nvec <= 12u * 64u && size_t(p.n_sets) * p.dim * 2 * sizeof(float) <= kCoefLdsMax)
        return launch_rows_wave<DT, OP>(p, stream);
    // (The choice between the two kernels depends on the two-plane table size for every op, so gate_add_mod reduces
    // in the same order as rms_mod and their norms agree bit for bit.)
    // Threads a row: enough for VPT vectors each, rounded up to whole waves.
    const size_t table = size_t(p.n_sets) * p.dim * kPlanes<OP> * sizeof(float);
    const int src = p.n_sets == 1 ? kCoefReg : (table <= kCoefLdsMax ? kCoefLds : kCoefGlobal);
    const void* k = nullptr;
    uint32_t threads = 0;
    if ((p.nvec + 1) / 2 <= 1024) {
        threads = ((p.nvec + 1) / 2 + 63) / 64 * 64;
        k = pick_rows_kernel<DT, 2, OP>(src);
    } else if ((p.nvec + 3) / 4 <= 1024) {
        threads = ((p.nvec + 3) / 4 + 63) / 64 * 64;
        k = pick_rows_kernel<DT, 4, OP>(src);
    } else {
        return MH3_ERR_UNSUPPORTED;
    }
    const size_t lds = 128 * sizeof(float) + (src == kCoefLds ? table : 0);
    const int per_cu = host::blocks_per_cu(k, int(threads), lds);
    // As many workgroups as keep every CU's slots busy once; each streams through its share of the rows.
    uint64_t blocks = p.rows;
    const uint64_t cap = uint64_t(host::cu_count()) * per_cu;
    if (blocks > cap)
        blocks = cap;
    RowsParams arg = p;
    void* args[] = {&arg};
    if (const hipError_t e = hipLaunchKernel(k, dim3(uint32_t(blocks)), dim3(threads), args, lds, stream);
        e != hipSuccess) {
        (void)hipGetLastError(); // the launch's error is reported here; clear it for the next call
        return host::hip_error(e);
    }
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
    p.set_stride = a->set_stride ? a->set_stride : a->dim;
    p.eps = a->eps;
    p.inv_dim = 1.0f / float(a->dim);
    if constexpr (OP != kFused) { // the fused op takes no flags (refused in its validation)
        if (a->flags) {
            p.nvec = a->dim / 4u; // 4-column units
            return launch_rows_f32_stream<OP>(p, a->flags, stream);
        }
    }
    return a->dtype == MH3_BF16 ? launch_rows_dt<MH3_BF16, OP>(p, stream) : launch_rows_dt<MH3_F32, OP>(p, stream);
}

// Shared validation of the row entry points. `needs_eps` for the normed ops; `allowed` the flags the entry point
// takes (with dtype MH3_F32 only: the float stream with bf16 GEMM rows).
int check_rows(const MH3RowsArgs* a, bool needs_eps, uint32_t allowed)
{
    if (!a)
        return MH3_ERR_POINTER;
    if (a->dtype != MH3_F32 && a->dtype != MH3_BF16)
        return MH3_ERR_PARAM;
    if (needs_eps && !(a->eps > 0.0f))
        return MH3_ERR_PARAM;
    if ((a->flags & ~allowed) != 0 || (a->flags && a->dtype != MH3_F32))
        return MH3_ERR_PARAM;
    const uint32_t e = a->dtype == MH3_BF16 || a->flags ? 8u : 4u;
    if (a->dim == 0 || a->dim % e != 0 || a->n_sets == 0 || a->n_sets > 256)
        return MH3_ERR_SHAPE;
    if (a->set_stride != 0 && (a->set_stride < a->dim || a->set_stride % 4 != 0))
        return MH3_ERR_PARAM;
    if (a->dim / e > (a->flags ? 12u * 64u : 4096u))
        return MH3_ERR_UNSUPPORTED;
    if (a->rows >= (1u << 31))
        return MH3_ERR_SHAPE;
    return MH3_OK;
}

// Bytes of a [rows][dim] row array: of the stream's dtype, or bf16 where `bf16` (a GEMM's row under the flags).
uint64_t row_bytes(const MH3RowsArgs* a, bool bf16)
{
    return uint64_t(a->rows) * a->dim * (bf16 || a->dtype == MH3_BF16 ? 2u : 4u);
}

// Aliasing rules of the row entry points. An output is a [rows][dim] array; it may equal an input row array of the
// same element type where `same_ok` (each wave or workgroup reads a row whole before it writes that row), but any
// other overlap with an input row array races across rows.
bool rows_clash(const MH3RowsArgs* a, const void* out, bool out_bf16, const void* in, bool in_bf16, bool same_ok)
{
    return in && host::overlaps(out, row_bytes(a, out_bf16), in, row_bytes(a, in_bf16)) &&
           !(same_ok && out == in && out_bf16 == in_bf16);
}

// Whether an output overlaps the vectors every workgroup reads: w [dim], shift / scale / gate (n_sets sets of dim
// floats, set_stride apart) and set_of_row [rows].
bool params_clash(const MH3RowsArgs* a, const void* out, bool out_bf16, const float* w, const float* shift,
                  const float* scale, const float* gate, const uint8_t* sets)
{
    const uint64_t bytes = row_bytes(a, out_bf16);
    const uint64_t vec = (uint64_t(a->n_sets - 1u) * (a->set_stride ? a->set_stride : a->dim) + a->dim) * 4u;
    return host::overlaps(out, bytes, w, w ? uint64_t(a->dim) * 4u : 0u) ||
           host::overlaps(out, bytes, shift, shift ? vec : 0u) || host::overlaps(out, bytes, scale, scale ? vec : 0u) ||
           host::overlaps(out, bytes, gate, gate ? vec : 0u) || host::overlaps(out, bytes, sets, sets ? a->rows : 0u);
}

} // namespace

extern "C" {

int mh3_rms_mod_rows(const MH3RowsArgs* args, const void* x, const float* w, const float* shift, const float* scale,
                     const uint8_t* set_of_row, void* y, mh3_stream_t stream)
{
    int rc = check_rows(args, true, MH3_ROWS_NORM_BF16);
    if (rc != MH3_OK)
        return rc;
    if (args->rows == 0)
        return MH3_OK;
    if (!x || !shift || !scale || !y)
        return MH3_ERR_POINTER;
    if (!host::aligned16(x) || !host::aligned16(y) || !host::aligned16(w) || !host::aligned16(shift) ||
        !host::aligned16(scale))
        return MH3_ERR_ALIGN;
    const bool yb = (args->flags & MH3_ROWS_NORM_BF16) != 0;
    if (rows_clash(args, y, yb, x, false, true) || params_clash(args, y, yb, w, shift, scale, nullptr, set_of_row))
        return MH3_ERR_PARAM;
    RowsParams p{};
    p.x = static_cast<const u32x4_t*>(x);
    p.out = static_cast<u32x4_t*>(y);
    p.w = w;
    p.shift = shift;
    p.scale = scale;
    p.set_of_row = set_of_row;
    return launch_rows<kRmsMod>(args, p, static_cast<hipStream_t>(stream));
}

int mh3_gate_add_rows(const MH3RowsArgs* args, void* x, const void* y, const float* gate, const uint8_t* set_of_row,
                      mh3_stream_t stream)
{
    int rc = check_rows(args, false, MH3_ROWS_Y_BF16);
    if (rc != MH3_OK)
        return rc;
    if (args->rows == 0)
        return MH3_OK;
    if (!x || !y || !gate)
        return MH3_ERR_POINTER;
    if (!host::aligned16(x) || !host::aligned16(y) || !host::aligned16(gate))
        return MH3_ERR_ALIGN;
    const bool yb = (args->flags & MH3_ROWS_Y_BF16) != 0;
    if (rows_clash(args, x, false, y, yb, true) ||
        params_clash(args, x, false, nullptr, nullptr, nullptr, gate, set_of_row))
        return MH3_ERR_PARAM;
    RowsParams p{};
    p.x = static_cast<const u32x4_t*>(y);
    p.res = static_cast<const u32x4_t*>(x);
    p.out = static_cast<u32x4_t*>(x);
    p.out2 = static_cast<u32x4_t*>(x); // the float stream's kernel writes the updated x here
    p.gate = gate;
    p.set_of_row = set_of_row;
    return launch_rows<kGateAdd>(args, p, static_cast<hipStream_t>(stream));
}

int mh3_rms_mod_gate_add_rows(const MH3RowsArgs* args, const void* x, const void* residual, const float* w,
                              const float* shift, const float* scale, const float* gate, const uint8_t* set_of_row,
                              void* out, mh3_stream_t stream)
{
    int rc = check_rows(args, true, 0u);
    if (rc != MH3_OK)
        return rc;
    if (args->rows == 0)
        return MH3_OK;
    if (!x || !residual || !shift || !scale || !gate || !out)
        return MH3_ERR_POINTER;
    if (!host::aligned16(x) || !host::aligned16(residual) || !host::aligned16(out) || !host::aligned16(w) ||
        !host::aligned16(shift) || !host::aligned16(scale) || !host::aligned16(gate))
        return MH3_ERR_ALIGN;
    if (rows_clash(args, out, false, x, false, true) || rows_clash(args, out, false, residual, false, true) ||
        params_clash(args, out, false, w, shift, scale, gate, set_of_row))
        return MH3_ERR_PARAM;
    RowsParams p{};
    p.x = static_cast<const u32x4_t*>(x);
    p.res = static_cast<const u32x4_t*>(residual);
    p.out = static_cast<u32x4_t*>(out);
    p.w = w;
    p.shift = shift;
    p.scale = scale;
    p.gate = gate;
    p.set_of_row = set_of_row;
    return launch_rows<kFused>(args, p, static_cast<hipStream_t>(stream));
}

int mh3_gate_add_rms_mod_rows(const MH3RowsArgs* args, void* x, const void* y, const float* gate, const float* w,
                              const float* shift, const float* scale, const uint8_t* set_of_row, void* h,
                              mh3_stream_t stream)
{
    // Flags: none, a bf16 h, or a bf16 h from a bf16 y (a bf16 y alone would need a float norm of its own order).
    int rc = check_rows(args, true, MH3_ROWS_NORM_BF16 | MH3_ROWS_Y_BF16);
    if (rc != MH3_OK)
        return rc;
    if (args->flags == MH3_ROWS_Y_BF16)
        return MH3_ERR_PARAM;
    if (args->rows == 0)
        return MH3_OK;
    if (!x || !y || !gate || !shift || !scale || !h)
        return MH3_ERR_POINTER;
    if (h == x || h == y)
        return MH3_ERR_PARAM; // h is a separate tensor
    if (!host::aligned16(x) || !host::aligned16(y) || !host::aligned16(h) || !host::aligned16(gate) ||
        !host::aligned16(w) || !host::aligned16(shift) || !host::aligned16(scale))
        return MH3_ERR_ALIGN;
    const bool hb = (args->flags & MH3_ROWS_NORM_BF16) != 0, yb = (args->flags & MH3_ROWS_Y_BF16) != 0;
    if (rows_clash(args, h, hb, x, false, false) || rows_clash(args, h, hb, y, yb, false) ||
        rows_clash(args, x, false, y, yb, true) || params_clash(args, h, hb, w, shift, scale, gate, set_of_row) ||
        params_clash(args, x, false, w, shift, scale, gate, set_of_row))
        return MH3_ERR_PARAM;
    RowsParams p{};
    p.x = static_cast<const u32x4_t*>(y);
    p.res = static_cast<const u32x4_t*>(x);
    p.out2 = static_cast<u32x4_t*>(x);
    p.out = static_cast<u32x4_t*>(h);
    p.w = w;
    p.shift = shift;
    p.scale = scale;
    p.gate = gate;
    p.set_of_row = set_of_row;
    return launch_rows<kGateAddMod>(args, p, static_cast<hipStream_t>(stream));
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
    {
        // out may equal gate or up in the split layout (elementwise in place); any other overlap races.
        const uint64_t ob = uint64_t(a->rows) * vpr * 16u;
        const uint64_t gb = a->layout == MH3_SWIGLU_FUSED ? 2u * ob : ob;
        const bool split = a->layout == MH3_SWIGLU_SPLIT;
        if ((host::overlaps(out, ob, gate, gb) && !(split && out == gate)) ||
            (up && host::overlaps(out, ob, up, ob) && out != up))
            return MH3_ERR_PARAM;
    }
    const uint4* g = static_cast<const uint4*>(gate);
    const uint4* u = a->layout == MH3_SWIGLU_FUSED ? g + vpr : static_cast<const uint4*>(up);
    const uint32_t stride = a->layout == MH3_SWIGLU_FUSED ? 2u * vpr : vpr;
    const uint32_t total = a->rows * vpr;
    constexpr int U = kSwigluVecs;
    const uint32_t blocks = (total + 256u * U - 1) / (256u * U);
    const FastDiv div = FastDiv::make(vpr);
    hipStream_t s = static_cast<hipStream_t>(stream);
    // The fused-row layout reads its two streams from one array, a half row apart: there four workgroups a CU (the LDS
    // they reserve allows no more) streamed 1.5% faster than the ten the registers allow (6.47 against 6.38 TB/s at
    // 768p, alternating runs); the split layout measured best unlimited (6.53 against 6.17 TB/s).
    const size_t lds = a->layout == MH3_SWIGLU_FUSED ? kSwigluFusedLds : 0;
    if (a->dtype == MH3_BF16)
        hipLaunchKernelGGL((swiglu_kernel<MH3_BF16, U>), dim3(blocks), dim3(256), lds, s, g, u,
                           static_cast<uint4*>(out), vpr, stride, stride, total, div);
    else
        hipLaunchKernelGGL((swiglu_kernel<MH3_F32, U>), dim3(blocks), dim3(256), lds, s, g, u,
                           static_cast<uint4*>(out), vpr, stride, stride, total, div);
    return host::check_launch();
}

} // extern "C"
