// fc1 as an int8 weight-only GEMM with the SwiGLU epilogue: out = silu(x Wg sg) * (x Wu su).
// Replaces the reference's `gemm_i8` + `swiglu_rows` pair for fc1 (mako-common; docs/performance.md:120-136,
// docs/architecture.md:65: fc1's [gate; value] rows, then SwiGLU).
//
// Design (gfx950, v_mfma_f32_32x32x16_bf16):
// - A workgroup of 4 wavefronts computes a 256-row x 128-column output tile, i.e. the 128 gate columns [n0, n0+128)
//   and the 128 up columns [n + n0, n + n0 + 128) of y, so the SwiGLU epilogue has both halves in registers. Each
//   wave owns 128 rows x (64 gate + 64 up) columns: 4 x 4 MFMA tiles of 32 x 32, 256 float accumulators.
// - K advances 64 at a time through two LDS stages (A 256x64 bf16 and B 256x64 bf16 = 64 KiB a stage). The int8
//   weights are loaded as 16-byte vectors and widened to bf16 on the way into LDS (exact: |w| <= 127 fits bf16's
//   8-bit significand), so the dequantization costs no extra HBM or LDS traffic and the scale is applied once to the
//   float accumulator in the epilogue: x (W diag s) = (x W) diag s.
// - LDS rows are 128 bytes; the 16-byte chunk c of row r is stored at chunk c ^ (r & 7), so the MFMA operand reads
//   (32 rows at one chunk per half-wave) hit distinct banks.
// - Workgroups are mapped XCD-aware: the hardware deals workgroup b to XCD b % 8, so consecutive tiles are renumbered
//   onto one XCD, and grouped 4 row-tiles a band so the tiles running together on an XCD share x and w in its L2.
#include "mh3_common.hpp"

namespace mh3 {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr uint32_t kBM = 256, kBN = 128, kBK = 64;
constexpr int kGemmThreads = 256;
constexpr uint32_t kStageChunks = 4096; // 16-byte chunks a stage: A 256 x 8, then B 256 x 8
constexpr size_t kGemmLds = 2 * kStageChunks * 16;
constexpr uint32_t kBandM = 4;

__device__ __forceinline__ uint32_t swz(uint32_t row, uint32_t chunk) { return row * 8u + (chunk ^ (row & 7u)); }

// 16 int8 weights (one 16-byte vector) to 16 bf16 (two 16-byte vectors), exactly.
__device__ __forceinline__ void widen16(const u32x4_t& v, u32x4_t& lo, u32x4_t& hi)
{
    const uint32_t w[4] = {v[0], v[1], v[2], v[3]};
    uint32_t o[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float f0 = float(int32_t(w[i] << 24) >> 24);
        const float f1 = float(int32_t(w[i] << 16) >> 24);
        const float f2 = float(int32_t(w[i] << 8) >> 24);
        const float f3 = float(int32_t(w[i]) >> 24);
        o[2 * i] = (__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xffff0000u);
        o[2 * i + 1] = (__float_as_uint(f2) >> 16) | (__float_as_uint(f3) & 0xffff0000u);
    }
    lo = u32x4_t{o[0], o[1], o[2], o[3]};
    hi = u32x4_t{o[4], o[5], o[6], o[7]};
}

__device__ __forceinline__ void tile_of(uint32_t mt, uint32_t nt, uint32_t& tm, uint32_t& tn)
{
    const uint32_t nb = gridDim.x, b = blockIdx.x;
    const uint32_t logical = (nb % 8u == 0u) ? (b % 8u) * (nb / 8u) + b / 8u : b;
    const uint32_t band = logical / (kBandM * nt), within = logical - band * kBandM * nt;
    const uint32_t in_band = min(kBandM, mt - band * kBandM);
    tm = band * kBandM + within % in_band;
    tn = within / in_band;
}

__global__ __launch_bounds__(kGemmThreads) void gemm_w8a16_swiglu_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ w, const float* __restrict__ scale,
    uint16_t* __restrict__ out, uint32_t M, uint32_t N, uint32_t K, uint32_t mt, uint32_t nt)
{
    extern __shared__ uint4 smem[];
    uint32_t tm, tn;
    tile_of(mt, nt, tm, tn);
    const uint32_t m0 = tm * kBM, n0 = tn * kBN;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6, wm = wave >> 1, wn = wave & 1u;

    // Global -> register assignment, through buffer descriptors based at this tile (32-bit lane offsets; reads past
    // the descriptor's extent return zero, which covers the rows past M). A: chunk c = tid + 256 i (i < 8) is tile row
    // c / 8 = tid / 8 + 32 i, k-chunk c % 8 (8 bf16). B: chunk c = tid + 256 i (i < 4) is B-row c / 4 = tid / 4 + 64 i
    // (0..127 the gate rows n0.., 128..255 the up rows n + n0..), k-chunk c % 4 (16 int8).
    const uint64_t a_left = uint64_t(M - m0) * K * 2u;
    const __amdgpu_buffer_rsrc_t ra_src = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(x + uint64_t(m0) * K), 0, int(a_left < 0x7fffffffu ? a_left : 0x7fffffffu), kRsrcFlags);
    const __amdgpu_buffer_rsrc_t rg_src = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(w + uint64_t(n0) * K), 0, int(kBN * K), kRsrcFlags);
    const __amdgpu_buffer_rsrc_t ru_src = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(w + (uint64_t(N) + n0) * K), 0, int(kBN * K), kRsrcFlags);
    uint32_t a_off[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
        a_off[i] = ((tid >> 3) + 32u * i) * K * 2u + (tid & 7u) * 16u;
    const uint32_t b_off0 = (tid >> 2) * K + (tid & 3u) * 16u, b_off1 = b_off0 + 64u * K;
    u32x4_t ra[8], rb[4];
    auto gload = [&](uint32_t kt) {
        const int sa = int(kt * kBK * 2u), sb = int(kt * kBK);
#pragma unroll
        for (int i = 0; i < 8; ++i)
            ra[i] = __builtin_amdgcn_raw_buffer_load_b128(ra_src, a_off[i], sa, 0);
        rb[0] = __builtin_amdgcn_raw_buffer_load_b128(rg_src, b_off0, sb, 0);
        rb[1] = __builtin_amdgcn_raw_buffer_load_b128(rg_src, b_off1, sb, 0);
        rb[2] = __builtin_amdgcn_raw_buffer_load_b128(ru_src, b_off0, sb, 0);
        rb[3] = __builtin_amdgcn_raw_buffer_load_b128(ru_src, b_off1, sb, 0);
    };
    auto swrite = [&](uint32_t stage) {
        u32x4_t* A = reinterpret_cast<u32x4_t*>(smem) + stage * kStageChunks;
        u32x4_t* B = A + kStageChunks / 2;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t c = tid + 256u * i;
            A[swz(c >> 3, c & 7u)] = ra[i];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t c = tid + 256u * i, brow = c >> 2, kc = c & 3u;
            u32x4_t lo, hi;
            widen16(rb[i], lo, hi);
            B[swz(brow, 2u * kc)] = lo;
            B[swz(brow, 2u * kc + 1u)] = hi;
        }
    };

    floatx16 acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int e = 0; e < 16; ++e)
                acc[a][b][e] = 0.0f;

    const uint32_t KT = K / kBK;
    gload(0);
    swrite(0);
    __syncthreads();
    const uint32_t half = lane >> 5, r32 = lane & 31u;
    // LDS chunk of this lane's operand rows: A rows wm*128 + t*32 + r32, B rows (gate) wn*64 + t*32 + r32 and
    // (up) 128 + wn*64 + (t-2)*32 + r32; the k-chunk (ks*2 + half) is XOR-swizzled by the row.
    auto load_frags = [&](const uint4* A, const uint4* B, uint32_t ks, bf16x8_t (&fa)[4], bf16x8_t (&fb)[4]) {
#pragma unroll
        for (uint32_t t = 0; t < 4; ++t) {
            const uint32_t row = wm * 128u + t * 32u + r32;
            fa[t] = __builtin_bit_cast(bf16x8_t, A[swz(row, ks * 2u + half)]);
            const uint32_t brow = (t < 2 ? wn * 64u + t * 32u : kBN + wn * 64u + (t - 2u) * 32u) + r32;
            fb[t] = __builtin_bit_cast(bf16x8_t, B[swz(brow, ks * 2u + half)]);
        }
    };
    for (uint32_t kt = 0; kt < KT; ++kt) {
        if (kt + 1 < KT)
            gload(kt + 1);
        const uint4* A = smem + (kt & 1u) * kStageChunks;
        const uint4* B = A + kStageChunks / 2;
        bf16x8_t fa[2][4], fb[2][4];
        load_frags(A, B, 0, fa[0], fb[0]);
#pragma unroll
        for (uint32_t ks = 0; ks < kBK / 16u; ++ks) {
            // The next sub-step's operands are read from LDS while this sub-step's 16 MFMAs run.
            if (ks + 1 < kBK / 16u)
                load_frags(A, B, ks + 1, fa[(ks + 1) & 1u], fb[(ks + 1) & 1u]);
            __builtin_amdgcn_sched_barrier(0); // keep those reads ahead of this sub-step's MFMAs
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[ks & 1u][a], fb[ks & 1u][b], acc[a][b],
                                                                         0, 0, 0);
        }
        if (kt + 1 < KT)
            swrite((kt + 1) & 1u);
        __syncthreads();
    }

    // Epilogue: acc[a][b][e] is y[row][col] with row = m0 + wm 128 + a 32 + 8 (e / 4) + 4 (lane / 32) + e % 4 and
    // col = lane % 32 + 32 b within the wave's columns (b < 2: gate, b >= 2: the matching up columns).
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const uint32_t col = n0 + wn * 64u + uint32_t(b) * 32u + r32;
        const float sg = scale[col], su = scale[N + col];
#pragma unroll
        for (int a = 0; a < 4; ++a) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const uint32_t row = m0 + wm * 128u + uint32_t(a) * 32u + 8u * (uint32_t(e) >> 2) + 4u * half +
                                     (uint32_t(e) & 3u);
                if (row < M) {
                    const float g = acc[a][b][e] * sg, u = acc[a][b + 2][e] * su;
                    const float o = g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
                    out[uint64_t(row) * N + col] = __builtin_bit_cast(uint16_t, __bf16(o));
                }
            }
        }
    }
}

} // namespace mh3

extern "C" int mh3_gemm_w8a16_swiglu(const MH3GemmArgs* a, const uint16_t* x, const int8_t* w, const float* scale,
                                     uint16_t* out, mh3_stream_t stream)
{
    using namespace mh3;
    if (!a)
        return MH3_ERR_POINTER;
    if (a->m == 0 || a->k == 0 || a->n == 0 || a->k % kBK != 0 || a->n % kBN != 0)
        return MH3_ERR_SHAPE;
    if (a->m >= (1u << 31) || uint64_t(a->n) * 2u >= (uint64_t(1) << 31))
        return MH3_ERR_SHAPE;
    if (!x || !w || !scale || !out)
        return MH3_ERR_POINTER;
    if (!host::aligned16(x) || !host::aligned16(w) || !host::aligned16(out))
        return MH3_ERR_ALIGN;
    static const int lds_ok = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_w8a16_swiglu_kernel),
                                                  hipFuncAttributeMaxDynamicSharedMemorySize, int(kGemmLds));
    if (lds_ok != hipSuccess)
        return MH3_ERR_HIP;
    const uint32_t mt = (a->m + kBM - 1) / kBM, nt = a->n / kBN;
    const uint64_t tiles = uint64_t(mt) * nt;
    if (tiles >= (uint64_t(1) << 31))
        return MH3_ERR_SHAPE;
    hipLaunchKernelGGL(gemm_w8a16_swiglu_kernel, dim3(uint32_t(tiles)), dim3(kGemmThreads), kGemmLds,
                       static_cast<hipStream_t>(stream), x, w, scale, out, a->m, a->n, a->k, mt, nt);
    return host::check_launch();
}
