// The block's GEMMs on one kernel. fc1 as an int8 weight-only GEMM with the SwiGLU epilogue:
// out = silu(x Wg sg) * (x Wu su), replacing the reference's `gemm_i8` + `swiglu_rows` pair for fc1 (mako-common;
// docs/performance.md:120-136, docs/architecture.md:65: fc1's [gate; value] rows, then SwiGLU). The same kernel with
// bf16 weights is the dense fc1 of the `--int8 none` path (the reference's bf16 `Gemm::encode`,
// docs/performance.md:52-69): its B tiles then stream into LDS like A's, one K-step ahead, and there is no scale.
// With int8 x as well (W8A8, the reference's own `gemm_i8`: activations quantized per row) both operands stream
// into LDS and the int8 MFMA (v_mfma_i32_16x16x64_i8, exact int32 sums) takes 128 k a K-step; the epilogue applies
// both scales. Two more epilogues make the same kernel the qkv projection (a plain store) and the out and fc2
// projections (gate_add_rows folded in: the residual += gate * y, in place).
//
// Design (gfx950, v_mfma_f32_16x16x32_bf16):
// - A workgroup of 8 wavefronts (2 along rows x 4 along columns) computes a 256-row x 128-column output tile, i.e.
//   the 128 gate columns [n0, n0+128) and the 128 up columns [n + n0, n + n0 + 128) of y, so the SwiGLU epilogue has
//   both halves in registers. Each wave owns 128 rows x (32 gate + 32 up) columns: 8 x 4 MFMA tiles of 16 x 16.
// - K advances 64 at a time. A (x, bf16) streams from HBM straight into a 3-stage LDS ring with buffer loads that
//   write LDS (no VGPR round trip); B (int8 w) is loaded as 16-byte vectors into registers one K-step ahead and
//   widened to bf16 into a 2-stage LDS ring (exact: |w| <= 127 fits bf16's 8-bit significand), so dequantization
//   costs no extra HBM traffic and the scale is applied once to the float accumulator in the epilogue:
//   x (W diag s) = (x W) diag s. The five stages fill gfx950's 160 KiB of LDS.
// - LDS rows are 128 bytes; the 16-byte chunk c of row r is stored at chunk c ^ ((r >> 1) & 7), so the MFMA operand
//   reads (16 rows at one chunk per quarter-wave) hit distinct banks, and B's 16-byte writes are spread over 8 chunk
//   columns per 8 lanes by the chunk-to-thread mapping.
// - Workgroups are mapped XCD-aware: the hardware deals workgroup b to XCD b % 8, so consecutive tiles are renumbered
//   onto one XCD, and grouped 4 row-tiles a band so the tiles running together on an XCD share x and w in its L2.
// - The epilogue goes through the LDS, idle by then: results staged as floats, then written (and the gate-add
//   residual read) in coalesced 16-byte accesses.
// - 16 x 16 MFMA tiles rather than 32 x 32: the matrix cores sustain a higher clock on them under the same power
//   limit (a register-only loop of random operands: 1.91 against 1.69-1.76 GHz at 98% busy), with the same LDS bytes
//   a flop for the same wave tile.
// - 4 wavefronts of 128 x 128 (fewer LDS bytes a MFMA) measured 10-15% slower than these 8: with one wave a SIMD
//   nothing hides the fragment reads and the barrier.
#include "mh3_common.hpp"

#include <type_traits>

namespace mh3 {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kBM = 256, kBN = 128, kBK = 64;
// LDS: a ring of 3 A stages (256 rows x 64 k bf16 = 2048 16-byte chunks each), then 2 B stages (256 B-rows x 64 k,
// widened to bf16: 2048 chunks each): 160 KiB, gfx950's whole LDS.
constexpr uint32_t kStageChunks = 2048, kAStages = 3, kBStages = 2;
constexpr uint32_t kBBase = kAStages * kStageChunks;
constexpr size_t kGemmLds = size_t(kAStages + kBStages) * kStageChunks * 16;
constexpr uint32_t kBandM = 4; // row tiles an XCD sweeps across all column tiles before moving on

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// 16 bytes a lane from a buffer straight into LDS: lane L's bytes land at lds + 16 L (buffer_load_dwordx4 ... lds).
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t rsrc, void* lds, uint32_t voffset, int soffset)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_ptr_t)lds, 16, voffset, soffset, 0, 0);
}

// 16-byte chunk c of a 128-byte LDS row r sits at chunk c ^ ((r >> 1) & 7): the 16 rows an MFMA operand read touches
// per half-wave then cover all 64 banks once.
__device__ __forceinline__ uint32_t swz(uint32_t row, uint32_t chunk) { return row * 8u + (chunk ^ ((row >> 1) & 7u)); }

// 8 int8 weights (two dwords) to 8 bf16 (one 16-byte vector), exactly: each byte to float, then the upper halves
// of two floats are the bf16 pair (|w| <= 127 has at most 8 significant bits, so the truncation is exact).
__device__ __forceinline__ u32x4_t widen8(uint32_t w0, uint32_t w1)
{
    u32x4_t r;
#pragma unroll
    for (int d = 0; d < 2; ++d) {
        const uint32_t w = d ? w1 : w0;
        const float f0 = float(int32_t(w << 24) >> 24);
        const float f1 = float(int32_t(w << 16) >> 24);
        const float f2 = float(int32_t(w << 8) >> 24);
        const float f3 = float(int32_t(w) >> 24);
        r[2 * d] = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
        r[2 * d + 1] = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
    }
    return r;
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

// s_waitcnt immediate that waits for vmcnt <= n only (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4,
// lgkmcnt 11:8).
constexpr int waitcnt_vm(int n) { return (n & 0xF) | (((n >> 4) & 3) << 14) | (0x7 << 4) | (0xF << 8); }

// All LDS accesses before it done, then the workgroup barrier; the asm statements keep the compiler from moving
// memory accesses across it.
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F); // lgkmcnt(0), vmcnt and expcnt unconstrained
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

constexpr int kGemmWM = 2; // wavefronts along the tile's rows
constexpr int kGemmWN = 4; // wavefronts along its columns

// The three fc1 forms: int8 weights widened to bf16 with bf16 activations (weight-only), bf16 weights, and int8
// weights with int8 activations (each row of x with its own scale) on the int8 MFMA.
enum GemmMode { kW8A16 = 0, kBf16 = 1, kW8A8 = 2 };
// What the epilogue does with y = x w^T (scaled):
//   kSwiGLU:  out[m][N] = silu(y gate column) * y up column; w holds N gate rows then N up rows (fc1);
//   kStore:   out[m][N] = y; w holds N rows (the qkv projection);
//   kGateAdd: out[m][N] += gate[set(row)] * y, in place on the bf16 residual (the out projection and fc2, with the
//             reference's gate_add_rows folded in);
//   kGateAddF32: the same on a float residual (the reference's float residual stream), out read as float [m][N].
// With kSwiGLU a tile's 256 weight rows are 128 gate rows from n0 and the 128 matching up rows from N + n0; otherwise
// they are 256 consecutive rows, so both halves of the wave's accumulators are output columns.
enum GemmEpi { kSwiGLU = 0, kStore = 1, kGateAdd = 2, kGateAddF32 = 3 };

// The epilogue's extra operands (kGateAdd): gate vectors [n_sets][gate_stride] floats, a set per row (NULL: set 0).
struct GemmGate {
    const float* gate;
    const uint8_t* set_of_row;
    uint32_t gate_stride, n_sets;
};

typedef int int32x4 __attribute__((ext_vector_type(4)));

// The epilogue shared by the GEMM kernels, through the LDS (idle after the last K-step). acc[a][b][e] is y[r][c]
// with c = lane % 16 + 16 b + wn 16 TN within the tile's first 128 w rows (b < TN) or, for acc[a][TN + b], the same
// position in its second 128, and tile row r = wm (256 / WM) + a 16 + 4 (lane / 16) + e. A
// 128-column half of the tile at a time, each wave writes its scaled results as floats into a [256][kEpiStride] LDS
// tile (the two half-waves' rows, 4 apart, fall on disjoint banks); then each thread takes 8 consecutive columns of
// a row, so the output, and with kGateAdd the residual, moves in 16-byte accesses, 16 threads to a row's 256 bytes.
// The results round to bf16 once, at the end, as they would written straight from the registers.
template <int WM, int WN, int MODE, int EPI, int TM, int TN, typename Acc>
__device__ __forceinline__ void gemm_epilogue(Acc (&acc)[TM][2 * TN], u32x4_t* smem, uint32_t M, uint32_t N,
                                              uint32_t m0, uint32_t w_lo, uint32_t w_hi,
                                              const float* __restrict__ scale, const float* __restrict__ xscale,
                                              uint16_t* __restrict__ out, const GemmGate& gg)
{
    constexpr uint32_t kThreads = WM * WN * 64;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6, wm = wave / WN, wn = wave % WN;
    const uint32_t rl = lane % 16u;
    constexpr uint32_t kEpiStride = kBN + 8u; // floats a staged row: 4 rows apart = 32 banks apart
    static_assert(kBM * kEpiStride * sizeof(float) <= kGemmLds, "the staged half-tile fits in the LDS");
    constexpr int kHalves = EPI == kSwiGLU ? 1 : 2;
    float* const stage = reinterpret_cast<float*>(smem);
    lds_barrier(); // every wave is done with the last K-step's fragments
#pragma unroll
    for (int hv = 0; hv < kHalves; ++hv) {
        if (hv)
            lds_barrier(); // the first half is read out
#pragma unroll
        for (int b = 0; b < TN; ++b) {
            const uint32_t c = wn * 16u * TN + uint32_t(b) * 16u + rl;
            const float s_lo = MODE != kBf16 ? scale[w_lo + c] : 1.0f, s_hi = MODE != kBf16 ? scale[w_hi + c] : 1.0f;
#pragma unroll
            for (int a = 0; a < TM; ++a) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t r = wm * (kBM / WM) + uint32_t(a) * 16u + 4u * (lane >> 4) + uint32_t(e);
                    const float sx = MODE == kW8A8 ? xscale[min(m0 + r, M - 1u)] : 1.0f;
                    float v;
                    if constexpr (EPI == kSwiGLU) {
                        const float lo = float(acc[a][b][e]) * s_lo * sx, hi = float(acc[a][TN + b][e]) * s_hi * sx;
                        v = lo * __builtin_amdgcn_rcpf(1.0f + __expf(-lo)) * hi;
                    } else {
                        v = hv == 0 ? float(acc[a][b][e]) * s_lo * sx : float(acc[a][TN + b][e]) * s_hi * sx;
                    }
                    stage[r * kEpiStride + c] = v;
                }
            }
        }
        lds_barrier();
        // Output column of staged column 0: the tile's gate columns (SwiGLU), else its first or second 128 columns.
        const uint32_t col0 = hv == 0 ? w_lo : w_hi;
        for (uint32_t q = tid; q < kBM * 16u; q += kThreads) {
            const uint32_t r = q >> 4, c8 = (q & 15u) * 8u, row = m0 + r;
            if (row >= M)
                break; // rows grow with q
            const float4 v0 = *reinterpret_cast<const float4*>(stage + r * kEpiStride + c8);
            const float4 v1 = *reinterpret_cast<const float4*>(stage + r * kEpiStride + c8 + 4u);
            float o[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
            if constexpr (EPI == kGateAddF32) {
                // The float residual: 32 bytes a thread, x += gate * y with one float rounding.
                const uint32_t set = gg.set_of_row ? min(uint32_t(gg.set_of_row[row]), gg.n_sets - 1u) : 0u;
                const float* g = gg.gate + uint64_t(set) * gg.gate_stride + col0 + c8;
                float4* fdst = reinterpret_cast<float4*>(reinterpret_cast<float*>(out) + uint64_t(row) * N + col0 + c8);
                const float4 r0 = fdst[0], r1 = fdst[1];
                fdst[0] = float4{fmaf(g[0], o[0], r0.x), fmaf(g[1], o[1], r0.y), fmaf(g[2], o[2], r0.z),
                                 fmaf(g[3], o[3], r0.w)};
                fdst[1] = float4{fmaf(g[4], o[4], r1.x), fmaf(g[5], o[5], r1.y), fmaf(g[6], o[6], r1.z),
                                 fmaf(g[7], o[7], r1.w)};
                continue;
            }
            uint4* dst = reinterpret_cast<uint4*>(out + uint64_t(row) * N + col0 + c8);
            if constexpr (EPI == kGateAdd) {
                const uint32_t set = gg.set_of_row ? min(uint32_t(gg.set_of_row[row]), gg.n_sets - 1u) : 0u;
                const float* g = gg.gate + uint64_t(set) * gg.gate_stride + col0 + c8;
                const uint4 res = *dst;
                const uint32_t rw[4] = {res.x, res.y, res.z, res.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    o[2 * i] = fmaf(g[2 * i], o[2 * i], bf16_lo(rw[i]));
                    o[2 * i + 1] = fmaf(g[2 * i + 1], o[2 * i + 1], bf16_hi(rw[i]));
                }
            }
            *dst = uint4{pack_bf16(o[0], o[1]), pack_bf16(o[2], o[3]), pack_bf16(o[4], o[5]), pack_bf16(o[6], o[7])};
        }
    }
}

// WM x WN wavefronts: wave (wm, wn) computes rows wm * (256 / WM) ... of the tile against its TN gate column tiles
// (16 columns each, from wn * 16 TN) and the TN matching up column tiles, on 16 x 16 MFMA tiles
// (v_mfma_f32_16x16x32_bf16, v_mfma_i32_16x16x64_i8). Every LDS row holds 128 bytes of k: 64 k of bf16 or 128 k of
// int8, so a K-step is 64 or 128 k.
template <int WM, int WN, int MODE, int EPI>
__global__ __launch_bounds__(kGemmWM * kGemmWN * 64) void gemm_kernel(
    const void* __restrict__ xv, const void* __restrict__ wv, const float* __restrict__ scale,
    const float* __restrict__ xscale, uint16_t* __restrict__ out, uint32_t M, uint32_t N, uint32_t K, uint32_t mt,
    uint32_t nt, GemmGate gg)
{
    constexpr bool I8 = MODE == kW8A16;                   // B through registers, widened
    constexpr uint32_t kEA = MODE == kW8A8 ? 1u : 2u;     // bytes of an x element
    constexpr uint32_t kEB = MODE == kBf16 ? 2u : 1u;     // bytes of a w element
    constexpr uint32_t kKS = 128u / kEA;                  // k of a K-step
    using Acc = typename std::conditional<MODE == kW8A8, int32x4, floatx4>::type;
    constexpr uint32_t kThreads = WM * WN * 64, kWaves = WM * WN;
    constexpr int TM = int(kBM / WM / 16), TN = int(kBN / WN / 16); // MFMA tiles: rows, and gate (= up) columns
    // Row tiles whose A fragments a sub-step holds: half of them (a sub-step is one 32-k half of the K-step over one
    // half of the wave's rows).
    constexpr int FA = TM / 2;
    extern __shared__ u32x4_t smem[];
    uint32_t tm, tn;
    tile_of(mt, nt, tm, tn);
    const uint32_t m0 = tm * kBM;
    // The tile's two 128-row halves of w (and the output columns they give): gate and up rows, or consecutive rows.
    const uint32_t w_lo = EPI == kSwiGLU ? tn * kBN : tn * 2u * kBN;
    const uint32_t w_hi = EPI == kSwiGLU ? N + w_lo : w_lo + kBN;
    const uint32_t w_rows = EPI == kSwiGLU ? 2u * N : N;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6, wm = wave / WN, wn = wave % WN;
    const uint32_t KT = K / kKS;

    // A: straight from global memory into the LDS ring (buffer_load ... lds). A stage is 2048 16-byte chunks; each
    // wave fills 2048 / kWaves of them, 64 a instruction; lane L of instruction i lands in chunk q = (wave * AI + i) *
    // 64 + L = row * 8 + physical chunk and fetches the logical chunk the swizzle puts there. The descriptor starts
    // at this tile's first row; rows past M read zero.
    constexpr int AI = int(kStageChunks / 64 / kWaves);
    const uint64_t a_left = uint64_t(M - m0) * K * kEA;
    const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(reinterpret_cast<const char*>(xv) + uint64_t(m0) * K * kEA,
                                                  uint32_t(a_left < 0x7fffffffu ? a_left : 0x7fffffffu));
    uint32_t a_off[AI];
#pragma unroll
    for (int i = 0; i < AI; ++i) {
        const uint32_t row = (wave * AI + uint32_t(i)) * 8u + (lane >> 3);
        const uint32_t c = (lane & 7u) ^ ((row >> 1) & 7u);
        a_off[i] = row * K * kEA + c * 16u;
    }
    auto a_issue = [&](uint32_t kt) {
        u32x4_t* stage = smem + (kt % kAStages) * kStageChunks + wave * AI * 64u;
#pragma unroll
        for (int i = 0; i < AI; ++i)
            lds_dma16(ra, stage + i * 64, a_off[i], int(kt * 128u));
    };

    // B: 16-byte int8 vectors into registers a K-step ahead, widened to bf16 into the B ring. The stage's 1024 int8
    // chunks (256 B-rows x 4 k-chunks; rows 0..127 the gate rows n0.., 128..255 the up rows n + n0..) go BI to a
    // thread: chunk q = tid + kThreads i is k-chunk q % 4 of B-row 4 (G / 2) + 2 ((q / 4) % 2) + G % 2, G = q / 8.
    // Each 8 consecutive lanes thus write two rows whose swizzles differ in parity, i.e. 8 distinct chunk columns.
    constexpr int BI = int(1024 / kThreads);
    // N * K < 2^30 (int8) or 2^29 (bf16) is checked on the host.
    const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(wv, uint32_t(w_rows * K * kEB));
    uint32_t b_src[BI], b_lo[BI], b_hi[BI];
#pragma unroll
    for (int i = 0; i < BI && I8; ++i) {
        const uint32_t q = tid + kThreads * uint32_t(i), kc = q & 3u, G = q >> 3;
        const uint32_t brow = 4u * (G >> 1) + 2u * ((q >> 2) & 1u) + (G & 1u);
        const uint32_t wrow = brow < kBN ? w_lo + brow : w_hi + (brow - kBN);
        const uint32_t sx = (brow >> 1) & 7u;
        b_src[i] = wrow * K + kc * 16u;
        b_lo[i] = brow * 128u + ((2u * kc) ^ sx) * 16u;
        b_hi[i] = brow * 128u + ((2u * kc + 1u) ^ sx) * 16u;
    }
    auto b_issue = [&](uint32_t kt, u32x4_t (&rb)[BI]) {
#pragma unroll
        for (int i = 0; i < BI; ++i)
            rb[i] = __builtin_amdgcn_raw_buffer_load_b128(rw, b_src[i], int(kt * kBK), 0);
    };
    char* const lds = reinterpret_cast<char*>(smem);
    u32x4_t rb[BI];
    // Piece p of tile kt's B write: half p % 2 of register chunk p / 2, widened and stored.
    auto b_piece = [&](uint32_t kt, const u32x4_t (&rb)[BI], int p) {
        char* B = lds + (kBBase + (kt % kBStages) * kStageChunks) * 16u;
        const int i = p >> 1, h = p & 1;
        *reinterpret_cast<u32x4_t*>(B + (h ? b_hi[i] : b_lo[i])) = widen8(rb[i][2 * h], rb[i][2 * h + 1]);
    };
    auto b_write = [&](uint32_t kt, const u32x4_t (&rb)[BI]) {
#pragma unroll
        for (int p = 0; p < 2 * BI; ++p)
            b_piece(kt, rb, p);
    };
    // bf16 weights, and int8 weights with int8 x: B goes straight into its LDS ring like A, B-row r of the tile from
    // weight row n0 + r (gate) or n + n0 + r - 128 (up), with A's chunk-to-lane assignment and swizzle.
    uint32_t bd_off[AI];
#pragma unroll
    for (int i = 0; i < AI && !I8; ++i) {
        const uint32_t row = (wave * AI + uint32_t(i)) * 8u + (lane >> 3);
        const uint32_t c = (lane & 7u) ^ ((row >> 1) & 7u);
        const uint32_t wrow = row < kBN ? w_lo + row : w_hi + (row - kBN);
        bd_off[i] = wrow * K * kEB + c * 16u;
    }
    auto b_dma = [&](uint32_t kt) {
        u32x4_t* stage = smem + kBBase + (kt % kBStages) * kStageChunks + wave * AI * 64u;
#pragma unroll
        for (int i = 0; i < AI; ++i)
            lds_dma16(rw, stage + i * 64, bd_off[i], int(kt * 128u));
    };

    // MFMA operands, 16 bytes a lane (8 bf16 or 16 int8 of k). Sub-step ks: k-half h = ks/2 and the wave's row tiles
    // (ks%2)*FA .. +FA-1, A rows wm*(256/WM) + t*16 + lane%16, B rows wn*16TN + t*16 + lane%16 (and 128 + that),
    // k-chunk 4h + lane/16. Every row a lane reads has (row >> 1) & 7 = (lane % 16 >> 1) & 7, so one offset per
    // sub-step serves all tiles; t moves it by 16 rows. (The 16 rows a quarter-wave reads at one chunk then cover the
    // 64 banks once.)
    const uint32_t rs = lane % 16u, fsx = (rs >> 1) & 7u;
    const uint32_t fa_base = (wm * (kBM / WM) + rs) * 128u, fb_base = (wn * 16u * TN + rs) * 128u;
    constexpr uint32_t kRowBytes = 16u * 128u; // one MFMA tile's rows in a stage
    uint32_t fko[4];
#pragma unroll
    for (uint32_t ks = 0; ks < 4; ++ks)
        fko[ks] = (((ks >> 1) * 4u + (lane >> 4)) ^ fsx) * 16u;
    auto frags_a = [&](uint32_t kt, uint32_t ks, bf16x8_t (&fa)[FA]) {
        const uint32_t t0 = (ks & 1u) * uint32_t(FA);
        const char* A = lds + (kt % kAStages) * kStageChunks * 16u + fa_base + fko[ks] + t0 * kRowBytes;
#pragma unroll
        for (int t = 0; t < FA; ++t)
            fa[t] = *reinterpret_cast<const bf16x8_t*>(A + t * kRowBytes);
    };
    auto frags_b = [&](uint32_t kt, uint32_t ks, bf16x8_t (&fb)[2 * TN]) {
        const char* B = lds + (kBBase + (kt % kBStages) * kStageChunks) * 16u + fb_base + fko[ks];
#pragma unroll
        for (int t = 0; t < TN; ++t) {
            fb[t] = *reinterpret_cast<const bf16x8_t*>(B + t * kRowBytes);
            fb[TN + t] = *reinterpret_cast<const bf16x8_t*>(B + kBN * 128 + t * kRowBytes);
        }
    };
    // Sub-step ks's fragments; B only at the start of a k-half (the second sub-step of a half keeps it).
    auto frags = [&](uint32_t kt, uint32_t ks, bf16x8_t (&fa)[FA], bf16x8_t (&fb)[2 * TN]) {
        frags_a(kt, ks, fa);
        if ((ks & 1u) == 0u)
            frags_b(kt, ks, fb);
    };

    Acc acc[TM][2 * TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < 2 * TN; ++b)
            acc[a][b] = Acc{};
    // One MFMA: acc[a][b] += A fragment fa * B fragment fb.
    auto mfma = [&](Acc& c, const bf16x8_t& fa, const bf16x8_t& fb) {
        if constexpr (MODE == kW8A8)
            c = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(int32x4, fa), __builtin_bit_cast(int32x4, fb),
                                                      c, 0, 0, 0);
        else
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa, fb, c, 0, 0, 0);
    };
    // Sub-step ks's MFMAs: its FA row tiles (from t0) against the 2 TN column tiles.
    auto mfmas = [&](uint32_t ks, const bf16x8_t (&fa)[FA], const bf16x8_t (&fb)[2 * TN]) {
        const int t0 = int(ks & 1u) * FA;
#pragma unroll
        for (int a = 0; a < FA; ++a)
#pragma unroll
            for (int b = 0; b < 2 * TN; ++b)
                mfma(acc[t0 + a][b], fa[a], fb[b]);
    };
    // The same MFMAs with B pieces p0 .. p0 + np - 1 of tile kt placed between them, at even spacing, so the
    // widening's VALU work issues while the matrix core is busy.
    auto mfmas_b = [&](uint32_t ks, const bf16x8_t (&fa)[FA], const bf16x8_t (&fb)[2 * TN], uint32_t kt, int p0,
                       int np) {
        constexpr int n = FA * 2 * TN;
        const int t0 = int(ks & 1u) * FA;
#pragma unroll
        for (int j = 0; j < n; ++j) {
            const int a = j / (2 * TN), b = j % (2 * TN);
            if constexpr (MODE == kW8A16)
                mfma(acc[t0 + a][b], fa[a], fb[b]);
            __builtin_amdgcn_sched_barrier(0);
            if (j % (n / np) == 0 && j / (n / np) < np) {
                b_piece(kt, rb, p0 + j / (n / np));
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };

    // Prologue: tile 0's B widened into LDS and tile 0's A in LDS; tile 1's B in registers and A in flight to LDS.
    // The explicit wait is needed: the compiler may issue the B loads ahead of the LDS-bound A loads, and then the
    // waits it places for the B registers leave tile 0's A outstanding.
    a_issue(0);
    if constexpr (I8)
        b_issue(0, rb);
    else
        b_dma(0);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (I8)
        b_write(0, rb);
    if (KT > 1) {
        if constexpr (I8)
            b_issue(1, rb);
        a_issue(1);
    }
    // The epilogue's kernel arguments are read here, before the barrier: a scalar load still in flight at the loop
    // would turn every LDS wait in it into a full wait (scalar loads complete out of order).
    asm volatile("" ::"s"(scale), "s"(xscale), "s"(out), "s"(gg.gate), "s"(gg.set_of_row));
    lds_barrier();
    // Fragment double buffers: A by sub-step parity, B by k-half (a half's two sub-steps share one B set).
    bf16x8_t fa[2][FA], fb[2][2 * TN];
    frags(0, 0, fa[0], fb[0]);

    // One K-step over tile kt (four sub-steps of 16 k). Tile kt+1's B is widened from registers into LDS in four
    // pieces placed between the MFMAs of the first two sub-steps. Then the wave waits for everything it has in
    // flight (tile kt+1's A, issued a step ago) and tile kt+2's B and A loads go out. The barrier publishing tile kt+1
    // comes after the third sub-step's MFMAs, and
    // the fourth sub-step's operands are already in registers: the MFMAs keep running while tile kt+1's first
    // fragments load. LDS stages written in step kt (A stage (kt+2) % 3, B stage (kt+1) % 2) were last read before
    // step kt-1's barrier. The last step is a separate instance (kLast) so that the loop body has no branch around
    // the barrier: at such a join the compiler's LDS wait would also cover tile kt+1's fragment reads.
    // B sets of sub-steps 0..3: one a k-half (0, 0, 1, 1).
    constexpr int B1 = 0, B2 = 1, B3 = 1;
    auto kstep = [&](uint32_t kt, auto last) {
        constexpr bool kLast = decltype(last)::value;
        if constexpr (!I8 && !kLast)
            b_dma(kt + 1); // into B stage (kt+1) % 2, last read before step kt-1's barrier
        frags(kt, 1, fa[1], fb[B1]);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (kLast || !I8)
            mfmas(0, fa[0], fb[0]);
        else
            mfmas_b(0, fa[0], fb[0], kt + 1, 0, BI);
        frags(kt, 2, fa[0], fb[B2]);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (kLast || !I8)
            mfmas(1, fa[1], fb[B1]);
        else
            mfmas_b(1, fa[1], fb[B1], kt + 1, BI, BI);
        if constexpr (!kLast) {
            if constexpr (I8) {
                __builtin_amdgcn_s_waitcnt(waitcnt_vm(0)); // tile kt+1's A complete too
                if (kt + 2 < KT) {
                    b_issue(kt + 2, rb);
                    a_issue(kt + 2);
                }
            } else if (kt + 2 < KT) {
                a_issue(kt + 2);
            }
        }
        frags(kt, 3, fa[1], fb[B3]);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(2, fa[0], fb[B2]);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (!kLast) {
            if constexpr (!I8) {
                // Loads complete in order: all but tile kt+2's AI A loads means tile kt+1's A and B are in LDS.
                if (kt + 2 < KT)
                    __builtin_amdgcn_s_waitcnt(waitcnt_vm(AI));
                else
                    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
            }
            lds_barrier();
            frags(kt + 1, 0, fa[0], fb[0]);
        }
        __builtin_amdgcn_sched_barrier(0);
        mfmas(3, fa[1], fb[B3]);
    };
    for (uint32_t kt = 0; kt + 1 < KT; ++kt)
        kstep(kt, std::false_type{});
    kstep(KT - 1, std::true_type{});

    gemm_epilogue<WM, WN, MODE, EPI, TM, TN>(acc, smem, M, N, m0, w_lo, w_hi, scale, xscale, out, gg);
}

} // namespace mh3

namespace {

// Shared checks and launch of the three forms and three epilogues.
template <int MODE, int EPI>
int launch_gemm(const MH3GemmArgs* a, const void* x, const void* w, const float* scale, const float* xscale,
                uint16_t* out, const mh3::GemmGate& gg, mh3_stream_t stream)
{
    using namespace mh3;
    constexpr uint32_t kEA = MODE == kW8A8 ? 1u : 2u, kEB = MODE == kBf16 ? 2u : 1u, kKS = 128u / kEA;
    constexpr uint32_t kCols = EPI == kSwiGLU ? kBN : 2u * kBN; // output columns a tile
    if (!a)
        return MH3_ERR_POINTER;
    if (a->m == 0 || a->k == 0 || a->n == 0 || a->k % kKS != 0 || a->n % kCols != 0)
        return MH3_ERR_SHAPE;
    const uint64_t w_rows = EPI == kSwiGLU ? 2ull * a->n : a->n;
    if (a->m >= (1u << 31) || w_rows >= (uint64_t(1) << 31))
        return MH3_ERR_SHAPE;
    if (uint64_t(a->k) * kBM * kEA >= (uint64_t(1) << 31) || w_rows * a->k * kEB >= (uint64_t(1) << 31))
        return MH3_ERR_UNSUPPORTED; // 32-bit buffer offsets: a tile's A rows, and all of w
    if (!x || !w || (MODE != kBf16 && !scale) || (MODE == kW8A8 && !xscale) || !out)
        return MH3_ERR_POINTER;
    if ((EPI == kGateAdd || EPI == kGateAddF32) &&
        (!gg.gate || gg.n_sets == 0 || gg.n_sets > 256 || gg.gate_stride < a->n))
        return gg.gate ? MH3_ERR_PARAM : MH3_ERR_POINTER;
    if (!host::aligned16(x) || !host::aligned16(w) || !host::aligned16(out))
        return MH3_ERR_ALIGN;
    // The output (for the gate-add epilogue, the residual updated in place) may not overlap an operand: while one
    // tile writes its columns, the other tiles of its row band still read the same rows of x.
    const uint64_t out_bytes = uint64_t(a->m) * a->n * (EPI == kGateAddF32 ? 4u : 2u);
    if (host::overlaps(out, out_bytes, x, uint64_t(a->m) * a->k * kEA) ||
        host::overlaps(out, out_bytes, w, w_rows * a->k * kEB))
        return MH3_ERR_PARAM;
    // Nor the vectors every epilogue reads: the scales, the gate sets and the row-to-set map.
    if (host::overlaps(out, out_bytes, scale, scale ? w_rows * 4u : 0u) ||
        host::overlaps(out, out_bytes, xscale, xscale ? uint64_t(a->m) * 4u : 0u) ||
        ((EPI == kGateAdd || EPI == kGateAddF32) &&
         (host::overlaps(out, out_bytes, gg.gate, (uint64_t(gg.n_sets) - 1u) * gg.gate_stride * 4u + a->n * 4ull) ||
          host::overlaps(out, out_bytes, gg.set_of_row, gg.set_of_row ? uint64_t(a->m) : 0u))))
        return MH3_ERR_PARAM;
    constexpr int WM = kGemmWM, WN = kGemmWN;
    const void* kernel = reinterpret_cast<const void*>(&gemm_kernel<WM, WN, MODE, EPI>);
    if (const hipError_t e = host::allow_dynamic_lds(kernel, kGemmLds); e != hipSuccess)
        return host::hip_error(e);
    const uint32_t mt = (a->m + kBM - 1) / kBM, nt = a->n / kCols;
    const uint64_t tiles = uint64_t(mt) * nt;
    if (tiles >= (uint64_t(1) << 31))
        return MH3_ERR_SHAPE;
    hipLaunchKernelGGL((gemm_kernel<WM, WN, MODE, EPI>), dim3(uint32_t(tiles)), dim3(WM * WN * 64), kGemmLds,
                       static_cast<hipStream_t>(stream), x, w, scale, xscale, out, a->m, a->n, a->k, mt, nt, gg);
    return host::check_launch();
}

const mh3::GemmGate kNoGate{nullptr, nullptr, 0, 0};

// The gate-add epilogue's operands from the C-ABI's arguments.
mh3::GemmGate gate_of(const MH3GemmArgs* a, const float* gate, const uint8_t* set_of_row)
{
    const uint32_t n_sets = a && a->n_sets ? a->n_sets : 1u;
    const uint32_t stride = a && a->gate_stride ? a->gate_stride : (a ? a->n : 0u);
    return mh3::GemmGate{gate, set_of_row, stride, n_sets};
}

// The three weight forms of one epilogue, by the C-ABI's weight dtype.
template <int EPI>
int launch_by_form(const MH3GemmArgs* a, uint32_t form, const void* x, const float* x_scale, const void* w,
                   const float* w_scale, uint16_t* out, const mh3::GemmGate& gg, mh3_stream_t stream)
{
    switch (form) {
    case MH3_GEMM_W8A16:
        return launch_gemm<mh3::kW8A16, EPI>(a, x, w, w_scale, nullptr, out, gg, stream);
    case MH3_GEMM_BF16:
        return launch_gemm<mh3::kBf16, EPI>(a, x, w, nullptr, nullptr, out, gg, stream);
    case MH3_GEMM_W8A8:
        return launch_gemm<mh3::kW8A8, EPI>(a, x, w, w_scale, x_scale, out, gg, stream);
    default:
        return MH3_ERR_PARAM;
    }
}

} // namespace

extern "C" int mh3_gemm_w8a16_swiglu(const MH3GemmArgs* a, const uint16_t* x, const int8_t* w, const float* scale,
                                     uint16_t* out, mh3_stream_t stream)
{
    return launch_gemm<mh3::kW8A16, mh3::kSwiGLU>(a, x, w, scale, nullptr, out, kNoGate, stream);
}

extern "C" int mh3_gemm_bf16_swiglu(const MH3GemmArgs* a, const uint16_t* x, const uint16_t* w, uint16_t* out,
                                    mh3_stream_t stream)
{
    return launch_gemm<mh3::kBf16, mh3::kSwiGLU>(a, x, w, nullptr, nullptr, out, kNoGate, stream);
}

extern "C" int mh3_gemm_i8_swiglu(const MH3GemmArgs* a, const int8_t* x, const float* x_scale, const int8_t* w,
                                  const float* w_scale, uint16_t* out, mh3_stream_t stream)
{
    return launch_gemm<mh3::kW8A8, mh3::kSwiGLU>(a, x, w, w_scale, x_scale, out, kNoGate, stream);
}

extern "C" int mh3_gemm(const MH3GemmArgs* a, uint32_t form, const void* x, const float* x_scale, const void* w,
                        const float* w_scale, uint16_t* out, mh3_stream_t stream)
{
    return launch_by_form<mh3::kStore>(a, form, x, x_scale, w, w_scale, out, kNoGate, stream);
}

extern "C" int mh3_gemm_gate_add(const MH3GemmArgs* a, uint32_t form, const void* x, const float* x_scale,
                                 const void* w, const float* w_scale, const float* gate, const uint8_t* set_of_row,
                                 uint16_t* residual, mh3_stream_t stream)
{
    return launch_by_form<mh3::kGateAdd>(a, form, x, x_scale, w, w_scale, residual, gate_of(a, gate, set_of_row),
                                         stream);
}

extern "C" int mh3_gemm_gate_add_f32(const MH3GemmArgs* a, uint32_t form, const void* x, const float* x_scale,
                                     const void* w, const float* w_scale, const float* gate,
                                     const uint8_t* set_of_row, float* residual, mh3_stream_t stream)
{
    return launch_by_form<mh3::kGateAddF32>(a, form, x, x_scale, w, w_scale, reinterpret_cast<uint16_t*>(residual),
                                            gate_of(a, gate, set_of_row), stream);
}
