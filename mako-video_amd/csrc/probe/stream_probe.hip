// HBM streaming probe: the bandwidth a plain streaming kernel reaches on this GPU, as the ceiling against which the
// row kernels' fractions of the 8 TB/s nameplate are read. Four access mixes over 16-byte vectors (kind % 4):
//   0 (read):  read a (n vectors); nothing is written unless the XOR of all data equals a fixed value;
//   1 (copy):  c = a;                                 one read stream, one write stream;
//   2 (r2w1):  c = a + b (as 32-bit lanes);            two read streams, one write: the fused row op's and SwiGLU's
//                                                       mix;
//   3 (r2w2):  c[i] = a + b, c[n + i] = a - b;          two read streams, two write streams (c holds 2 n vectors): the
//                                                       mix of the block's own order (x += gate y, h = norm of x).
// Kinds 0-3 use global loads and stores, on a flat grid or a grid-stride loop; kinds 4-7 are the same mixes through
// buffer loads and stores (a descriptor over each whole buffer, 32-bit byte offsets, so every buffer stays below
// 4 GiB), the access form the row kernels use, on a flat grid only.
// 256 threads a workgroup; each thread moves U vectors 256 apart per step, non-temporal loads and stores; a flat grid
// (blocks = 0: one step a thread) or a grid-stride loop over `blocks` workgroups. Every access is i < n (or n + i <
// 2 n). bench.py sweeps the form, U and the grid and reports the best of each mix as the ceiling.
// This library is a measurement tool beside libmako_h3.so; it has no counterpart in the reference.
//
//   int mh3_probe_stream(int kind, const void* a, const void* b, void* c, uint64_t n, int unroll, uint32_t blocks,
//                        void* stream);   unroll 2, 4 or 8
//   returns 0, -1 for a bad kind, unroll or null pointer, -2 for misaligned pointers, -3 for a launch failure.
//   int mh3_probe_device(int* cus, int* max_clock_khz);  the current device's CU count and peak engine clock, from
//   which the MFMA peak is CUs x clock x flops a clock a CU.
//
// Two more probes with the shapes of the hot path's own kernels:
//   int mh3_probe_rows(const void* a, const void* b, void* c, uint32_t rows, uint32_t nvec, uint32_t lds_bytes,
//                      void* stream);
//     the fused row op's access pattern with no arithmetic: one row of nvec 16-byte vectors a wave (vector lane +
//     64 j of the row, j < 10), all of a's row loaded, then all of b's, then c = a + b stored; 8-wave workgroups of 8
//     consecutive rows, `lds_bytes` of dynamic LDS a workgroup (which sets how many share a CU), buffer loads and
//     stores with the non-temporal hint. nvec <= 640.
//   int mh3_probe_mfma(int kind, uint32_t blocks, uint32_t iters, float* out, uint64_t* clocks, void* stream);
//     a register-only loop of matrix instructions, kind 0 v_mfma_f32_16x16x32_bf16, 1 v_mfma_i32_16x16x64_i8 (the
//     GEMMs' forms), 2 v_mfma_f32_32x32x16_bf16, 3 v_mfma_i32_32x32x32_i8: 8 waves a workgroup, each wave `iters` (a
//     multiple of 8; rounded up) rounds of 16 (16 x 16) or 8 (32 x 32) independent accumulators, the operands cycling
//     through 8
//     register fragments of random bits (so the matrix core's inputs change from one instruction to the next, as in
//     a GEMM). out gets one value a thread (keeps the results live); clocks gets, for each workgroup, the shader
//     clock counter's and the 100 MHz real-time counter's advance over its loop (s_memtime, s_memrealtime), from
//     which the clock the loop ran at follows.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t kThreads = 256;
enum Mix { kRead = 0, kCopy = 1, kR2W1 = 2, kR2W2 = 3 };

template <int MIX, int U>
__global__ __launch_bounds__(kThreads) void stream_kernel(const u32x4* __restrict__ a, const u32x4* __restrict__ b,
                                                          u32x4* __restrict__ c, uint64_t n)
{
    const uint64_t stride = uint64_t(gridDim.x) * kThreads * U;
    uint32_t acc = 0;
    for (uint64_t base = uint64_t(blockIdx.x) * kThreads * U + threadIdx.x; base < n; base += stride) {
        u32x4 va[U], vb[U];
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const uint64_t i = base + uint64_t(j) * kThreads;
            va[j] = i < n ? __builtin_nontemporal_load(a + i) : u32x4{0u, 0u, 0u, 0u};
            if constexpr (MIX >= kR2W1)
                vb[j] = i < n ? __builtin_nontemporal_load(b + i) : u32x4{0u, 0u, 0u, 0u};
        }
        if constexpr (MIX == kRead) {
#pragma unroll
            for (int j = 0; j < U; ++j)
                acc ^= va[j][0] ^ va[j][1] ^ va[j][2] ^ va[j][3];
        } else {
#pragma unroll
            for (int j = 0; j < U; ++j) {
                const uint64_t i = base + uint64_t(j) * kThreads;
                if (i < n) {
                    __builtin_nontemporal_store(MIX >= kR2W1 ? va[j] + vb[j] : va[j], c + i);
                    if constexpr (MIX == kR2W2)
                        __builtin_nontemporal_store(va[j] - vb[j], c + n + i);
                }
            }
        }
    }
    if (MIX == kRead && acc == 0x9E3779B9u)
        c[0] = u32x4{acc, 0u, 0u, 0u};
}

constexpr int kRsrcFlags = 0x00020000; // raw buffer, 32-bit byte offsets; out-of-range reads return 0
constexpr int kNonTemporal = 2;

// The buffer-op form, flat grid: workgroup g's thread t takes vectors g * 256 U + t + 256 j, j < U.
template <int MIX, int U>
__global__ __launch_bounds__(kThreads) void stream_buffer_kernel(const u32x4* a, const u32x4* b, u32x4* c, uint32_t n)
{
    const uint32_t bytes = n * 16u;
    const auto ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<u32x4*>(a), 0, int(bytes), kRsrcFlags);
    const auto rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<u32x4*>(b ? b : a), 0, int(bytes), kRsrcFlags);
    const auto rc = __builtin_amdgcn_make_buffer_rsrc(c, 0, int(bytes), kRsrcFlags);
    const auto rd = __builtin_amdgcn_make_buffer_rsrc(c + (MIX == kR2W2 ? n : 0u), 0, int(bytes), kRsrcFlags);
    const uint32_t base = (blockIdx.x * kThreads * U + threadIdx.x) * 16u;
    u32x4 va[U], vb[U];
#pragma unroll
    for (int j = 0; j < U; ++j) {
        va[j] = __builtin_amdgcn_raw_buffer_load_b128(ra, base + uint32_t(j) * kThreads * 16u, 0, kNonTemporal);
        if constexpr (MIX >= kR2W1)
            vb[j] = __builtin_amdgcn_raw_buffer_load_b128(rb, base + uint32_t(j) * kThreads * 16u, 0, kNonTemporal);
    }
    if constexpr (MIX == kRead) {
        uint32_t acc = 0;
#pragma unroll
        for (int j = 0; j < U; ++j)
            acc ^= va[j][0] ^ va[j][1] ^ va[j][2] ^ va[j][3];
        if (acc == 0x9E3779B9u)
            __builtin_amdgcn_raw_buffer_store_b128(u32x4{acc, 0u, 0u, 0u}, rc, 0, 0, 0);
    } else {
#pragma unroll
        for (int j = 0; j < U; ++j) {
            __builtin_amdgcn_raw_buffer_store_b128(MIX >= kR2W1 ? va[j] + vb[j] : va[j], rc,
                                                   base + uint32_t(j) * kThreads * 16u, 0, kNonTemporal);
            if constexpr (MIX == kR2W2)
                __builtin_amdgcn_raw_buffer_store_b128(va[j] - vb[j], rd, base + uint32_t(j) * kThreads * 16u, 0,
                                                       kNonTemporal);
        }
    }
}

template <int MIX>
void launch(int unroll, dim3 grid, hipStream_t s, const u32x4* a, const u32x4* b, u32x4* c, uint64_t n)
{
    if (unroll == 2)
        hipLaunchKernelGGL((stream_kernel<MIX, 2>), grid, dim3(kThreads), 0, s, a, b, c, n);
    else if (unroll == 4)
        hipLaunchKernelGGL((stream_kernel<MIX, 4>), grid, dim3(kThreads), 0, s, a, b, c, n);
    else
        hipLaunchKernelGGL((stream_kernel<MIX, 8>), grid, dim3(kThreads), 0, s, a, b, c, n);
}

template <int MIX>
void launch_buffer(int unroll, hipStream_t s, const u32x4* a, const u32x4* b, u32x4* c, uint32_t n)
{
    const dim3 grid{(n + kThreads * unroll - 1) / (kThreads * unroll)};
    if (unroll == 2)
        hipLaunchKernelGGL((stream_buffer_kernel<MIX, 2>), grid, dim3(kThreads), 0, s, a, b, c, n);
    else if (unroll == 4)
        hipLaunchKernelGGL((stream_buffer_kernel<MIX, 4>), grid, dim3(kThreads), 0, s, a, b, c, n);
    else
        hipLaunchKernelGGL((stream_buffer_kernel<MIX, 8>), grid, dim3(kThreads), 0, s, a, b, c, n);
}

// ---- the fused row op's shape ----------------------------------------------------------------------------------------
constexpr uint32_t kRowVecs = 10; // 16-byte vectors a lane: a 5120-wide bf16 row

__global__ __launch_bounds__(512) void rows_probe_kernel(const u32x4* a, const u32x4* b, u32x4* c, uint32_t rows,
                                                         uint32_t nvec)
{
    const uint32_t lane = threadIdx.x & 63u, row = blockIdx.x * 8u + (threadIdx.x >> 6);
    const uint32_t bytes = row < rows ? nvec * 16u : 0u, rr = row < rows ? row : 0u;
    const auto ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<u32x4*>(a + uint64_t(rr) * nvec), 0, int(bytes),
                                                      kRsrcFlags);
    const auto rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<u32x4*>(b + uint64_t(rr) * nvec), 0, int(bytes),
                                                      kRsrcFlags);
    const auto rc = __builtin_amdgcn_make_buffer_rsrc(c + uint64_t(rr) * nvec, 0, int(bytes), kRsrcFlags);
    u32x4 va[kRowVecs], vb[kRowVecs];
#pragma unroll
    for (uint32_t j = 0; j < kRowVecs; ++j)
        va[j] = __builtin_amdgcn_raw_buffer_load_b128(ra, (lane + 64u * j) * 16u, 0, kNonTemporal);
#pragma unroll
    for (uint32_t j = 0; j < kRowVecs; ++j)
        vb[j] = __builtin_amdgcn_raw_buffer_load_b128(rb, (lane + 64u * j) * 16u, 0, kNonTemporal);
#pragma unroll
    for (uint32_t j = 0; j < kRowVecs; ++j)
        __builtin_amdgcn_raw_buffer_store_b128(va[j] + vb[j], rc, (lane + 64u * j) * 16u, 0, kNonTemporal);
}

// ---- the matrix cores' sustained rate ------------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef int intx4 __attribute__((ext_vector_type(4)));
typedef int intx16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ uint32_t mix32(uint32_t x)
{
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    return x ^ (x >> 16);
}

typedef float floatx4 __attribute__((ext_vector_type(4)));

// KIND 0: v_mfma_f32_16x16x32_bf16, 1: v_mfma_i32_16x16x64_i8 (the GEMMs' forms), 2: v_mfma_f32_32x32x16_bf16,
// 3: v_mfma_i32_32x32x32_i8. 16 independent 16 x 16 accumulators a wave, or 8 of 32 x 32 (64 or 128 registers).
template <int KIND>
__global__ __launch_bounds__(512) void mfma_probe_kernel(uint32_t iters, float* out, uint64_t* clocks)
{
    constexpr bool kI8 = KIND == 1 || KIND == 3, k32 = KIND >= 2;
    constexpr int kFrag = 8, kAcc = k32 ? 8 : 16;
    // Operand fragments of random bits; bf16 ones with the exponent held to 2^-15 .. 2^0 so no sum overflows.
    intx4 fa[kFrag], fb[kFrag];
    const uint32_t seed = (blockIdx.x * 512u + threadIdx.x) * 64u;
#pragma unroll
    for (int f = 0; f < kFrag; ++f)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            uint32_t ra = mix32(seed + f * 8u + e), rb = mix32(seed + f * 8u + 4u + e);
            if (!kI8) {
                ra = (ra & 0x87ff87ffu) | 0x38003800u; // sign, 4 low exponent bits and 7 mantissa bits random
                rb = (rb & 0x87ff87ffu) | 0x38003800u;
            }
            fa[f][e] = int(ra);
            fb[f][e] = int(rb);
        }
    using Acc = typename std::conditional<
        k32, typename std::conditional<kI8, intx16, floatx16>::type,
        typename std::conditional<kI8, intx4, floatx4>::type>::type;
    Acc acc[kAcc];
#pragma unroll
    for (int i = 0; i < kAcc; ++i)
        acc[i] = Acc{};
    __syncthreads();
    const uint64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    // Rounds of 8 (iters is taken in multiples of 8): the fragment of each instruction is then known at compile time.
    for (uint32_t it = 0; it < iters; it += 8u) {
#pragma unroll
        for (int u = 0; u < 8; ++u)
#pragma unroll
            for (int i = 0; i < kAcc; ++i) {
                const int f = (i + u) & (kFrag - 1), g = (i * 3 + u) & (kFrag - 1);
                if constexpr (KIND == 0)
                    acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8, fa[f]), __builtin_bit_cast(bf16x8, fb[g]), acc[i], 0, 0, 0);
                else if constexpr (KIND == 1)
                    acc[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[f], fb[g], acc[i], 0, 0, 0);
                else if constexpr (KIND == 2)
                    acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        __builtin_bit_cast(bf16x8, fa[f]), __builtin_bit_cast(bf16x8, fb[g]), acc[i], 0, 0, 0);
                else
                    acc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[f], fb[g], acc[i], 0, 0, 0);
            }
    }
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < kAcc; ++i)
#pragma unroll
        for (int e = 0; e < (k32 ? 16 : 4); ++e)
            sum += float(acc[i][e]);
    const uint64_t t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    out[blockIdx.x * 512u + threadIdx.x] = sum;
    if (threadIdx.x == 0) {
        clocks[2u * blockIdx.x] = t1 - t0;
        clocks[2u * blockIdx.x + 1u] = r1 - r0;
    }
}

} // namespace

extern "C" int mh3_probe_rows(const void* a, const void* b, void* c, uint32_t rows, uint32_t nvec, uint32_t lds_bytes,
                              void* stream)
{
    if (!a || !b || !c || nvec == 0 || nvec > 64u * kRowVecs || lds_bytes > 160u * 1024u)
        return -1;
    if ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) | reinterpret_cast<uintptr_t>(c)) & 15u)
        return -2;
    if (rows == 0)
        return 0;
    const auto k = reinterpret_cast<const void*>(&rows_probe_kernel);
    if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, int(lds_bytes)) != hipSuccess)
        return -3;
    hipLaunchKernelGGL(rows_probe_kernel, dim3((rows + 7u) / 8u), dim3(512), lds_bytes,
                       static_cast<hipStream_t>(stream), static_cast<const u32x4*>(a), static_cast<const u32x4*>(b),
                       static_cast<u32x4*>(c), rows, nvec);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

extern "C" int mh3_probe_mfma(int kind, uint32_t blocks, uint32_t iters, float* out, uint64_t* clocks, void* stream)
{
    if (kind < 0 || kind > 3 || blocks == 0 || !out || !clocks)
        return -1;
    if ((reinterpret_cast<uintptr_t>(clocks) & 7u) != 0)
        return -2;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (kind == 0)
        hipLaunchKernelGGL(mfma_probe_kernel<0>, dim3(blocks), dim3(512), 0, s, iters, out, clocks);
    else if (kind == 1)
        hipLaunchKernelGGL(mfma_probe_kernel<1>, dim3(blocks), dim3(512), 0, s, iters, out, clocks);
    else if (kind == 2)
        hipLaunchKernelGGL(mfma_probe_kernel<2>, dim3(blocks), dim3(512), 0, s, iters, out, clocks);
    else
        hipLaunchKernelGGL(mfma_probe_kernel<3>, dim3(blocks), dim3(512), 0, s, iters, out, clocks);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

extern "C" int mh3_probe_stream(int kind, const void* a, const void* b, void* c, uint64_t n, int unroll,
                                uint32_t blocks, void* stream)
{
    const int mix = kind % 4;
    const bool buffer = kind >= 4;
    if (kind < 0 || kind > 7 || !a || !c || (mix >= kR2W1 && !b) || (unroll != 2 && unroll != 4 && unroll != 8))
        return -1;
    if ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) | reinterpret_cast<uintptr_t>(c)) & 15u)
        return -2;
    if (n == 0)
        return 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const auto* pa = static_cast<const u32x4*>(a);
    const auto* pb = static_cast<const u32x4*>(b);
    auto* pc = static_cast<u32x4*>(c);
    if (buffer) {
        // Buffer offsets are 32-bit bytes: each buffer's vectors, rounded up to the grid, stay below 2^32 bytes.
        if (blocks != 0 || n >= (uint64_t(1) << 28) - uint64_t(kThreads) * unroll)
            return -1;
        if (mix == kRead)
            launch_buffer<kRead>(unroll, s, pa, pb, pc, uint32_t(n));
        else if (mix == kCopy)
            launch_buffer<kCopy>(unroll, s, pa, pb, pc, uint32_t(n));
        else if (mix == kR2W1)
            launch_buffer<kR2W1>(unroll, s, pa, pb, pc, uint32_t(n));
        else
            launch_buffer<kR2W2>(unroll, s, pa, pb, pc, uint32_t(n));
        return hipGetLastError() == hipSuccess ? 0 : -3;
    }
    const uint64_t flat = (n + kThreads * unroll - 1) / (kThreads * unroll);
    const uint64_t grid_blocks = blocks ? (blocks < flat ? blocks : flat) : flat;
    if (grid_blocks >= (1ull << 31))
        return -1;
    const dim3 grid{uint32_t(grid_blocks)};
    if (mix == kRead)
        launch<kRead>(unroll, grid, s, pa, pb, pc, n);
    else if (mix == kCopy)
        launch<kCopy>(unroll, grid, s, pa, pb, pc, n);
    else if (mix == kR2W1)
        launch<kR2W1>(unroll, grid, s, pa, pb, pc, n);
    else
        launch<kR2W2>(unroll, grid, s, pa, pb, pc, n);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

extern "C" int mh3_probe_device(int* cus, int* max_clock_khz)
{
    if (!cus || !max_clock_khz)
        return -1;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipDeviceGetAttribute(max_clock_khz, hipDeviceAttributeClockRate, dev) != hipSuccess)
        return -3;
    return 0;
}
