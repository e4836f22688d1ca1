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
#include <hip/hip_runtime.h>

#include <cstdint>

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

} // namespace

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
