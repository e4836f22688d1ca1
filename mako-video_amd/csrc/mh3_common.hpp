// Shared device and host helpers of the mako_h3 kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "mako_h3.h"

namespace mh3 {

constexpr int kWave = 64;

// ---- bf16 <-> float ------------------------------------------------------------------------------------------------
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

// Two floats to a packed bf16 pair, each rounded to nearest even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi)
{
    bf16x2_t v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

// ---- wave reductions (64 lanes) ---------------------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
        v += __shfl_xor(v, o, kWave);
    return v;
}

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
        v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// Wave-uniform minimum / maximum of a uint32 through DPP within 16-lane rows and four readlanes.
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v)
{
    v = min(v, uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0xB1, 0xF, 0xF, false)));
    v = min(v, uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0x4E, 0xF, 0xF, false)));
    v = min(v, uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0x141, 0xF, 0xF, false)));
    v = min(v, uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0x140, 0xF, 0xF, false)));
    return min(min(uint32_t(__builtin_amdgcn_readlane(int(v), 0)), uint32_t(__builtin_amdgcn_readlane(int(v), 16))),
               min(uint32_t(__builtin_amdgcn_readlane(int(v), 32)), uint32_t(__builtin_amdgcn_readlane(int(v), 48))));
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v)
{
    v = max(v, uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0xB1, 0xF, 0xF, false)));
    v = max(v, uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0x4E, 0xF, 0xF, false)));
    v = max(v, uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0x141, 0xF, 0xF, false)));
    v = max(v, uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0x140, 0xF, 0xF, false)));
    return max(max(uint32_t(__builtin_amdgcn_readlane(int(v), 0)), uint32_t(__builtin_amdgcn_readlane(int(v), 16))),
               max(uint32_t(__builtin_amdgcn_readlane(int(v), 32)), uint32_t(__builtin_amdgcn_readlane(int(v), 48))));
}

// Exclusive prefix sum over the wave's lanes (lane 0 gets 0), through DPP: row_shr 1, 2, 4, 8 give each 16-lane row
// its inclusive scan (lanes shifted in from outside the row read 0), row_bcast15 and row_bcast31 carry the totals of
// rows 0 and 0..1 into the rows above.
__device__ __forceinline__ uint32_t wave_excl_scan_u32(uint32_t v)
{
    uint32_t s = v;
    s += uint32_t(__builtin_amdgcn_update_dpp(0, int(s), 0x111, 0xF, 0xF, false));
    s += uint32_t(__builtin_amdgcn_update_dpp(0, int(s), 0x112, 0xF, 0xF, false));
    s += uint32_t(__builtin_amdgcn_update_dpp(0, int(s), 0x114, 0xF, 0xF, false));
    s += uint32_t(__builtin_amdgcn_update_dpp(0, int(s), 0x118, 0xF, 0xF, false));
    s += uint32_t(__builtin_amdgcn_update_dpp(0, int(s), 0x142, 0xA, 0xF, false));
    s += uint32_t(__builtin_amdgcn_update_dpp(0, int(s), 0x143, 0xC, 0xF, false));
    return s - v;
}

// Sum over each 16-lane row of the wave, through DPP (no LDS): every lane of a row ends with its row's total.
// quad_perm [1,0,3,2] and [2,3,0,1] sum the quads, row_half_mirror pairs the quads of each half-row and row_mirror
// the half-rows.
__device__ __forceinline__ float row16_sum(float v)
{
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, true));
    return v;
}

// Integer sum over the whole wave through DPP row sums and four readlanes; the result is wave-uniform.
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v)
{
    v += uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0xB1, 0xF, 0xF, true));
    v += uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0x4E, 0xF, 0xF, true));
    v += uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0x141, 0xF, 0xF, true));
    v += uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0x140, 0xF, 0xF, true));
    return uint32_t(__builtin_amdgcn_readlane(int(v), 0)) + uint32_t(__builtin_amdgcn_readlane(int(v), 16)) +
           uint32_t(__builtin_amdgcn_readlane(int(v), 32)) + uint32_t(__builtin_amdgcn_readlane(int(v), 48));
}

// Lanes below this one in a 64-bit ballot.
__device__ __forceinline__ uint64_t lanes_below(int lane) { return (uint64_t(1) << lane) - 1; }

// n / d for any 32-bit n by a multiply-high and shifts (Granlund & Montgomery 1994, fig. 4.1).
struct FastDiv {
    uint32_t m, s1, s2;
    __host__ static FastDiv make(uint32_t d)
    {
        uint32_t l = 0;
        while ((uint64_t(1) << l) < d)
            ++l;
        FastDiv f;
        f.m = uint32_t(((uint64_t(1) << 32) * ((uint64_t(1) << l) - d)) / d + 1);
        f.s1 = l < 1 ? l : 1;
        f.s2 = l > 1 ? l - 1 : 0;
        return f;
    }
    __device__ __forceinline__ uint32_t div(uint32_t n) const
    {
        const uint32_t t = __umulhi(n, m);
        return (t + ((n - t) >> s1)) >> s2;
    }
};

// ---- streaming memory access -----------------------------------------------------------------------------------------
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// Buffer descriptor word 3 for raw (stride 0) buffers with 32-bit byte offsets on gfx9: reads past num_records
// return zero without touching memory, writes past it are dropped.
constexpr int kRsrcFlags = 0x00020000;
constexpr int kNonTemporal = 2; // buffer op cache policy: nt

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, int(bytes), kRsrcFlags);
}

// 16-byte loads and stores with the non-temporal hint, for data read or written once.
__device__ __forceinline__ uint4 ld_stream(const uint4* p)
{
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return uint4{v[0], v[1], v[2], v[3]};
}
__device__ __forceinline__ void st_stream(uint4* p, const uint4& v)
{
    const u32x4_t t = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(t, reinterpret_cast<u32x4_t*>(p));
}

} // namespace mh3

// ---- host side ------------------------------------------------------------------------------------------------------
namespace mh3::host {

// Records the HIP error of the last launch on this thread; returns MH3_ERR_HIP if there was one.
int check_launch();
// Records `e` as this thread's last HIP error (mh3_last_hip_error) and returns MH3_ERR_HIP.
int hip_error(hipError_t e);
// The CU count of the current device (cached per device).
int cu_count();
// How many blocks of `kernel` fit on one CU with `block` threads and `lds` dynamic LDS bytes (cached by the caller).
int blocks_per_cu(const void* kernel, int block, size_t lds);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
// Whether the byte ranges [a, a + an) and [b, b + bn) share a byte.
inline bool overlaps(const void* a, uint64_t an, const void* b, uint64_t bn)
{
    const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    return an && bn && x < y + bn && y < x + an;
}
// Lets `kernel` take `bytes` of dynamic LDS on the current device (hipFuncSetAttribute, once per kernel and device).
hipError_t allow_dynamic_lds(const void* kernel, size_t bytes);

// Whether any of the outputs (pointer, bytes; null pointers skipped) overlaps an input or another output: a launch
// would read what its other workgroups are writing.
struct Span {
    const void* p;
    uint64_t n;
};
template <size_t NI, size_t NO>
bool any_overlap(const Span (&in)[NI], const Span (&out)[NO])
{
    for (size_t i = 0; i < NO; ++i) {
        for (size_t j = 0; j < NI; ++j)
            if (out[i].p && in[j].p && overlaps(out[i].p, out[i].n, in[j].p, in[j].n))
                return true;
        for (size_t j = i + 1; j < NO; ++j)
            if (out[i].p && out[j].p && overlaps(out[i].p, out[i].n, out[j].p, out[j].n))
                return true;
    }
    return false;
}

} // namespace mh3::host
