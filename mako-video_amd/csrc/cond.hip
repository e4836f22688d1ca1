// Time conditioning of the H3 blocks: what turns each distinct noise level of a step into the modulation vectors that
// rms_mod_rows and gate_add_rows read.
//   time_embed: the sinusoidal embedding of t (freq_dim values, the cos half first), the F32 time MLP
//               (freq_dim -> hidden, silu, hidden -> out_dim), and silu of its output rounded to bf16, the input of the
//               AdaLN projections;
//   adaln_mod:  a block's AdaLN projection (bf16 weights [n][k], float accumulation), which writes the
//               [levels][3][6][D] modulation table the row kernels index by (level, tag);
//   curve_mods: the pruned checkpoints' path: a curve c(t) tabulated at `points` values of t in [0, 1], linearly
//               interpolated, through float projections [n][width] with no silu.
// Reference: docs/architecture.md:49-58 (the step's conditioning), tools/check_pruned_curve.py:57-73 (the embedding,
// the MLP, the projection and the curve, written out in torch), tests/h3_ref_test.cpp:226-241 (the time embedding
// compared at 1e-4, block 0's modulation at 5e-3, the projection's rows in [U][3][6][D] order).
//
// The AdaLN projections are the heavy part: at H3's shapes a block's weight is 96,768 x 2688 bf16 (520 MB), read once a
// step for one to three levels, so the projection is a matrix-vector stream bound by HBM. Each wave takes four weight
// rows at a time, every lane 16-byte pieces of each row at the same positions, so a lane's share of the bf16 input
// vectors is loaded once and kept in registers; v_dot2_f32_bf16 multiplies a pair of weights by a pair of inputs and
// accumulates in float, so no weight is widened.
#include "mh3_common.hpp"

#include <cmath>
#include <mutex>

namespace mh3 {

constexpr int kLevelGroup = 4;      // levels a pass of the MLP or the projection handles (H3 has one to three)
constexpr int kMaxLevels = 64;
constexpr int kFreqChunks = 4;      // float4 pieces of the embedding a lane holds: freq_dim <= 4 * 64 * 4
constexpr uint32_t kMaxFreqDim = 1024;
constexpr uint32_t kMaxHidden = 8192;
constexpr int kAdalnMaxChunks = 8;  // 16-byte pieces a lane holds of a row: k <= 8 * 64 * 8
// Weight rows a wave takes at a time: four, or two where a lane holds more than six pieces of a row (k > 3072), so
// that the loaded pieces and the input vectors stay within the registers of two waves a SIMD.
template <int NI>
constexpr int adaln_rows() { return NI <= 6 ? 4 : 2; }

// ---- the time MLP --------------------------------------------------------------------------------------------------

struct TimeParams {
    const float* t;
    const float* w_in;
    const float* b_in;
    const float* w_out;
    const float* b_out;
    float* hid;   // workspace: silu of the first layer, [levels][hidden]
    float* temb;  // [levels][out_dim]
    uint16_t* cond; // [levels][out_dim] bf16, or null
    uint32_t levels, freq_dim, hidden, out_dim;
    double log_period;
};

__device__ __forceinline__ float silu(float v) { return v / (1.0f + __expf(-v)); }

// Layer 1: hid[u][r] = silu(w_in[r] . emb(t[u]) + b_in[r]). A wave per weight row (freq_dim floats, a lane's float4
// pieces at c = lane + 64 i). The block's threads compute the embedding of its levels once, in double, one value a
// thread, into LDS (each wave computing all of its lanes' values itself took 16 times the double-precision
// transcendentals and most of the kernel's time); each lane then holds its pieces in registers.
__global__ __launch_bounds__(256) void time_mlp_in_kernel(TimeParams p)
{
    __shared__ __attribute__((aligned(16))) float emb_s[kLevelGroup][kMaxFreqDim];
    const int lane = threadIdx.x & 63;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t u0 = blockIdx.y * kLevelGroup;
    const int nu = min(kLevelGroup, int(p.levels - u0));
    const uint32_t half = p.freq_dim / 2, nchunk = p.freq_dim / 4;
    for (uint32_t v = threadIdx.x; v < p.freq_dim; v += blockDim.x) {
        const uint32_t f = v < half ? v : v - half;
        const double freq = exp(-p.log_period * double(f) / double(half));
        for (int u = 0; u < nu; ++u) {
            const double arg = double(p.t[u0 + u]) * freq;
            emb_s[u][v] = float(v < half ? cos(arg) : sin(arg));
        }
    }
    __syncthreads();
    float emb[kFreqChunks][kLevelGroup][4];
#pragma unroll
    for (int i = 0; i < kFreqChunks; ++i) {
        const uint32_t c = lane + 64u * i;
#pragma unroll
        for (int u = 0; u < kLevelGroup; ++u) {
            const float4 e = c < nchunk && u < nu ? *reinterpret_cast<const float4*>(&emb_s[u][4u * c])
                                                  : float4{0.0f, 0.0f, 0.0f, 0.0f};
            emb[i][u][0] = e.x, emb[i][u][1] = e.y, emb[i][u][2] = e.z, emb[i][u][3] = e.w;
        }
    }
    for (uint32_t r = blockIdx.x * 4u + wave; r < p.hidden; r += gridDim.x * 4u) {
        float acc[kLevelGroup] = {};
        const float4* row = reinterpret_cast<const float4*>(p.w_in + uint64_t(r) * p.freq_dim);
#pragma unroll
        for (int i = 0; i < kFreqChunks; ++i) {
            const uint32_t c = lane + 64u * i;
            if (c < nchunk) {
                const float4 w = row[c];
#pragma unroll
                for (int u = 0; u < kLevelGroup; ++u)
                    acc[u] += w.x * emb[i][u][0] + w.y * emb[i][u][1] + w.z * emb[i][u][2] + w.w * emb[i][u][3];
            }
        }
#pragma unroll
        for (int u = 0; u < kLevelGroup; ++u) {
            const float s = wave_sum(acc[u]) + (p.b_in ? p.b_in[r] : 0.0f);
            if (lane == 0 && u < nu)
                p.hid[uint64_t(u0 + u) * p.hidden + r] = silu(s);
        }
    }
}

// Layer 2: temb[u][j] = w_out[j] . hid[u] + b_out[j], and cond[u][j] = bf16(silu(temb[u][j])). One 16-wave block a
// CU stages its levels' hidden vectors in LDS once; a wave per weight row (hidden floats, float4 pieces
// c = lane + 64 i), rows dealt round-robin over the blocks so every CU streams the same share of w_out.
constexpr uint32_t kOutWaves = 16;
__global__ __launch_bounds__(kOutWaves * 64) void time_mlp_out_kernel(TimeParams p)
{
    extern __shared__ float4 hs[]; // [nu][hidden / 4]
    const int lane = threadIdx.x & 63;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t u0 = blockIdx.y * kLevelGroup;
    const int nu = min(kLevelGroup, int(p.levels - u0));
    const uint32_t hc = p.hidden / 4;
    const float4* src = reinterpret_cast<const float4*>(p.hid + uint64_t(u0) * p.hidden);
    for (uint32_t i = threadIdx.x; i < uint32_t(nu) * hc; i += blockDim.x)
        hs[i] = src[i];
    __syncthreads();
    for (uint32_t j = blockIdx.x + wave * gridDim.x; j < p.out_dim; j += gridDim.x * kOutWaves) {
        float acc[kLevelGroup] = {};
        const float4* row = reinterpret_cast<const float4*>(p.w_out + uint64_t(j) * p.hidden);
#pragma unroll 4
        for (uint32_t c = lane; c < hc; c += 64u) {
            const float4 w = row[c];
#pragma unroll
            for (int u = 0; u < kLevelGroup; ++u) {
                if (u < nu) {
                    const float4 h = hs[u * hc + c];
                    acc[u] += w.x * h.x + w.y * h.y + w.z * h.z + w.w * h.w;
                }
            }
        }
#pragma unroll
        for (int u = 0; u < kLevelGroup; ++u) {
            const float s = wave_sum(acc[u]) + (p.b_out ? p.b_out[j] : 0.0f);
            if (lane == 0 && u < nu) {
                const uint64_t o = uint64_t(u0 + u) * p.out_dim + j;
                p.temb[o] = s;
                if (p.cond)
                    p.cond[o] = uint16_t(pack_bf16(silu(s), 0.0f) & 0xffffu);
            }
        }
    }
}

// ---- the AdaLN projection ------------------------------------------------------------------------------------------

struct AdalnParams {
    const uint16_t* cond; // bf16 [levels][k]
    const uint16_t* w;    // bf16 [n][k]
    const float* bias;    // [n] or null
    float* mod;           // [levels][n]
    uint32_t levels, n, k;
};

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc)
{
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), acc,
                                           false);
}

// Sum over the wave, the result in every lane: DPP sums of the 16-lane rows, then the four row totals.
__device__ __forceinline__ float lane_value(float v, int lane)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

__device__ __forceinline__ float wave_sum_rows(float v)
{
    v = row16_sum(v);
    return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}

// mod[u][r] = w[r] . cond[u] + bias[r]. A lane holds the 16-byte pieces c = lane + 64 i (i < NI) of every row it
// reads and of the levels' input vectors; a wave takes adaln_rows<NI>() consecutive rows at a time, their pieces all loaded
// before any arithmetic, through a buffer descriptor that covers just those rows, so pieces past a row's end or past
// the last row read zeros.
template <int NI>
__global__ __launch_bounds__(256) void adaln_mod_kernel(AdalnParams p)
{
    constexpr int kAdalnRows = adaln_rows<NI>();
    const int lane = threadIdx.x & 63;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t u0 = blockIdx.y * kLevelGroup;
    const int nu = min(kLevelGroup, int(p.levels - u0));
    const uint32_t kc = p.k / 8;
    const uint32_t row_bytes = p.k * 2u;
    uint4 cv[NI][kLevelGroup];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const uint32_t c = lane + 64u * i;
#pragma unroll
        for (int u = 0; u < kLevelGroup; ++u)
            cv[i][u] = (c < kc && u < nu)
                           ? *reinterpret_cast<const uint4*>(p.cond + uint64_t(u0 + u) * p.k + 8u * c)
                           : uint4{0u, 0u, 0u, 0u};
    }
    const uint32_t groups = (p.n + kAdalnRows - 1) / kAdalnRows;
    for (uint32_t g = blockIdx.x * 4u + wave; g < groups; g += gridDim.x * 4u) {
        const uint32_t r0 = g * kAdalnRows;
        const uint32_t nr = min(uint32_t(kAdalnRows), p.n - r0);
        const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(p.w + uint64_t(r0) * p.k, nr * row_bytes);
        uint4 wv[kAdalnRows][NI];
#pragma unroll
        for (int r = 0; r < kAdalnRows; ++r) {
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const uint32_t c = lane + 64u * i;
                const uint32_t off = c < kc ? r * row_bytes + 16u * c : 0x80000000u;
                const u32x4_t v = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0,
                                                                                                    kNonTemporal));
                wv[r][i] = uint4{v[0], v[1], v[2], v[3]};
            }
        }
        float mine = 0.0f;
#pragma unroll
        for (int r = 0; r < kAdalnRows; ++r) {
#pragma unroll
            for (int u = 0; u < kLevelGroup; ++u) {
                if (u >= nu)
                    continue;
                float acc = 0.0f;
#pragma unroll
                for (int i = 0; i < NI; ++i) {
                    acc = dot2_bf16(wv[r][i].x, cv[i][u].x, acc);
                    acc = dot2_bf16(wv[r][i].y, cv[i][u].y, acc);
                    acc = dot2_bf16(wv[r][i].z, cv[i][u].z, acc);
                    acc = dot2_bf16(wv[r][i].w, cv[i][u].w, acc);
                }
                const float s = wave_sum_rows(acc);
                if (lane == r * kLevelGroup + u)
                    mine = s;
            }
        }
        const int r = lane / kLevelGroup, u = lane % kLevelGroup;
        if (lane < kAdalnRows * kLevelGroup && uint32_t(r) < nr && u < nu)
            p.mod[uint64_t(u0 + u) * p.n + r0 + r] = mine + (p.bias ? p.bias[r0 + r] : 0.0f);
    }
}

// ---- the pruned checkpoints' curve ---------------------------------------------------------------------------------

struct CurveParams {
    const float* t;
    const float* table; // [points][width]
    const float* w;     // [n][width]
    const float* bias;  // [n] or null
    float* mod;         // [levels][n]
    uint32_t levels, n, points, width;
};

constexpr uint32_t kMaxCurveWidth = 32;

// A thread per output row r: for each level, c = the table interpolated at t (points - 1) (clamped to the table), in
// float as (1 - f) table[i0] + f table[i0 + 1]; mod[u][r] = w[r] . c + bias[r].
__global__ __launch_bounds__(256) void curve_mods_kernel(CurveParams p)
{
    const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= p.n)
        return;
    float w[kMaxCurveWidth];
    for (uint32_t j = 0; j < p.width; ++j)
        w[j] = p.w[uint64_t(r) * p.width + j];
    const float b = p.bias ? p.bias[r] : 0.0f;
    const float last = float(p.points - 1);
    for (uint32_t u = 0; u < p.levels; ++u) {
        const float pos = fminf(fmaxf(p.t[u] * last, 0.0f), last);
        const uint32_t i0 = min(uint32_t(pos), p.points - 2);
        const float f = pos - float(i0);
        const float* a = p.table + uint64_t(i0) * p.width;
        float acc = 0.0f;
        for (uint32_t j = 0; j < p.width; ++j)
            acc += w[j] * ((1.0f - f) * a[j] + f * a[p.width + j]);
        p.mod[uint64_t(u) * p.n + r] = acc + b;
    }
}

namespace {

int check_time_args(const MH3TimeArgs* a)
{
    if (!a)
        return MH3_ERR_POINTER;
    if (a->levels == 0 || a->levels > kMaxLevels || a->freq_dim == 0 || a->freq_dim % 8 != 0 ||
        a->freq_dim > kMaxFreqDim || a->hidden == 0 || a->hidden % 4 != 0 || a->hidden > kMaxHidden ||
        a->out_dim == 0)
        return MH3_ERR_SHAPE;
    if (!(a->max_period > 1.0f) || !std::isfinite(a->max_period))
        return MH3_ERR_PARAM;
    return MH3_OK;
}

uint64_t time_workspace(const MH3TimeArgs* a) { return (uint64_t(a->levels) * a->hidden * 4u + 255u) & ~uint64_t(255); }

template <int NI>
void launch_adaln(const AdalnParams& p, hipStream_t st)
{
    const uint32_t groups = (p.n + adaln_rows<NI>() - 1) / adaln_rows<NI>();
    const uint32_t blocks = min((groups + 3u) / 4u, uint32_t(host::cu_count()) * 8u);
    hipLaunchKernelGGL(adaln_mod_kernel<NI>, dim3(blocks, (p.levels + kLevelGroup - 1) / kLevelGroup), dim3(256), 0,
                       st, p);
}

} // namespace

// Shared by the time-embedding entry points: launches the two MLP layers with `hid` as the layer-1 buffer.
int time_embed_launch(const MH3TimeArgs* args, const float* t, const float* w_in, const float* b_in, const float* w_out,
                      const float* b_out, float* hid, float* temb, uint16_t* cond, hipStream_t st)
{
    TimeParams p{t, w_in, b_in, w_out, b_out, hid, temb, cond, args->levels, args->freq_dim, args->hidden,
                 args->out_dim, std::log(double(args->max_period))};
    const uint32_t groups = (args->levels + kLevelGroup - 1) / kLevelGroup;
    const uint32_t in_blocks = min((args->hidden + 3u) / 4u, uint32_t(host::cu_count()) * 4u);
    hipLaunchKernelGGL(time_mlp_in_kernel, dim3(in_blocks, groups), dim3(256), 0, st, p);
    int rc = host::check_launch();
    if (rc != MH3_OK)
        return rc;
    const size_t lds = size_t(min(args->levels, uint32_t(kLevelGroup))) * args->hidden * 4u;
    if (lds > 64u * 1024u)
        if (const hipError_t e = host::allow_dynamic_lds(reinterpret_cast<const void*>(&time_mlp_out_kernel), lds);
            e != hipSuccess)
            return host::hip_error(e);
    const uint32_t out_blocks = min(args->out_dim, uint32_t(host::cu_count()));
    hipLaunchKernelGGL(time_mlp_out_kernel, dim3(out_blocks, groups), dim3(kOutWaves * 64u), lds, st, p);
    return host::check_launch();
}

int time_embed_check(const MH3TimeArgs* args, const float* t, const float* w_in, const float* w_out, float* temb)
{
    const int rc = check_time_args(args);
    if (rc != MH3_OK)
        return rc;
    if (!t || !w_in || !w_out || !temb)
        return MH3_ERR_POINTER;
    if (!host::aligned16(w_in) || !host::aligned16(w_out))
        return MH3_ERR_ALIGN;
    return MH3_OK;
}

// The time MLP's outputs (temb, cond, and the hidden layer's buffer) may not overlap each other or any input: a
// kernel would read what another workgroup of the same pass is writing. MH3_ERR_PARAM if they do.
int time_embed_aliasing(const MH3TimeArgs* a, const float* t, const float* w_in, const float* b_in, const float* w_out,
                        const float* b_out, const void* hid, uint64_t hid_bytes, const float* temb, const uint16_t* cond)
{
    const uint64_t lv = a->levels;
    const struct {
        const void* p;
        uint64_t n;
    } in[] = {{t, lv * 4u},
              {w_in, uint64_t(a->hidden) * a->freq_dim * 4u},
              {b_in, b_in ? uint64_t(a->hidden) * 4u : 0u},
              {w_out, uint64_t(a->out_dim) * a->hidden * 4u},
              {b_out, b_out ? uint64_t(a->out_dim) * 4u : 0u}},
      out[] = {{temb, lv * a->out_dim * 4u}, {cond, cond ? lv * a->out_dim * 2u : 0u}, {hid, hid_bytes}};
    for (size_t i = 0; i < 3; ++i) {
        for (const auto& x : in)
            if (host::overlaps(out[i].p, out[i].n, x.p, x.n))
                return MH3_ERR_PARAM;
        for (size_t j = i + 1; j < 3; ++j)
            if (host::overlaps(out[i].p, out[i].n, out[j].p, out[j].n))
                return MH3_ERR_PARAM;
    }
    return MH3_OK;
}

// ---- the variant that allocates nothing ------------------------------------------------------------------------------
// mh3_time_embed_noalloc keeps the hidden layer in this file-scope array instead of a caller's workspace: each GPU the
// library runs on holds its own copy (256 KiB) until the process ends. Its address on the current device comes from
// hipGetSymbolAddress, once per device; host code passes that address to the kernels, never the array's name (which
// in host code is only a stand-in for the symbol).
constexpr uint32_t kScratchFloats = 65536; // levels x hidden at most: e.g. 12 levels of H3's 5376
static __device__ __align__(256) float scratch[kScratchFloats];

namespace {
constexpr int kMaxScratchDevices = 64;
std::once_flag g_scratch_once[kMaxScratchDevices];
float* g_scratch_ptr[kMaxScratchDevices];
hipError_t g_scratch_rc[kMaxScratchDevices];
} // namespace

// The current device's copy of `scratch`; null if its address is not available, with the HIP error in *rc.
float* scratch_on_current_device(hipError_t* rc)
{
    int dev = 0;
    *rc = hipGetDevice(&dev);
    if (*rc != hipSuccess)
        return nullptr;
    if (dev < 0 || dev >= kMaxScratchDevices) {
        *rc = hipErrorInvalidDevice;
        return nullptr;
    }
    std::call_once(g_scratch_once[dev], [dev] {
        void* ptr = nullptr;
        g_scratch_rc[dev] = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        g_scratch_ptr[dev] = g_scratch_rc[dev] == hipSuccess ? static_cast<float*>(ptr) : nullptr;
    });
    *rc = g_scratch_rc[dev];
    return g_scratch_ptr[dev];
}

} // namespace mh3

using namespace mh3;

extern "C" {

int64_t mh3_time_embed_workspace_bytes(const MH3TimeArgs* args)
{
    const int rc = check_time_args(args);
    return rc != MH3_OK ? int64_t(rc) : int64_t(time_workspace(args));
}

int mh3_time_embed(const MH3TimeArgs* args, const float* t, const float* w_in, const float* b_in, const float* w_out,
                   const float* b_out, void* workspace, uint64_t workspace_bytes, float* temb, uint16_t* cond,
                   mh3_stream_t stream)
{
    int rc = time_embed_check(args, t, w_in, w_out, temb);
    if (rc != MH3_OK)
        return rc;
    if (!workspace)
        return MH3_ERR_POINTER;
    if (!host::aligned16(workspace))
        return MH3_ERR_ALIGN;
    if (workspace_bytes < time_workspace(args))
        return MH3_ERR_SHAPE;
    rc = time_embed_aliasing(args, t, w_in, b_in, w_out, b_out, workspace, time_workspace(args), temb, cond);
    if (rc != MH3_OK)
        return rc;
    return time_embed_launch(args, t, w_in, b_in, w_out, b_out, static_cast<float*>(workspace), temb, cond,
                             static_cast<hipStream_t>(stream));
}

int mh3_time_embed_noalloc(const MH3TimeArgs* args, const float* t, const float* w_in, const float* b_in,
                           const float* w_out, const float* b_out, float* temb, uint16_t* cond, mh3_stream_t stream)
{
    int rc = time_embed_check(args, t, w_in, w_out, temb);
    if (rc != MH3_OK)
        return rc;
    if (uint64_t(args->levels) * args->hidden > kScratchFloats)
        return MH3_ERR_UNSUPPORTED;
    rc = time_embed_aliasing(args, t, w_in, b_in, w_out, b_out, nullptr, 0, temb, cond);
    if (rc != MH3_OK)
        return rc;
    hipError_t e = hipSuccess;
    float* hid = scratch_on_current_device(&e);
    if (!hid)
        return host::hip_error(e);
    if (stream) {
        // The array's address is the current device's copy: a stream of another GPU would run the kernels there
        // against this GPU's address.
        int cur = 0;
        hipDevice_t sdev = 0;
        if ((e = hipGetDevice(&cur)) != hipSuccess ||
            (e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev)) != hipSuccess)
            return host::hip_error(e);
        if (int(sdev) != cur)
            return MH3_ERR_PARAM;
    }
    return time_embed_launch(args, t, w_in, b_in, w_out, b_out, hid, temb, cond, static_cast<hipStream_t>(stream));
}

int mh3_adaln_mod(const MH3GemmArgs* args, const uint16_t* cond, const uint16_t* w, const float* bias, float* mod,
                  mh3_stream_t stream)
{
    if (!args)
        return MH3_ERR_POINTER;
    const uint32_t levels = args->m, n = args->n, k = args->k;
    if (levels == 0 || levels > kMaxLevels || n == 0 || k == 0 || k % 8 != 0)
        return MH3_ERR_SHAPE;
    if (k > 8u * 64u * kAdalnMaxChunks)
        return MH3_ERR_UNSUPPORTED;
    if (!cond || !w || !mod)
        return MH3_ERR_POINTER;
    if (!host::aligned16(cond) || !host::aligned16(w))
        return MH3_ERR_ALIGN;
    // mod may not overlap an input: other workgroups of the launch still read them.
    const uint64_t mod_bytes = uint64_t(levels) * n * 4u;
    if (host::overlaps(mod, mod_bytes, cond, uint64_t(levels) * k * 2u) ||
        host::overlaps(mod, mod_bytes, w, uint64_t(n) * k * 2u) ||
        (bias && host::overlaps(mod, mod_bytes, bias, uint64_t(n) * 4u)))
        return MH3_ERR_PARAM;
    const AdalnParams p{cond, w, bias, mod, levels, n, k};
    hipStream_t st = static_cast<hipStream_t>(stream);
    switch ((k / 8 + 63) / 64) {
    case 1: launch_adaln<1>(p, st); break;
    case 2: launch_adaln<2>(p, st); break;
    case 3: launch_adaln<3>(p, st); break;
    case 4: launch_adaln<4>(p, st); break;
    case 5: launch_adaln<5>(p, st); break;
    case 6: launch_adaln<6>(p, st); break;
    case 7: launch_adaln<7>(p, st); break;
    default: launch_adaln<8>(p, st); break;
    }
    return host::check_launch();
}

int mh3_curve_mods(const MH3CurveArgs* args, const float* t, const float* table, const float* w, const float* bias,
                   float* mod, mh3_stream_t stream)
{
    if (!args)
        return MH3_ERR_POINTER;
    if (args->levels == 0 || args->levels > kMaxLevels || args->n == 0 || args->points < 2 || args->width == 0 ||
        args->width > kMaxCurveWidth)
        return MH3_ERR_SHAPE;
    if (!t || !table || !w || !mod)
        return MH3_ERR_POINTER;
    // mod may not overlap an input: other threads of the launch still read them.
    const uint64_t mod_bytes = uint64_t(args->levels) * args->n * 4u;
    if (host::overlaps(mod, mod_bytes, t, uint64_t(args->levels) * 4u) ||
        host::overlaps(mod, mod_bytes, table, uint64_t(args->points) * args->width * 4u) ||
        host::overlaps(mod, mod_bytes, w, uint64_t(args->n) * args->width * 4u) ||
        (bias && host::overlaps(mod, mod_bytes, bias, uint64_t(args->n) * 4u)))
        return MH3_ERR_PARAM;
    const CurveParams p{t, table, w, bias, mod, args->levels, args->n, args->points, args->width};
    hipLaunchKernelGGL(curve_mods_kernel, dim3((args->n + 255u) / 256u), dim3(256), 0,
                       static_cast<hipStream_t>(stream), p);
    return host::check_launch();
}

} // extern "C"
