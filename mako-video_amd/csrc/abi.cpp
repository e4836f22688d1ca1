// The host-only part of the C-ABI: error strings, launch checks, device queries and H3's option parsing.
#include "mh3_common.hpp"

#include <cmath>
#include <cstring>
#include <map>
#include <mutex>
#include <string>

namespace {

thread_local std::string g_last_hip_error;

constexpr int kMaxDevices = 64;
int g_cu_count[kMaxDevices];
std::once_flag g_cu_once[kMaxDevices];

} // namespace

namespace mh3::host {

int check_launch()
{
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? MH3_OK : hip_error(e);
}

int hip_error(hipError_t e)
{
    g_last_hip_error = hipGetErrorString(e);
    return MH3_ERR_HIP;
}

int cu_count()
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return 256;
    std::call_once(g_cu_once[dev], [dev] {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        g_cu_count[dev] = n;
    });
    return g_cu_count[dev];
}

hipError_t allow_dynamic_lds(const void* kernel, size_t bytes)
{
    static std::mutex mu;
    static std::map<std::pair<int, const void*>, size_t> allowed;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess)
        dev = -1;
    std::lock_guard<std::mutex> lock(mu);
    auto it = allowed.find({dev, kernel});
    if (it != allowed.end() && it->second >= bytes)
        return hipSuccess;
    const hipError_t e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, int(bytes));
    if (e == hipSuccess)
        allowed[{dev, kernel}] = bytes;
    return e;
}

int blocks_per_cu(const void* kernel, int block, size_t lds)
{
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, block, lds) != hipSuccess || n <= 0)
        n = 1;
    return n;
}

} // namespace mh3::host

extern "C" {

int mh3_abi_version(void) { return MH3_ABI_VERSION; }

const char* mh3_strerror(int code)
{
    switch (code) {
    case MH3_OK: return "ok";
    case MH3_ERR_SHAPE: return "bad shape";
    case MH3_ERR_POINTER: return "null pointer";
    case MH3_ERR_ALIGN: return "misaligned pointer";
    case MH3_ERR_PARAM: return "parameter out of range";
    case MH3_ERR_HIP: return "HIP launch failed";
    case MH3_ERR_UNSUPPORTED: return "unsupported";
    default: return "unknown error";
    }
}

const char* mh3_last_hip_error(void) { return g_last_hip_error.c_str(); }

// H3::parse_int8's grammar (tools/mako_video.cpp:108-114, src/server/video_models.cpp:127-131): "none", "all", or a
// comma list of qkv, out, fc1, fc2. Empty items, unknown names and an empty string are refused.
int mh3_parse_int8(const char* text, uint32_t* mask)
{
    if (!text || !mask)
        return MH3_ERR_POINTER;
    const std::string s(text);
    if (s == "none") {
        *mask = 0;
        return MH3_OK;
    }
    if (s == "all") {
        *mask = MH3_INT8_ALL;
        return MH3_OK;
    }
    if (s.empty())
        return MH3_ERR_PARAM;
    uint32_t m = 0;
    size_t at = 0;
    while (true) {
        const size_t comma = s.find(',', at);
        const std::string item = s.substr(at, comma == std::string::npos ? std::string::npos : comma - at);
        if (item == "qkv")
            m |= MH3_INT8_QKV;
        else if (item == "out")
            m |= MH3_INT8_OUT;
        else if (item == "fc1")
            m |= MH3_INT8_FC1;
        else if (item == "fc2")
            m |= MH3_INT8_FC2;
        else
            return MH3_ERR_PARAM;
        if (comma == std::string::npos)
            break;
        at = comma + 1;
    }
    *mask = m;
    return MH3_OK;
}

// src/server/video_models.cpp:117-126: sparse in [0, 1], sparse_local in {0, 1, 3}.
int mh3_check_sparse(float ratio, uint32_t local)
{
    if (!(ratio >= 0.0f && ratio <= 1.0f))
        return MH3_ERR_PARAM;
    if (local != 0 && local != 1 && local != 3)
        return MH3_ERR_PARAM;
    return MH3_OK;
}

int64_t mh3_topk_k(float ratio, uint32_t cubes)
{
    if (!(ratio >= 0.0f && ratio <= 1.0f))
        return MH3_ERR_PARAM;
    // The ratio arrives as a float (the reference's Options::sparse, src/video/engine.hpp:35), so 0.1 is 0.1 + 1.5e-9:
    // a product that exceeds an integer by no more than the float's representation error of the ratio (at most
    // 2^-24 of it, times the cubes; 2^-22 cubes allows for it with margin) counts as that integer, so 0.1 of 660 cubes
    // is 66, not 67.
    const double k = std::ceil(double(ratio) * double(cubes) - std::ldexp(double(cubes), -22));
    return k < 0 ? 0 : (k > cubes ? int64_t(cubes) : int64_t(k));
}

int64_t mh3_cube_count(uint32_t grid_t, uint32_t grid_h, uint32_t grid_w)
{
    return int64_t((grid_t + 3u) / 4u) * int64_t((grid_h + 3u) / 4u) * int64_t((grid_w + 3u) / 4u);
}

} // extern "C"
