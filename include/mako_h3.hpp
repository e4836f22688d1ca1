// mako_h3.hpp — C++ host layer over the C-ABI in mako_h3.h, for C++ callers of the H3 block's hot-path kernels.
//
// The reference drives these kernels from C++ through named dispatch (mako-common's TransformerRuntime; the in-repo
// instance is src/video/audio_vae.cpp:151-177): the host validates shapes and throws std::runtime_error
// (audio_vae.cpp:231-232, src/video/engine.cpp:681-682), buffers belong to the caller (reserve()/scratch()), and
// finish(cb) waits for the queue (audio_vae.cpp:242-247). This layer keeps that shape on MI355X:
//   - one member function of Kernels per reference kernel name, with the reference's argument meaning;
//   - errors from the library (MH3_ERR_*) and from HIP become std::runtime_error naming the kernel;
//   - Kernels::finish() is hipStreamSynchronize on the Kernels' stream;
//   - DeviceBuffer<T> is caller-owned device memory; no kernel allocates;
//   - parse_int8 returns std::optional like H3::parse_int8 (tools/mako_video.cpp:110).
// Header-only; link libmako_h3.so and libamdhip64.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

#include "mako_h3.h"

namespace mako::h3 {

inline std::runtime_error error(const char* what, int rc)
{
    char msg[256];
    std::snprintf(msg, sizeof msg, "%s: %s%s%s", what, mh3_strerror(rc), rc == MH3_ERR_HIP ? ": " : "",
                  rc == MH3_ERR_HIP ? mh3_last_hip_error() : "");
    return std::runtime_error(msg);
}

inline void check(int rc, const char* what)
{
    if (rc != MH3_OK)
        throw error(what, rc);
}

inline void check_hip(hipError_t e, const char* what)
{
    if (e != hipSuccess)
        throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// Caller-owned device memory of n elements of T.
template <class T>
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t n) : n_(n)
    {
        if (n)
            check_hip(hipMalloc(reinterpret_cast<void**>(&p_), n * sizeof(T)), "hipMalloc");
    }
    explicit DeviceBuffer(const std::vector<T>& host) : DeviceBuffer(host.size()) { upload(host); }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&& o) noexcept : p_(o.p_), n_(o.n_) { o.p_ = nullptr, o.n_ = 0; }
    ~DeviceBuffer()
    {
        if (p_)
            (void)hipFree(p_);
    }
    T* get() const { return p_; }
    size_t size() const { return n_; }
    void upload(const std::vector<T>& host)
    {
        if (host.size() != n_)
            throw std::runtime_error("DeviceBuffer::upload: size mismatch");
        check_hip(hipMemcpy(p_, host.data(), n_ * sizeof(T), hipMemcpyHostToDevice), "hipMemcpy");
    }
    std::vector<T> download() const
    {
        std::vector<T> h(n_);
        check_hip(hipMemcpy(h.data(), p_, n_ * sizeof(T), hipMemcpyDeviceToHost), "hipMemcpy");
        return h;
    }

private:
    T* p_ = nullptr;
    size_t n_ = 0;
};

// The per-row modulation of a row kernel: set s(r) = set_of_row[r] (device; nullptr: set 0) picks row s of the
// [n_sets][dim] shift, scale and gate vectors; w is the norm's [dim] weight (nullptr: all 1).
struct Modulation {
    const float* w = nullptr;
    const float* shift = nullptr;
    const float* scale = nullptr;
    const float* gate = nullptr;
    const uint8_t* set_of_row = nullptr;
    uint32_t n_sets = 1;
    // Floats from one set's shift / scale / gate vector to the next set's; 0: dim. With the reference's
    // [U][3][6][D] table, shift = table + i D (i the vector's slot), and set_stride = 6 D.
    uint32_t set_stride = 0;
};

// The H3 grid of generated video rows and the sparse selector's parameters (H3::Cubes, H3::set_sparse).
struct Cubes {
    uint32_t heads = 0, t = 0, h = 0, w = 0;
    float ratio = 0.1f;
    uint32_t local = 1;
    uint32_t layout = MH3_CUBES_GRID;
    uint64_t row0 = 0, head_stride = 0, row_stride = 128;

    uint32_t count() const { return uint32_t(mh3_cube_count(t, h, w)); }
    uint32_t k() const
    {
        const int64_t k = mh3_topk_k(ratio, count());
        if (k < 0)
            throw error("set_sparse", int(k));
        return uint32_t(k);
    }
    uint32_t out_stride() const { return k() + local; }
    MH3CubeArgs args() const
    {
        check(mh3_check_sparse(ratio, local), "set_sparse");
        return MH3CubeArgs{heads, 128, t, h, w, layout, row0, head_stride ? head_stride : uint64_t(t) * h * w * 128,
                           row_stride, k(), local, out_stride(), 0};
    }
};

// The shape of a heads_partial call: qkv rows [q heads | k heads | v heads] in, head tiles out. Zero strides take
// the defaults: qkv_stride 3 heads 128, outputs [heads][rows][128].
struct Heads {
    uint32_t rows = 0, model_rows = 0, heads = 0;
    uint32_t rot = 96;
    float eps = 1e-6f;
    uint64_t qkv_stride = 0, out_head_stride = 0, out_row_stride = 0;

    MH3HeadsArgs args() const
    {
        return MH3HeadsArgs{rows,
                            model_rows ? model_rows : rows,
                            heads,
                            128,
                            rot,
                            eps,
                            qkv_stride ? qkv_stride : 3ull * heads * 128,
                            out_head_stride ? out_head_stride : uint64_t(rows) * 128,
                            out_row_stride ? out_row_stride : 128};
    }
};

inline std::optional<uint32_t> parse_int8(const std::string& text)
{
    uint32_t mask = 0;
    if (mh3_parse_int8(text.c_str(), &mask) != MH3_OK)
        return std::nullopt;
    return mask;
}

// The block's row, sparse-selector and int8 kernels on one stream, asynchronous until finish().
class Kernels {
public:
    // Refuses a library built from another version of mako_h3.h (its argument structs would not match).
    explicit Kernels(hipStream_t stream = nullptr) : s_(stream)
    {
        if (mh3_abi_version() != MH3_ABI_VERSION)
            throw std::runtime_error("libmako_h3: ABI version " + std::to_string(mh3_abi_version()) +
                                     ", the header is " + std::to_string(MH3_ABI_VERSION));
    }
    hipStream_t stream() const { return s_; }
    void finish() const { check_hip(hipStreamSynchronize(s_), "finish"); }

    // y = rmsnorm(x) * w * (1 + scale[s]) + shift[s]. flags (dtype MH3_F32): MH3_ROWS_NORM_BF16 gives the bf16 row
    // the next GEMM takes from the float residual stream.
    void rms_mod_rows(uint32_t rows, uint32_t dim, uint32_t dtype, const void* x, const Modulation& m, void* y,
                      float eps = 1e-6f, uint32_t flags = 0) const
    {
        const MH3RowsArgs a = rows_args(rows, dim, dtype, m, eps, flags);
        check(mh3_rms_mod_rows(&a, x, m.w, m.shift, m.scale, m.set_of_row, y, s_), "rms_mod_rows");
    }
    // x += gate[s] * y. flags (dtype MH3_F32): MH3_ROWS_Y_BF16 adds a GEMM's bf16 output into the float stream.
    void gate_add_rows(uint32_t rows, uint32_t dim, uint32_t dtype, void* x, const void* y, const Modulation& m,
                       uint32_t flags = 0) const
    {
        const MH3RowsArgs a = rows_args(rows, dim, dtype, m, 1.0f, flags);
        check(mh3_gate_add_rows(&a, x, y, m.gate, m.set_of_row, s_), "gate_add_rows");
    }
    // out = residual + gate[s] * rms_mod(x)
    void rms_mod_gate_add_rows(uint32_t rows, uint32_t dim, uint32_t dtype, const void* x, const void* residual,
                               const Modulation& m, void* out, float eps = 1e-6f) const
    {
        const MH3RowsArgs a = rows_args(rows, dim, dtype, m, eps);
        check(mh3_rms_mod_gate_add_rows(&a, x, residual, m.w, m.shift, m.scale, m.gate, m.set_of_row, out, s_),
              "rms_mod_gate_add_rows");
    }
    // x += gate[s] * y; h = rms_mod(x)  (the block's order: gate_add_rows then rms_mod_rows, in one pass). flags
    // (dtype MH3_F32): MH3_ROWS_NORM_BF16, alone or with MH3_ROWS_Y_BF16, for the float residual stream.
    void gate_add_rms_mod_rows(uint32_t rows, uint32_t dim, uint32_t dtype, void* x, const void* y,
                               const Modulation& m, void* h, float eps = 1e-6f, uint32_t flags = 0) const
    {
        const MH3RowsArgs a = rows_args(rows, dim, dtype, m, eps, flags);
        check(mh3_gate_add_rms_mod_rows(&a, x, y, m.gate, m.w, m.shift, m.scale, m.set_of_row, h, s_),
              "gate_add_rms_mod_rows");
    }
    // out = silu(gate) * up; up == nullptr: gate is fc1's [rows][2 dim] row [gate | up]
    void swiglu_rows(uint32_t rows, uint32_t dim, uint32_t dtype, const void* gate, const void* up, void* out) const
    {
        const MH3SwigluArgs a{rows, dim, up ? uint32_t(MH3_SWIGLU_SPLIT) : uint32_t(MH3_SWIGLU_FUSED), dtype};
        check(mh3_swiglu_rows(&a, gate, up, out, s_), "swiglu_rows");
    }

    void cube_pool(const Cubes& c, const uint16_t* q, const uint16_t* k, float* qc, float* kc,
                   int32_t* counts = nullptr) const
    {
        const MH3CubeArgs a = c.args();
        check(mh3_cube_pool(&a, q, k, qc, kc, counts, s_), "cube_pool");
    }
    void cube_scores(const Cubes& c, const float* qc, const float* kc, float* s) const
    {
        const MH3CubeArgs a = c.args();
        check(mh3_cube_scores(&a, qc, kc, s, s_), "cube_scores");
    }
    void cube_topk(const Cubes& c, const float* s, int32_t* idx, int32_t* cnt) const
    {
        const MH3CubeArgs a = c.args();
        check(mh3_cube_topk(&a, s, idx, cnt, s_), "cube_topk");
    }
    // cube_scores + cube_topk with the scores on chip; `workspace` of at least cube_select_workspace_bytes() bytes
    // holds the split key operands (overwritten by every call).
    static uint64_t cube_select_workspace_bytes(const Cubes& c)
    {
        const MH3CubeArgs a = c.args();
        const int64_t n = mh3_cube_select_workspace_bytes(&a);
        check(n < 0 ? int(n) : MH3_OK, "cube_select_workspace_bytes");
        return uint64_t(n);
    }
    void cube_select(const Cubes& c, const float* qc, const float* kc, void* workspace, uint64_t workspace_bytes,
                     int32_t* idx, int32_t* cnt) const
    {
        const MH3CubeArgs a = c.args();
        check(mh3_cube_select(&a, qc, kc, workspace, workspace_bytes, idx, cnt, s_), "cube_scores+cube_topk");
    }
    // The query-cube order for the ordered attention: each head's cubes sorted by the middle entry of their pass lists.
    void cube_order(const Cubes& c, const int32_t* idx, const int32_t* cnt, int32_t* order) const
    {
        const MH3CubeArgs a = c.args();
        check(mh3_cube_order(&a, idx, cnt, order, s_), "cube_order");
    }

    // H3::Cubes' map of begin(): attention row -> model row (-1 for a cube's padding slot), the cubes' 64 rows each
    // and then the n_dense dense rows; counts (may be null) the cubes' token counts.
    void cube_map(uint32_t grid_t, uint32_t grid_h, uint32_t grid_w, uint32_t n_dense, uint64_t video_row0,
                  uint64_t dense_row0, int32_t* map, int32_t* counts = nullptr) const
    {
        const MH3CubeMapArgs a{grid_t, grid_h, grid_w, n_dense, video_row0, dense_row0};
        check(mh3_cube_map(&a, map, counts, s_), "H3::Cubes");
    }

    // A step's conditioning: the sinusoidal embedding of each level t[u] through the F32 time MLP (temb) and
    // bf16(silu(temb)) (cond), with `workspace` of at least time_embed_workspace_bytes() bytes for its hidden layer.
    static uint64_t time_embed_workspace_bytes(const MH3TimeArgs& a)
    {
        const int64_t n = mh3_time_embed_workspace_bytes(&a);
        check(n < 0 ? int(n) : MH3_OK, "time_embed");
        return uint64_t(n);
    }
    void time_embed(const MH3TimeArgs& a, const float* t, const float* w_in, const float* b_in, const float* w_out,
                    const float* b_out, void* workspace, uint64_t workspace_bytes, float* temb, uint16_t* cond) const
    {
        check(mh3_time_embed(&a, t, w_in, b_in, w_out, b_out, workspace, workspace_bytes, temb, cond, s_),
              "time_embed");
    }
    // The same without a workspace, for callers that cannot allocate (code under HIP graph capture, serving loops):
    // the hidden layer in the library's own per-GPU array (levels x hidden at most 65,536 floats). Calls that
    // overlap in time on one GPU share that array and race; calls on one stream do not.
    void time_embed_noalloc(const MH3TimeArgs& a, const float* t, const float* w_in, const float* b_in,
                            const float* w_out, const float* b_out, float* temb, uint16_t* cond) const
    {
        check(mh3_time_embed_noalloc(&a, t, w_in, b_in, w_out, b_out, temb, cond, s_), "time_embed");
    }
    // A block's AdaLN projection: mod[levels][n] = w cond^T + bias, n = 3 x 6 x dim (the [U][3][6][D] table whose
    // (level, tag) sets the row kernels read at set_stride = 6 dim).
    void adaln_mod(uint32_t levels, uint32_t n, uint32_t k, const uint16_t* cond, const uint16_t* w, const float* bias,
                   float* mod) const
    {
        const MH3GemmArgs a{levels, n, k, 0, 0, 0};
        check(mh3_adaln_mod(&a, cond, w, bias, mod, s_), "adaln_proj");
    }
    // The pruned checkpoints' modulation: the curve table interpolated at each t, through w [n][width] plus bias.
    void curve_mods(uint32_t levels, uint32_t n, uint32_t points, uint32_t width, const float* t, const float* table,
                    const float* w, const float* bias, float* mod) const
    {
        const MH3CurveArgs a{levels, n, points, width};
        check(mh3_curve_mods(&a, t, table, w, bias, mod, s_), "curve_mods");
    }

    // After the QKV GEMM: the per-head RMS norm and rotary positions of q and k, v copied, written as head tiles;
    // with a cube map (map[r] = model row, -1 padding) in the cube order cube_pool, cube_select and
    // flash_attn_sparse_128 read as MH3_CUBES_GATHERED. v == nullptr skips v.
    void heads_partial(const Heads& hd, const uint16_t* qkv, const float* q_w, const float* k_w, const float* cos_t,
                       const float* sin_t, const int32_t* map, uint16_t* q, uint16_t* k, uint16_t* v) const
    {
        const MH3HeadsArgs a = hd.args();
        check(mh3_heads_partial(&a, qkv, q_w, k_w, cos_t, sin_t, map, q, k, v, s_), "heads_partial");
    }
    // heads_partial, then cube_pool over its output, in one pass: c is the geometry of the head tiles this call writes
    // (its strides those of hd's outputs), gathered through map, or in the model's order (MH3_CUBES_GRID, no map).
    void heads_partial_pool(const Heads& hd, const Cubes& c, const uint16_t* qkv, const float* q_w, const float* k_w,
                            const float* cos_t, const float* sin_t, const int32_t* map, uint16_t* q, uint16_t* k,
                            uint16_t* v, float* qc, float* kc, int32_t* counts = nullptr) const
    {
        const MH3HeadsArgs a = hd.args();
        const MH3CubeArgs ca = c.args();
        check(mh3_heads_partial_pool(&a, &ca, qkv, q_w, k_w, cos_t, sin_t, map, q, k, v, qc, kc, counts, s_),
              "heads_partial_pool");
    }
    // Flash attention over the pass lists idx / cnt of cube_select (or cube_topk) and the dense rows
    // [dense_row0, dense_row0 + n_dense); q, k, v and out in c's cube geometry. scale 0: 1 / sqrt(128).
    void flash_attn_sparse_128(const Cubes& c, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                               const int32_t* idx, const int32_t* cnt, uint64_t dense_row0, uint32_t n_dense,
                               uint16_t* out, float scale = 0.0f) const
    {
        const MH3AttnArgs a{c.args(), dense_row0, n_dense, scale};
        check(mh3_flash_attn_sparse_128(&a, q, k, v, idx, cnt, out, s_), "flash_attn_sparse_128");
    }
    // The same with the query cubes scheduled in cube_order's order (outputs equal up to summation order).
    void flash_attn_sparse_128(const Cubes& c, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                               const int32_t* idx, const int32_t* cnt, const int32_t* order, uint64_t dense_row0,
                               uint32_t n_dense, uint16_t* out, float scale = 0.0f) const
    {
        const MH3AttnArgs a{c.args(), dense_row0, n_dense, scale};
        check(mh3_flash_attn_sparse_128_ordered(&a, q, k, v, idx, cnt, order, out, s_), "flash_attn_sparse_128");
    }

    // Weight rows to int8 with one scale each (at load)
    void quant_rows_i8(uint32_t rows, uint32_t cols, uint32_t dtype, const void* w, int8_t* q, float* scale) const
    {
        const MH3QuantArgs a{rows, cols, dtype, 0};
        check(mh3_quant_rows_i8(&a, w, q, scale, s_), "quant_rows_i8");
    }
    // fc1 with int8 weights [2 ffn][dim] and SwiGLU: out[m][ffn] = silu(x Wg sg) * (x Wu su)
    void fc1_swiglu_i8(uint32_t m, uint32_t ffn, uint32_t dim, const uint16_t* x, const int8_t* w, const float* scale,
                       uint16_t* out) const
    {
        const MH3GemmArgs a{m, ffn, dim, 0, 0, 0};
        check(mh3_gemm_w8a16_swiglu(&a, x, w, scale, out, s_), "gemm_i8+swiglu_rows");
    }

    // The dense fc1 (--int8 none): bf16 weights [2 ffn][dim], no scale
    void fc1_swiglu_bf16(uint32_t m, uint32_t ffn, uint32_t dim, const uint16_t* x, const uint16_t* w,
                         uint16_t* out) const
    {
        const MH3GemmArgs a{m, ffn, dim, 0, 0, 0};
        check(mh3_gemm_bf16_swiglu(&a, x, w, out, s_), "Gemm::encode+swiglu_rows");
    }
    // The reference's own --int8 fc1: x quantized per row (quant_rows_i8), W8A8 gemm_i8 and SwiGLU
    void fc1_swiglu_w8a8(uint32_t m, uint32_t ffn, uint32_t dim, const int8_t* xq, const float* x_scale,
                         const int8_t* w, const float* w_scale, uint16_t* out) const
    {
        const MH3GemmArgs a{m, ffn, dim, 0, 0, 0};
        check(mh3_gemm_i8_swiglu(&a, xq, x_scale, w, w_scale, out, s_), "gemm_i8+swiglu_rows");
    }

    // The qkv projection (Gemm::encode, or gemm_i8 under --int8): out[m][n] = x w^T, w [n][k]. form: MH3_GEMM_BF16
    // (no scales), MH3_GEMM_W8A16 (int8 w with w_scale), MH3_GEMM_W8A8 (int8 x with x_scale, int8 w with w_scale).
    void gemm(uint32_t m, uint32_t n, uint32_t k, uint32_t form, const void* x, const float* x_scale, const void* w,
              const float* w_scale, uint16_t* out) const
    {
        const MH3GemmArgs a{m, n, k, 0, 0, 0};
        check(mh3_gemm(&a, form, x, x_scale, w, w_scale, out, s_), form == MH3_GEMM_BF16 ? "Gemm::encode" : "gemm_i8");
    }
    // The out projection and fc2 with gate_add_rows folded in: residual += gate[s] * (x w^T), in place; the gate,
    // its sets and set stride come from m (its norm fields are not used).
    void gemm_gate_add(uint32_t rows, uint32_t n, uint32_t k, uint32_t form, const void* x, const float* x_scale,
                       const void* w, const float* w_scale, const Modulation& m, uint16_t* residual) const
    {
        const MH3GemmArgs a{rows, n, k, m.n_sets, m.set_stride, 0};
        check(mh3_gemm_gate_add(&a, form, x, x_scale, w, w_scale, m.gate, m.set_of_row, residual, s_),
              form == MH3_GEMM_BF16 ? "Gemm::encode+gate_add_rows" : "gemm_i8+gate_add_rows");
    }
    // The same on the float residual stream: residual float [rows][n] += gate[s] * (x w^T).
    void gemm_gate_add(uint32_t rows, uint32_t n, uint32_t k, uint32_t form, const void* x, const float* x_scale,
                       const void* w, const float* w_scale, const Modulation& m, float* residual) const
    {
        const MH3GemmArgs a{rows, n, k, m.n_sets, m.set_stride, 0};
        check(mh3_gemm_gate_add_f32(&a, form, x, x_scale, w, w_scale, m.gate, m.set_of_row, residual, s_),
              form == MH3_GEMM_BF16 ? "Gemm::encode+gate_add_rows" : "gemm_i8+gate_add_rows");
    }

private:
    static MH3RowsArgs rows_args(uint32_t rows, uint32_t dim, uint32_t dtype, const Modulation& m, float eps,
                                 uint32_t flags = 0)
    {
        return MH3RowsArgs{rows, dim, m.n_sets, dtype, eps, m.set_stride, flags, 0};
    }
    hipStream_t s_;
};

} // namespace mako::h3
