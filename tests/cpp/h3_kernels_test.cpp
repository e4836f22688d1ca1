// The H3 block's hot-path kernels through the C++ host layer (mako_h3.hpp) on the GPU, against the CPU oracle
// (oracle/mh3_oracle.h), reported the way the reference's tests/h3_ref_test.cpp reports: one line per
// check, "ok" or "FAIL", the relative RMS error and the lowest row cosine of diff() (h3_ref_test.cpp:67-90), and
// the number of failures as the exit status.
//   h3_kernels_test [rows | swiglu | cubes | attn | int8 | proj | cond | errors | all]
#include "mako_h3.hpp"
#include "mh3_oracle.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

namespace {

using namespace mako::h3;

int failures = 0;

void check(bool ok, const std::string& what)
{
    std::printf("  %-4s %s\n", ok ? "ok" : "FAIL", what.c_str());
    std::fflush(stdout);
    failures += !ok;
}

// Relative RMS error over everything and the lowest cosine similarity of a row of `width` (the reference's diff()).
struct Diff {
    double rel = 0, min_cos = 1;
};
Diff diff(const std::vector<double>& got, const std::vector<double>& want, size_t width)
{
    Diff d;
    double e = 0, r = 0;
    for (size_t i = 0; i < want.size(); ++i) {
        e += (got[i] - want[i]) * (got[i] - want[i]);
        r += want[i] * want[i];
    }
    d.rel = r > 0 ? std::sqrt(e / r) : std::sqrt(e);
    for (size_t row = 0; row < want.size() / width; ++row) {
        double gw = 0, gg = 0, ww = 0;
        for (size_t i = row * width; i < (row + 1) * width; ++i)
            gw += got[i] * want[i], gg += got[i] * got[i], ww += want[i] * want[i];
        d.min_cos = std::min(d.min_cos, ww > 0 && gg > 0 ? gw / std::sqrt(gg * ww) : 1.0);
    }
    return d;
}

// Every element within rtol relative (plus atol), and the diff() pair, in one check line.
void compare(const std::string& what, const std::vector<double>& got, const std::vector<double>& want, size_t width,
             double rtol, double atol)
{
    if (got.size() != want.size()) {
        check(false, what + ": size mismatch");
        return;
    }
    size_t bad = 0;
    for (size_t i = 0; i < want.size(); ++i)
        bad += !(std::fabs(got[i] - want[i]) <= rtol * std::fabs(want[i]) + atol);
    const Diff d = diff(got, want, width);
    char msg[256];
    std::snprintf(msg, sizeof msg, "%s: %zu rows, rel error %.2e, lowest row cosine %.6f, %zu beyond tolerance",
                  what.c_str(), want.size() / width, d.rel, d.min_cos, bad);
    check(bad == 0, msg);
}

// Deterministic inputs: splitmix64 and Box-Muller.
struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed) {}
    uint64_t next()
    {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    double uniform() { return (double(next() >> 11) + 0.5) * 0x1.0p-53; }
    double normal() { return std::sqrt(-2.0 * std::log(uniform())) * std::cos(6.283185307179586 * uniform()); }
};

std::vector<float> normals(Rng& r, size_t n, double sd = 1.0, double mean = 0.0)
{
    std::vector<float> v(n);
    for (auto& x : v)
        x = float(mean + sd * r.normal());
    return v;
}
std::vector<uint16_t> bf16_normals(Rng& r, size_t n)
{
    std::vector<uint16_t> v(n);
    for (auto& x : v)
        x = mh3o_bf16_from_double(r.normal());
    return v;
}
std::vector<double> of_bf16(const std::vector<uint16_t>& v)
{
    std::vector<double> d(v.size());
    for (size_t i = 0; i < v.size(); ++i)
        d[i] = mh3o_bf16_to_float(v[i]);
    return d;
}
std::vector<double> of_f32(const std::vector<float>& v) { return {v.begin(), v.end()}; }

void rows()
{
    std::printf("rows\n");
    Rng r(0);
    {
        // Modulated RMS norm, fp32, 4096 x 1024 (the reference's CPU-runnable case), at 1e-5.
        const uint32_t n = 4096, d = 1024;
        auto x = normals(r, size_t(n) * d), shift = normals(r, d, 0.1), scale = normals(r, d, 0.1);
        auto w = normals(r, d, 0.02, 1.0);
        DeviceBuffer<float> dx(x), dw(w), dsh(shift), dsc(scale), dy(size_t(n) * d);
        Kernels k;
        Modulation m{dw.get(), dsh.get(), dsc.get(), nullptr, nullptr, 1};
        k.rms_mod_rows(n, d, MH3_F32, dx.get(), m, dy.get());
        k.finish();
        std::vector<float> want(x.size());
        mh3o_rms_mod_rows(n, d, 1e-6f, MH3O_F32, x.data(), w.data(), shift.data(), scale.data(), nullptr, want.data());
        compare("rms_mod_rows f32 4096x1024", of_f32(dy.download()), of_f32(want), d, 1e-5, 1e-6);
    }
    {
        // Fused modulated norm + gated residual, bf16, three modulation sets picked per row.
        const uint32_t n = 67, d = 5120, sets = 3;
        auto x = bf16_normals(r, size_t(n) * d), res = bf16_normals(r, size_t(n) * d);
        auto shift = normals(r, sets * d, 0.1), scale = normals(r, sets * d, 0.1), gate = normals(r, sets * d, 0.1);
        auto w = normals(r, d, 0.02, 1.0);
        std::vector<uint8_t> set(n);
        for (auto& s : set)
            s = uint8_t(r.next() % sets);
        DeviceBuffer<uint16_t> dx(x), dres(res), dout(size_t(n) * d);
        DeviceBuffer<float> dw(w), dsh(shift), dsc(scale), dg(gate);
        DeviceBuffer<uint8_t> dset(set);
        Kernels k;
        Modulation m{dw.get(), dsh.get(), dsc.get(), dg.get(), dset.get(), sets};
        k.rms_mod_gate_add_rows(n, d, MH3_BF16, dx.get(), dres.get(), m, dout.get());
        k.finish();
        std::vector<uint16_t> want(x.size());
        mh3o_rms_mod_gate_add_rows(n, d, 1e-6f, MH3O_BF16, x.data(), res.data(), w.data(), shift.data(), scale.data(),
                                   gate.data(), set.data(), want.data());
        compare("rms_mod_gate_add_rows bf16 67x5120, 3 sets", of_bf16(dout.download()), of_bf16(want), d, 1e-2, 1e-5);

        // The block's order in one pass equals gate_add_rows then rms_mod_rows, bit for bit.
        DeviceBuffer<uint16_t> xa(x), xb(x), ha(size_t(n) * d), hb(size_t(n) * d);
        k.gate_add_rms_mod_rows(n, d, MH3_BF16, xa.get(), dres.get(), m, ha.get());
        k.gate_add_rows(n, d, MH3_BF16, xb.get(), dres.get(), m);
        k.rms_mod_rows(n, d, MH3_BF16, xb.get(), m, hb.get());
        k.finish();
        check(xa.download() == xb.download() && ha.download() == hb.download(),
              "gate_add_rms_mod_rows == gate_add_rows then rms_mod_rows, bit for bit");
        std::vector<uint16_t> want_x = x;
        mh3o_gate_add_rows(n, d, MH3O_BF16, want_x.data(), res.data(), gate.data(), set.data());
        compare("gate_add_rows bf16 67x5120, 3 sets", of_bf16(xb.download()), of_bf16(want_x), d, 1e-2, 1e-5);
    }
}

void swiglu()
{
    std::printf("swiglu\n");
    Rng r(1);
    const uint32_t n = 130, d = 1000;
    auto gu = bf16_normals(r, size_t(n) * 2 * d);
    std::vector<uint16_t> g(size_t(n) * d), u(size_t(n) * d);
    for (uint32_t i = 0; i < n; ++i)
        for (uint32_t c = 0; c < d; ++c)
            g[size_t(i) * d + c] = gu[size_t(i) * 2 * d + c], u[size_t(i) * d + c] = gu[size_t(i) * 2 * d + d + c];
    DeviceBuffer<uint16_t> dgu(gu), dg(g), du(u), o1(size_t(n) * d), o2(size_t(n) * d);
    Kernels k;
    k.swiglu_rows(n, d, MH3_BF16, dgu.get(), nullptr, o1.get());
    k.swiglu_rows(n, d, MH3_BF16, dg.get(), du.get(), o2.get());
    k.finish();
    std::vector<uint16_t> want(size_t(n) * d);
    mh3o_swiglu_rows(n, d, MH3O_SWIGLU_FUSED, MH3O_BF16, gu.data(), nullptr, want.data());
    compare("swiglu_rows fused row bf16 130x1000", of_bf16(o1.download()), of_bf16(want), d, 1e-2, 1e-6);
    compare("swiglu_rows split bf16 130x1000", of_bf16(o2.download()), of_bf16(want), d, 1e-2, 1e-6);
}

void cubes()
{
    std::printf("cubes\n");
    Rng r(2);
    Cubes c;
    c.heads = 3, c.t = 8, c.h = 8, c.w = 12, c.ratio = 0.25f, c.local = 3;
    const uint32_t rows = c.t * c.h * c.w, C = c.count(), kk = c.k();
    auto q = bf16_normals(r, size_t(c.heads) * rows * 128), key = bf16_normals(r, size_t(c.heads) * rows * 128);
    DeviceBuffer<uint16_t> dq(q), dk(key);
    DeviceBuffer<float> qc(size_t(c.heads) * C * 128), kc(size_t(c.heads) * C * 128), s(size_t(c.heads) * C * C);
    DeviceBuffer<int32_t> counts(C), idx(size_t(c.heads) * C * c.out_stride()), cnt(size_t(c.heads) * C);
    DeviceBuffer<int32_t> idx2(size_t(c.heads) * C * c.out_stride()), cnt2(size_t(c.heads) * C);
    Kernels k;
    k.cube_pool(c, dq.get(), dk.get(), qc.get(), kc.get(), counts.get());
    k.cube_scores(c, qc.get(), kc.get(), s.get());
    k.cube_topk(c, s.get(), idx.get(), cnt.get());
    DeviceBuffer<uint8_t> ws(Kernels::cube_select_workspace_bytes(c));
    k.cube_select(c, qc.get(), kc.get(), ws.get(), ws.size(), idx2.get(), cnt2.get());
    k.finish();
    std::vector<float> wq(qc.size()), wk(kc.size());
    std::vector<int32_t> wc(C);
    mh3o_cube_pool(c.heads, 128, c.t, c.h, c.w, MH3O_CUBES_GRID, 0, uint64_t(rows) * 128, 128, q.data(), key.data(),
                   wq.data(), wk.data(), wc.data());
    compare("cube_pool q 3 heads, 8x8x12 grid", of_f32(qc.download()), of_f32(wq), 128, 1e-5, 1e-6);
    compare("cube_pool k 3 heads, 8x8x12 grid", of_f32(kc.download()), of_f32(wk), 128, 1e-5, 1e-6);
    check(counts.download() == wc, "cube_pool counts");
    std::vector<double> s64(s.size());
    mh3o_cube_scores(c.heads, C, 128, qc.download().data(), kc.download().data(), s64.data());
    const auto sg = s.download();
    double worst = 0;
    for (uint32_t row = 0; row < c.heads * C; ++row) {
        double m = 0;
        for (uint32_t j = 0; j < C; ++j)
            m = std::max(m, std::fabs(s64[size_t(row) * C + j]));
        for (uint32_t j = 0; j < C; ++j)
            worst = std::max(worst, std::fabs(sg[size_t(row) * C + j] - s64[size_t(row) * C + j]) / m);
    }
    check(worst <= 1e-5, "cube_scores within 1e-5 of the row's largest |score|");
    // The oracle's selection over the GPU's own float scores is the GPU's, bit for bit (fused and not).
    std::vector<double> sd(sg.begin(), sg.end());
    std::vector<int32_t> widx(idx.size()), wcnt(cnt.size());
    mh3o_cube_topk(c.heads, c.t, c.h, c.w, kk, c.local, c.out_stride(), sd.data(), widx.data(), wcnt.data());
    check(idx.download() == widx && cnt.download() == wcnt, "cube_topk == the oracle's top-k of the same scores");
    check(idx2.download() == widx && cnt2.download() == wcnt, "cube_select == cube_scores + cube_topk");
}

// heads_partial from one qkv tensor, gathered through the cube map, then the selector and flash_attn_sparse_128 on the
// gathered head tiles; each stage against the oracle run on the oracle's own outputs of the stage before.
void attn()
{
    std::printf("attn\n");
    Rng r(4);
    Cubes c;
    c.heads = 2, c.t = 7, c.h = 9, c.w = 10, c.ratio = 0.25f, c.local = 1, c.layout = MH3_CUBES_GATHERED;
    const uint32_t video = c.t * c.h * c.w, n_dense = 70, model_rows = n_dense + video, C = c.count();
    const uint32_t rows = 64 * C + n_dense, rot = 96, half = rot / 2;
    // The cube map: attention row 64 cube + slot -> the model row of that grid position (video after the text), -1
    // for padding slots; then the text rows.
    std::vector<int32_t> map(rows, -1);
    const uint32_t ch = (c.h + 3) / 4, cw = (c.w + 3) / 4;
    for (uint32_t cube = 0; cube < C; ++cube)
        for (uint32_t l = 0; l < 64; ++l) {
            const uint32_t t = 4 * (cube / (ch * cw)) + l / 16, y = 4 * (cube / cw % ch) + l / 4 % 4,
                           x = 4 * (cube % cw) + l % 4;
            if (t < c.t && y < c.h && x < c.w)
                map[64 * cube + l] = int32_t(n_dense + (t * c.h + y) * c.w + x);
        }
    for (uint32_t i = 0; i < n_dense; ++i)
        map[64 * C + i] = int32_t(i);
    auto qkv = bf16_normals(r, size_t(model_rows) * 3 * c.heads * 128);
    auto qw = normals(r, 128, 0.1, 1.0), kw = normals(r, 128, 0.1, 1.0);
    std::vector<float> cs(size_t(model_rows) * half), sn(cs.size());
    for (size_t i = 0; i < cs.size(); ++i) {
        const double a = 6.283185307179586 * (r.uniform() - 0.5);
        cs[i] = float(std::cos(a)), sn[i] = float(std::sin(a));
    }
    const size_t tile = size_t(c.heads) * rows * 128;
    DeviceBuffer<uint16_t> dqkv(qkv), q(tile), k(tile), v(tile), out(tile);
    DeviceBuffer<float> dqw(qw), dkw(kw), dcs(cs), dsn(sn), qc(size_t(c.heads) * C * 128), kc(qc.size());
    DeviceBuffer<int32_t> dmap(map), idx(size_t(c.heads) * C * c.out_stride()), cnt(size_t(c.heads) * C);
    Heads hd;
    hd.rows = rows, hd.model_rows = model_rows, hd.heads = c.heads, hd.rot = rot;
    c.head_stride = uint64_t(rows) * 128;
    Kernels kern;
    kern.heads_partial(hd, dqkv.get(), dqw.get(), dkw.get(), dcs.get(), dsn.get(), dmap.get(), q.get(), k.get(),
                       v.get());
    kern.cube_pool(c, q.get(), k.get(), qc.get(), kc.get());
    DeviceBuffer<uint8_t> ws(Kernels::cube_select_workspace_bytes(c));
    kern.cube_select(c, qc.get(), kc.get(), ws.get(), ws.size(), idx.get(), cnt.get());
    kern.flash_attn_sparse_128(c, q.get(), k.get(), v.get(), idx.get(), cnt.get(), 64ull * C, n_dense, out.get());
    kern.finish();
    std::vector<uint16_t> oq(tile), ok_(tile), ov(tile), oo(tile, 0);
    mh3o_heads_partial(rows, model_rows, c.heads, rot, 1e-6f, 3ull * c.heads * 128, uint64_t(rows) * 128, 128,
                       qkv.data(), qw.data(), kw.data(), cs.data(), sn.data(), map.data(), oq.data(), ok_.data(),
                       ov.data());
    compare("heads_partial q, gathered through the cube map", of_bf16(q.download()), of_bf16(oq), 128, 1e-2, 1e-3);
    compare("heads_partial k, gathered through the cube map", of_bf16(k.download()), of_bf16(ok_), 128, 1e-2, 1e-3);
    check(v.download() == ov, "heads_partial v (a copy) and padding rows (zeros) bit for bit");
    // Attention over the GPU's own pass lists, from the oracle's head tiles.
    const auto gi = idx.download(), gc = cnt.download();
    mh3o_attn_sparse(c.heads, c.t, c.h, c.w, MH3O_CUBES_GATHERED, 0, uint64_t(rows) * 128, 128, 64ull * C, n_dense,
                     1.0 / std::sqrt(128.0), oq.data(), ok_.data(), ov.data(), gi.data(), gc.data(), c.out_stride(),
                     oo.data());
    compare("flash_attn_sparse_128 over the gathered tiles, 2 heads, 7x9x10 grid + 70 text rows",
            of_bf16(out.download()), of_bf16(oo), 128, 1e-2, 3e-3);
    // cube_order: each head's cubes sorted by the middle entry of their pass lists, ties by index (a host sort); then
    // the attention with the query cubes in that order, against the same oracle outputs.
    DeviceBuffer<int32_t> order(size_t(c.heads) * C);
    DeviceBuffer<uint16_t> out2(tile);
    kern.cube_order(c, idx.get(), cnt.get(), order.get());
    kern.flash_attn_sparse_128(c, q.get(), k.get(), v.get(), idx.get(), cnt.get(), order.get(), 64ull * C, n_dense,
                               out2.get());
    kern.finish();
    std::vector<int32_t> want_order(size_t(c.heads) * C);
    for (uint32_t h = 0; h < c.heads; ++h) {
        auto mid = [&](int32_t cube) {
            const size_t item = size_t(h) * C + uint32_t(cube);
            const int32_t n = std::min(std::max(gc[item], 0), int32_t(c.out_stride()));
            const int32_t j = n > 0 ? gi[item * c.out_stride() + uint32_t(n) / 2] : -1;
            return j >= 0 && uint32_t(j) < C ? uint32_t(j) : C;
        };
        auto first = want_order.begin() + ptrdiff_t(h) * C;
        for (uint32_t i = 0; i < C; ++i)
            first[i] = int32_t(i);
        std::stable_sort(first, first + C, [&](int32_t a, int32_t b) { return mid(a) < mid(b); });
    }
    check(order.download() == want_order, "cube_order: cubes by the middle entry of their pass lists, ties by index");
    compare("flash_attn_sparse_128 with the query cubes in cube_order's order", of_bf16(out2.download()), of_bf16(oo),
            128, 1e-2, 3e-3);
    // heads_partial and cube_pool in one pass: the same bits as the two calls above.
    DeviceBuffer<uint16_t> q2(tile), k2(tile), v2(tile);
    DeviceBuffer<float> qc2(qc.size()), kc2(kc.size());
    DeviceBuffer<int32_t> counts2(C);
    kern.heads_partial_pool(hd, c, dqkv.get(), dqw.get(), dkw.get(), dcs.get(), dsn.get(), dmap.get(), q2.get(),
                            k2.get(), v2.get(), qc2.get(), kc2.get(), counts2.get());
    kern.finish();
    check(q2.download() == q.download() && k2.download() == k.download() && v2.download() == v.download(),
          "heads_partial_pool head tiles bit for bit as heads_partial's");
    check(qc2.download() == qc.download() && kc2.download() == kc.download(),
          "heads_partial_pool cube means bit for bit as cube_pool's over those tiles");
    std::vector<int32_t> want_counts(C);
    for (uint32_t cube = 0; cube < C; ++cube)
        want_counts[cube] = int32_t(std::count_if(map.begin() + 64 * cube, map.begin() + 64 * (cube + 1),
                                                  [](int32_t m) { return m >= 0; }));
    check(counts2.download() == want_counts, "heads_partial_pool token counts");
}

void int8()
{
    std::printf("int8\n");
    Rng r(3);
    const uint32_t m = 300, n = 384, d = 320;
    auto w = normals(r, size_t(2) * n * d, 0.05);
    DeviceBuffer<float> dw(w), ds(2 * n);
    DeviceBuffer<int8_t> dq(size_t(2) * n * d);
    Kernels k;
    k.quant_rows_i8(2 * n, d, MH3_F32, dw.get(), dq.get(), ds.get());
    k.finish();
    std::vector<int8_t> wq(dq.size());
    std::vector<float> ws(2 * n);
    mh3o_quant_rows_i8(2 * n, d, MH3O_F32, w.data(), wq.data(), ws.data());
    check(dq.download() == wq && ds.download() == ws, "quant_rows_i8 bit for bit, 768x320");
    auto x = bf16_normals(r, size_t(m) * d);
    DeviceBuffer<uint16_t> dx(x), out(size_t(m) * n);
    k.fc1_swiglu_i8(m, n, d, dx.get(), dq.get(), ds.get(), out.get());
    k.finish();
    std::vector<uint16_t> want(size_t(m) * n);
    mh3o_gemm_w8a16_swiglu(m, n, d, x.data(), wq.data(), ws.data(), want.data());
    compare("fc1 int8 + swiglu 300x320 -> 384", of_bf16(out.download()), of_bf16(want), n, 1e-2, 1e-4);

    // The dense bf16 fc1 and the W8A8 fc1 (x quantized per row), against the oracle.
    std::vector<uint16_t> wb(size_t(2) * n * d);
    for (size_t i = 0; i < wb.size(); ++i)
        wb[i] = mh3o_bf16_from_float(w[i]);
    DeviceBuffer<uint16_t> dwb(wb);
    k.fc1_swiglu_bf16(m, n, d, dx.get(), dwb.get(), out.get());
    k.finish();
    mh3o_gemm_bf16_swiglu(m, n, d, x.data(), wb.data(), want.data());
    compare("fc1 bf16 + swiglu 300x320 -> 384", of_bf16(out.download()), of_bf16(want), n, 1e-2, 1e-4);
    const uint32_t d8 = 384; // the W8A8 GEMM takes k in steps of 128
    auto x8 = bf16_normals(r, size_t(m) * d8);
    auto w8 = normals(r, size_t(2) * n * d8, 0.05);
    DeviceBuffer<uint16_t> dx8(x8);
    DeviceBuffer<float> dw8(w8), dxs(m), dws(2 * n);
    DeviceBuffer<int8_t> dxq(size_t(m) * d8), dwq(size_t(2) * n * d8);
    k.quant_rows_i8(m, d8, MH3_BF16, dx8.get(), dxq.get(), dxs.get());
    k.quant_rows_i8(2 * n, d8, MH3_F32, dw8.get(), dwq.get(), dws.get());
    k.fc1_swiglu_w8a8(m, n, d8, dxq.get(), dxs.get(), dwq.get(), dws.get(), out.get());
    k.finish();
    std::vector<int8_t> oxq(size_t(m) * d8), owq(size_t(2) * n * d8);
    std::vector<float> oxs(m), ows(2 * n);
    mh3o_quant_rows_i8(m, d8, MH3O_BF16, x8.data(), oxq.data(), oxs.data());
    mh3o_quant_rows_i8(2 * n, d8, MH3O_F32, w8.data(), owq.data(), ows.data());
    check(dxq.download() == oxq && dxs.download() == oxs, "quant_rows_i8 of bf16 activations bit for bit");
    mh3o_gemm_i8_swiglu(m, n, d8, oxq.data(), oxs.data(), owq.data(), ows.data(), want.data());
    compare("fc1 W8A8 gemm_i8 + swiglu 300x384 -> 384", of_bf16(out.download()), of_bf16(want), n, 1e-2, 1e-4);
}

// The qkv projection (plain store) and the out / fc2 projections with the gate-add epilogue, one operand form each.
void proj()
{
    std::printf("proj\n");
    Rng r(5);
    const uint32_t m = 300, n = 512, k = 384, sets = 3;
    auto x = bf16_normals(r, size_t(m) * k);
    std::vector<uint16_t> wb(size_t(n) * k);
    for (auto& v : wb)
        v = mh3o_bf16_from_double(0.02 * r.normal());
    std::vector<int8_t> w8(size_t(n) * k), x8(size_t(m) * k);
    for (auto& v : w8)
        v = int8_t(int(r.next() % 255) - 127);
    for (auto& v : x8)
        v = int8_t(int(r.next() % 255) - 127);
    std::vector<float> ws(n), xs(m);
    for (auto& v : ws)
        v = float(0.5e-3 + 1.5e-3 * r.uniform());
    for (auto& v : xs)
        v = float(0.5e-2 + 1.5e-2 * r.uniform());
    auto gate = normals(r, sets * n, 0.5);
    std::vector<uint8_t> set(m);
    for (auto& v : set)
        v = uint8_t(r.next() % sets);
    auto res = bf16_normals(r, size_t(m) * n);
    DeviceBuffer<uint16_t> dx(x), dwb(wb), out(size_t(m) * n), dres1(res), dres2(res);
    DeviceBuffer<int8_t> dw8(w8), dx8(x8);
    DeviceBuffer<float> dws(ws), dxs(xs), dgate(gate);
    DeviceBuffer<uint8_t> dset(set);
    Kernels kern;
    Modulation mod;
    mod.gate = dgate.get(), mod.set_of_row = dset.get(), mod.n_sets = sets;
    kern.gemm(m, n, k, MH3_GEMM_BF16, dx.get(), nullptr, dwb.get(), nullptr, out.get());
    kern.gemm_gate_add(m, n, k, MH3_GEMM_W8A16, dx.get(), nullptr, dw8.get(), dws.get(), mod, dres1.get());
    kern.gemm_gate_add(m, n, k, MH3_GEMM_W8A8, dx8.get(), dxs.get(), dw8.get(), dws.get(), mod, dres2.get());
    kern.finish();
    std::vector<uint16_t> want(size_t(m) * n), w1 = res, w2 = res;
    mh3o_gemm(m, n, k, 1, 0, x.data(), nullptr, wb.data(), nullptr, nullptr, nullptr, 0, want.data());
    mh3o_gemm(m, n, k, 0, 1, x.data(), nullptr, w8.data(), ws.data(), gate.data(), set.data(), n, w1.data());
    mh3o_gemm(m, n, k, 2, 1, x8.data(), xs.data(), w8.data(), ws.data(), gate.data(), set.data(), n, w2.data());
    compare("qkv projection bf16 300x384 -> 512", of_bf16(out.download()), of_bf16(want), n, 1e-2, 1e-3);
    compare("out / fc2 projection W8A16 + gate_add_rows, 3 sets", of_bf16(dres1.download()), of_bf16(w1), n, 1e-2,
            2e-2);
    compare("out / fc2 projection W8A8 + gate_add_rows, 3 sets", of_bf16(dres2.download()), of_bf16(w2), n, 1e-2,
            2e-2);
}

// H3::Cubes' map and a step's conditioning (the time MLP, a block's AdaLN projection, the pruned curve) through the
// C++ layer, against the oracle; the table then feeds the fused row op through set_stride = 6 D.
void cond()
{
    std::printf("cond\n");
    Kernels k;
    {
        const uint32_t T = 37, H = 24, W = 42, nd = 640;
        const int64_t C = mh3_cube_count(T, H, W);
        const size_t cubes = size_t(C);
        DeviceBuffer<int32_t> map(cubes * 64 + nd), counts(cubes);
        k.cube_map(T, H, W, nd, nd, 0, map.get(), counts.get());
        std::vector<int32_t> wm(map.size()), wc(counts.size());
        mh3o_cube_map(T, H, W, nd, nd, 0, wm.data(), wc.data());
        check(map.download() == wm && counts.download() == wc,
              "H3::Cubes map of the padded 37 x 24 x 42 grid (660 cubes) + 640 dense rows, bit for bit");
    }
    Rng r(7);
    const uint32_t levels = 3, fd = 256, hid = 1024, D = 1024, od = D / 2, n = 18 * D;
    auto w_in = normals(r, size_t(hid) * fd, 1.0 / 16), b_in = normals(r, hid, 0.1);
    auto w_out = normals(r, size_t(od) * hid, 1.0 / 32), b_out = normals(r, od, 0.1);
    const std::vector<float> t = {0.9230769f, 0.5f, 0.999f};
    DeviceBuffer<float> dt(t), dwi(w_in), dbi(b_in), dwo(w_out), dbo(b_out), temb(size_t(levels) * od);
    DeviceBuffer<uint16_t> cond(size_t(levels) * od);
    const MH3TimeArgs ta{levels, fd, hid, od, 10000.0f, {0, 0, 0}};
    DeviceBuffer<uint8_t> ws(Kernels::time_embed_workspace_bytes(ta));
    k.time_embed(ta, dt.get(), dwi.get(), dbi.get(), dwo.get(), dbo.get(), ws.get(), ws.size(), temb.get(),
                 cond.get());
    std::vector<float> wt(temb.size());
    std::vector<uint16_t> wcond(cond.size());
    mh3o_time_embed(levels, fd, hid, od, 10000.0, t.data(), w_in.data(), b_in.data(), w_out.data(), b_out.data(),
                    wt.data(), wcond.data());
    compare("time embedding (256 -> 1024 -> 512, 3 levels)", of_f32(temb.download()), of_f32(wt), od, 1e-4, 1e-5);
    {
        // Without a workspace: the same bits as the call above.
        DeviceBuffer<float> temb2(temb.size());
        DeviceBuffer<uint16_t> cond2(cond.size());
        k.time_embed_noalloc(ta, dt.get(), dwi.get(), dbi.get(), dwo.get(), dbo.get(), temb2.get(), cond2.get());
        check(temb2.download() == temb.download() && cond2.download() == cond.download(),
              "time embedding without a workspace, bit for bit the same as with one");
    }
    // The projection over the GPU's own cond, so that it is tested alone.
    std::vector<uint16_t> wa(size_t(n) * od);
    for (auto& x : wa)
        x = mh3o_bf16_from_double(0.02 * r.normal());
    auto bias = normals(r, n, 0.01);
    DeviceBuffer<uint16_t> dwa(wa);
    DeviceBuffer<float> dbias(bias), mod(size_t(levels) * n);
    k.adaln_mod(levels, n, od, cond.get(), dwa.get(), dbias.get(), mod.get());
    const auto gcond = cond.download();
    std::vector<float> wmod(mod.size());
    mh3o_adaln_mod(levels, n, od, gcond.data(), wa.data(), bias.data(), wmod.data());
    compare("AdaLN projection (512 -> 18 x 1024, 3 levels)", of_f32(mod.download()), of_f32(wmod), D, 1e-4, 1e-5);
    // The pruned checkpoints' curve.
    auto table = normals(r, 1025 * 8), wc8 = normals(r, size_t(n) * 8);
    DeviceBuffer<float> dtab(table), dwc(wc8), cmod(size_t(levels) * n);
    k.curve_mods(levels, n, 1025, 8, dt.get(), dtab.get(), dwc.get(), dbias.get(), cmod.get());
    std::vector<float> wcm(cmod.size());
    mh3o_curve_mods(levels, n, 1025, 8, t.data(), table.data(), wc8.data(), bias.data(), wcm.data());
    compare("pruned curve modulation ([1025][8] table, 3 levels)", of_f32(cmod.download()), of_f32(wcm), D, 1e-4,
            1e-5);
    // The table's (level, tag) sets into the fused row op: set 3 u + tag at set_stride 6 D.
    const uint32_t rows = 96;
    auto x = bf16_normals(r, size_t(rows) * D), res = bf16_normals(r, size_t(rows) * D);
    std::vector<uint8_t> sets(rows);
    for (uint32_t i = 0; i < rows; ++i)
        sets[i] = uint8_t(i % 9);
    auto nw = normals(r, D, 0.02, 1.0);
    DeviceBuffer<uint16_t> dx(x), dres(res), dout(size_t(rows) * D);
    DeviceBuffer<uint8_t> dsets(sets);
    DeviceBuffer<float> dnw(nw);
    Modulation m;
    m.w = dnw.get(), m.shift = mod.get(), m.scale = mod.get() + D, m.gate = mod.get() + 2 * D;
    m.set_of_row = dsets.get(), m.n_sets = 9, m.set_stride = 6 * D;
    k.rms_mod_gate_add_rows(rows, D, MH3_BF16, dx.get(), dres.get(), m, dout.get());
    const auto gmod = mod.download();
    std::vector<float> sh(9 * D), sc(9 * D), ga(9 * D);
    for (uint32_t s = 0; s < 9; ++s)
        for (uint32_t j = 0; j < D; ++j) {
            sh[s * D + j] = gmod[(size_t(s) * 6 + 0) * D + j];
            sc[s * D + j] = gmod[(size_t(s) * 6 + 1) * D + j];
            ga[s * D + j] = gmod[(size_t(s) * 6 + 2) * D + j];
        }
    std::vector<uint16_t> want(size_t(rows) * D);
    mh3o_rms_mod_gate_add_rows(rows, D, 1e-6f, MH3O_BF16, x.data(), res.data(), nw.data(), sh.data(), sc.data(),
                               ga.data(), sets.data(), want.data());
    compare("fused rows with 9 (level, tag) sets from the [3][3][6][D] table", of_bf16(dout.download()), of_bf16(want),
            D, 1e-2, 1e-5);
    k.finish();
}

void errors()
{
    std::printf("errors\n");
    Kernels k;
    auto throws = [](const std::function<void()>& f) {
        try {
            f();
        } catch (const std::runtime_error&) {
            return true;
        }
        return false;
    };
    DeviceBuffer<uint16_t> a(64), b(64);
    Modulation m;
    check(throws([&] { k.rms_mod_rows(8, 7, MH3_BF16, a.get(), m, b.get()); }), "a row width not a multiple of 8 throws");
    check(throws([&] { k.rms_mod_rows(8, 8, 9, a.get(), m, b.get()); }), "an unknown dtype throws");
    check(throws([&] { k.swiglu_rows(8, 8, MH3_BF16, nullptr, nullptr, b.get()); }), "a null gate throws");
    Cubes c;
    c.heads = 1, c.t = 4, c.h = 4, c.w = 4, c.local = 2;
    check(throws([&] { (void)c.args(); }), "local 2 throws (H3::set_sparse's domain is 0, 1, 3)");
    c.local = 1;
    DeviceBuffer<int32_t> lists(64), counts(16), order(16);
    check(throws([&] { k.cube_order(c, lists.get(), counts.get(), nullptr); }), "cube_order without an order throws");
    check(throws([&] { k.cube_order(c, lists.get(), counts.get(), counts.get()); }),
          "cube_order writing over the counts throws");
    Cubes big = c;
    big.t = 64, big.h = 64, big.w = 68; // 16 x 16 x 17 = 4352 cubes, above cube_order's 4096
    DeviceBuffer<int32_t> big_lists(size_t(big.count()) * big.out_stride()), big_counts(big.count()),
        big_order(big.count());
    check(throws([&] { k.cube_order(big, big_lists.get(), big_counts.get(), big_order.get()); }),
          "cube_order beyond 4096 cubes throws");
    check(parse_int8("fc1,qkv") == std::optional<uint32_t>(MH3_INT8_FC1 | MH3_INT8_QKV), "parse_int8 fc1,qkv");
    check(!parse_int8("fc3"), "parse_int8 fc3 has no value");
}

} // namespace

int main(int argc, char** argv)
{
    const std::string mode = argc > 1 ? argv[1] : "all";
    int devices = 0;
    if (hipGetDeviceCount(&devices) != hipSuccess || devices == 0) {
        std::printf("no GPU: skipped\n");
        return 77;
    }
    try {
        if (mode == "rows" || mode == "all")
            rows();
        if (mode == "swiglu" || mode == "all")
            swiglu();
        if (mode == "cubes" || mode == "all")
            cubes();
        if (mode == "attn" || mode == "all")
            attn();
        if (mode == "int8" || mode == "all")
            int8();
        if (mode == "proj" || mode == "all")
            proj();
        if (mode == "cond" || mode == "all")
            cond();
        if (mode == "errors" || mode == "all")
            errors();
    } catch (const std::exception& e) {
        std::printf("  FAIL %s\n", e.what());
        ++failures;
    }
    std::printf("%d failure%s\n", failures, failures == 1 ? "" : "s");
    return failures;
}
