// C-ABI entry points: argument validation, recipe resolution and dispatch.
//
// Each dg_* function mirrors one registered API of the reference pybind module
// and runs the reference's checks in the same order:
//   - major / shape / dtype checks: csrc/utils/layout.hpp:17-82
//   - early_return (empty problems, K == 0, C vs D): csrc/apis/gemm.hpp:17-53
//   - recipe and SF layout checks: csrc/apis/layout.hpp:11-87,
//     csrc/utils/layout.hpp:84-140
//   - the three GEMMs: csrc/apis/gemm.hpp:78-133, 181-250, 269-318
// Failures raise dgm::Error, converted at the boundary into a status code and
// the thread-local message returned by dg_last_error().
#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstring>
#include <string>
#include <tuple>

#include "dg_internal.hpp"

namespace dgm {
namespace {

thread_local std::string t_last_error;
thread_local std::string t_last_config;

// Process-wide knobs (the reference keeps them in lazily created singletons,
// csrc/runtime/runtime.hpp:104, csrc/jit_kernels/heuristics/runtime.hpp:67).
constexpr int kDefaultMKAlignment = 128;
// Dense calls of at most this many rows run on the weight-streaming kernel
// (measured on MI355X over the DeepSeek-V3 (N, K) shapes: faster than every
// tiled configuration up to 64 rows, slower from 128).
constexpr int kDenseStreamRows = 64;
// Dense calls of at most 64 rows, and of at most 128 (256, see below) rows with
// K <= 8192, take the tiny-M kernel (K split over a workgroup's waves, rows split over workgroups)
// unless the streaming kernel
// already has this many workgroups (N >= 8192 or so). Measured on MI355X at M = 1, 16, 17, 32
// and 64: 1.2-2.6x faster for N <= 7168, slower at N = 24576 and 32768 and
// even at 7168 x 2048 with 64 rows. At 80-128 rows (flushed, per launch) it
// takes 24-31 us against 46-51 us for the best tiled launch at 2112 x 7168,
// 14-18 against 45-51 at 576 x 7168 and 21 against 30-34 at 4096 x 4096, ties
// at 7168 x 2048, and loses at K = 16384 (97-120 against 93-102 us). At 129-256
// rows it wins only where the tiled launch is small and its own launch fits one
// round: 160-256 x 576 x 7168 18-24 against 48-50 us, 160-192 x 2112 x 7168 31
// against 48; it loses at 256 x 2112 (two rounds, 55 against 50) and wherever
// the tiled launch has 64 tiles or more (N >= 4096).
constexpr int64_t kTinyMWideMaxK = 8192;
constexpr int64_t kTinyMWideMaxTiles = 64;   // 128 x 128 tiles of the tiled launch
constexpr int kTinyMStreamGrid = 64;

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// The tiny-M kernel's workgroup shape: rows (16, 32 or 64) x columns (16 or 32).
// A workgroup reads (rows + columns) x K bytes (A's rows once, all of K, and its
// B rows), and the launch runs ceil(workgroups / CUs) rounds of them; the model
// takes the fewest bytes per CU, and on equal cost more columns. Measured
// (flushed, per launch): 64 x 2112 x 7168 29.3 -> 23.9 us (32 x 32 against
// 64 x 16), 64 x 576 x 7168 29.0 -> 14.7, 64 x 4096 x 4096 20.9 -> 15.0; the
// N = 7168 shapes keep 64-row workgroups. 8 waves pay with 16 columns, 16 rows
// and long K (at 32 columns they are slower: 21.6 against 18.1 us at
// 32 x 2112 x 7168).
TileConfig choose_tinym(int64_t m, int64_t n, int64_t k, int cus) {
    const int64_t m16 = ceil_div(m, 16) * 16;
    int best_rows = kTinyMRows, best_cols = 16;
    int64_t best = INT64_MAX;
    for (int cols : {32, 16})
        for (int rows : {64, 32, 16}) {
            const int64_t wgs = ceil_div(n, (int64_t)cols) * ceil_div(m, (int64_t)rows);
            const int64_t cost = ceil_div(wgs, (int64_t)cus) * (std::min<int64_t>(rows, m16) + cols);
            if (cost < best) best = cost, best_rows = rows, best_cols = cols;
        }
    const bool eight = std::min<int64_t>(best_rows, m16) <= 16 && k / 128 >= 48 && best_cols == 16;
    return TileConfig{best_rows, best_cols, eight ? 8 : 9};
}
std::atomic<int> g_num_sms{0};                 // 0: query the device
std::atomic<int> g_mk_alignment{kDefaultMKAlignment};
std::atomic<int> g_tile_variant{0}, g_tile_m{0}, g_tile_n{0};   // variant 0: heuristic

template <typename F>
int guarded(F&& f) {
    try {
        f();
        t_last_error.clear();
        return DG_OK;
    } catch (const Error& e) {
        t_last_error = e.what();
        return e.code();
    } catch (const std::exception& e) {
        t_last_error = std::string("Internal error: ") + e.what();
        return DG_ERR_INTERNAL;
    } catch (...) {
        t_last_error = "Internal error: unknown exception";
        return DG_ERR_INTERNAL;
    }
}

int64_t align_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

int elem_size(int dtype) {
    switch (dtype) {
        case DG_F32: case DG_I32: return 4;
        case DG_BF16: case DG_F16: return 2;
        case DG_E4M3: case DG_I8: case DG_U8: return 1;
        case DG_I64: return 8;
        default: return 0;
    }
}

// Light view over dg_tensor with Python-style negative indices.
struct View {
    const dg_tensor* t;
    int dim() const { return t->ndim; }
    int64_t size(int i) const { return t->sizes[i < 0 ? i + t->ndim : i]; }
    int64_t stride(int i) const { return t->strides[i < 0 ? i + t->ndim : i]; }
    int dtype() const { return t->dtype; }
    const void* data() const { return t->data; }
    bool on_device() const { return t->device >= 0; }
};

View view(const dg_tensor* t, const char* name) {
    if (t == nullptr) throw Error(DG_ERR_INVALID, "Assertion", __FILE__, __LINE__, std::string(name) + " != nullptr");
    DG_CHECK(t->ndim >= 0 && t->ndim <= 4);
    DG_CHECK(elem_size(t->dtype) > 0);
    return View{t};
}

// csrc/utils/layout.hpp:18-27
void major_check(const View& t) {
    DG_CHECK(t.dim() == 2 || t.dim() == 3);
    if (t.dim() == 3) DG_CHECK(t.stride(0) == t.size(-2) * t.size(-1));
    DG_CHECK(t.stride(-2) == 1 || t.stride(-1) == 1);
}

// csrc/utils/layout.hpp:29-33: true = K-major
bool is_k_major(const View& t) {
    major_check(t);
    return t.stride(-1) == 1;
}

// csrc/utils/layout.hpp:35-40
void check_major_type_cd(const View& t) {
    major_check(t);
    DG_CHECK(t.stride(-1) == 1);
}

// csrc/utils/layout.hpp:48-55 (the device check replaces is_cuda)
void check_shape(const View& t, int n) {
    DG_CHECK(t.on_device());
    DG_CHECK(t.dim() == n);
}

bool is_fp4(const View& t) { return t.dtype() == DG_I8; }

// csrc/utils/layout.hpp:66-73: (mn, logical k); packed FP4 doubles K.
std::pair<int64_t, int64_t> check_ab(const View& t) {
    check_shape(t, 2);
    int64_t mn = t.size(0), k = t.size(1);
    if (t.dtype() != DG_E4M3) {
        DG_CHECK(t.dtype() == DG_I8);
        k *= 2;
    }
    return {mn, k};
}

// csrc/utils/layout.hpp:75-82
void check_grouped_ab(const View& t, int64_t& g, int64_t& mn, int64_t& k) {
    check_shape(t, 3);
    g = t.size(0), mn = t.size(1), k = t.size(2);
    if (t.dtype() != DG_E4M3) {
        DG_CHECK(t.dtype() == DG_I8);
        k *= 2;
    }
}

// Alignment rules of the gfx950 kernels: operand rows are read as 16-byte
// vectors and D rows written as 8/16-byte vectors. The reference imposes the
// same 16-byte rule through its TMA descriptors (runtime_utils.hpp:119-159).
void check_vector_alignment(const View& t, const char* what) {
    const auto addr = reinterpret_cast<uintptr_t>(t.data());
    const int64_t row_bytes = t.stride(-2) * elem_size(t.dtype());
    if (addr % 16 != 0 || (t.size(-2) > 1 && row_bytes % 16 != 0) ||
        (t.dim() == 3 && t.size(0) > 1 && (t.stride(0) * elem_size(t.dtype())) % 16 != 0))
        throw Error(DG_ERR_INVALID, "Assertion", __FILE__, __LINE__,
                    std::string(what) + ": base address and row pitch must be 16-byte aligned");
}

struct Recipe {
    int gran_mn_a, gran_k_a, gran_mn_b, gran_k_b;
};

// csrc/utils/layout.hpp:84-98 for this device: FP32 SFB -> (1, 128, 128),
// packed UE8M0 SFB -> (1, 1, 128).
void default_recipe(const View& sfa, const View& sfb, int out[3]) {
    DG_CHECK(sfb.dtype() == DG_F32 || sfb.dtype() == DG_I32);
    (void)sfa;
    out[0] = 1;
    out[1] = sfb.dtype() == DG_F32 ? 128 : 1;
    out[2] = 128;
}

// csrc/apis/layout.hpp:60-87 (pair resolution)
Recipe resolve_recipe(const dg_recipe* r, const View& sfa, const View& sfb) {
    dg_recipe rr{};
    if (r) rr = *r;
    if (!rr.has_recipe_ab && !rr.has_recipe) {
        default_recipe(sfa, sfb, rr.recipe);
        rr.has_recipe = 1;
    }
    DG_CHECK((rr.has_recipe_ab != 0) != (rr.has_recipe != 0));
    Recipe out{};
    if (rr.has_recipe) {
        out = {rr.recipe[0], rr.recipe[2], rr.recipe[1], rr.recipe[2]};
    } else {
        out = {rr.recipe_a[0], rr.recipe_a[1], rr.recipe_b[0], rr.recipe_b[1]};
    }
    DG_CHECK(out.gran_mn_a > 0 && out.gran_k_a > 0 && out.gran_mn_b > 0 && out.gran_k_b > 0);
    return out;
}

// csrc/utils/layout.hpp:100-140 (shape part): SF [(G,) ceil(mn/gran_mn), ceil(k/(gran_k*(4 if int)))]
void check_sf_layout(const View& sf, int64_t mn, int64_t k, int gran_mn, int gran_k, int64_t num_groups) {
    DG_CHECK(sf.dtype() == DG_F32 || sf.dtype() == DG_I32);
    DG_CHECK(sf.on_device());
    DG_CHECK(sf.dim() == (num_groups >= 0 ? 3 : 2));
    if (num_groups >= 0) DG_CHECK(sf.size(-3) == num_groups);
    DG_CHECK(sf.size(-2) == ceil_div(mn, gran_mn));
    DG_CHECK(sf.size(-1) == ceil_div(k, (int64_t)gran_k * (sf.dtype() == DG_F32 ? 1 : 4)));
}

// Packed-UE8M0 layout requirement (csrc/utils/layout.hpp:121-130): MN-major words.
void check_packed_sf_strides(const View& sf, int64_t mn) {
    DG_CHECK(sf.stride(-2) == 1 || mn == 1);
    DG_CHECK(sf.stride(-1) >= align_up(mn, 4));
}

int num_sms_now() {
    int v = g_num_sms.load();
    if (v > 0) return v;
    int dev = 0;
    DG_HIP_CHECK(hipGetDevice(&dev));
    DG_HIP_CHECK(hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev));
    return v;
}

// ---------------------------------------------------------------- early return

// csrc/apis/gemm.hpp:17-53. Returns true when the call is fully handled.
// Unlike the reference, a C that differs from D is not copied into D first:
// the kernels read C and write D directly (D = C + A.B^T in the epilogue).
bool early_return(int64_t m, int64_t n, int64_t k, const View& d, const dg_tensor* c, hipStream_t stream) {
    if (m == 0 || n == 0) return true;
    bool same = false;
    if (c) {
        const View cv = view(c, "c");
        same = cv.data() == d.data();
        if (same) {
            DG_CHECK(cv.dim() == d.dim());
            for (int i = 0; i < d.dim(); ++i) DG_CHECK(cv.size(i) == d.size(i) && cv.stride(i) == d.stride(i));
        }
    }
    DG_CHECK(d.dtype() == DG_BF16 || d.dtype() == DG_F32 || d.dtype() == DG_E4M3);
    // An FP8 D needs an SFD output, which these entry points do not take (gemm.hpp:31).
    DG_CHECK(d.dtype() != DG_E4M3);
    if (c) {
        const View cv = view(c, "c");
        check_major_type_cd(cv);
        DG_CHECK(d.dtype() == cv.dtype());
        DG_CHECK(cv.on_device());
        DG_CHECK(cv.dim() == d.dim());
        for (int i = 0; i < d.dim(); ++i) DG_CHECK(cv.size(i) == d.size(i));
    }
    if (k == 0) {
        if (!same) {
            const View cv = c ? view(c, "c") : d;
            launch_fill_or_copy(const_cast<void*>(d.data()), c ? cv.data() : nullptr, (int)m, (int)n, 1, d.stride(-2),
                                0, c ? cv.stride(-2) : 0, 0, elem_size(d.dtype()), stream);
        }
        return true;
    }
    return false;
}

// ---------------------------------------------------------------- heuristics

const char* kind_name(GemmKind k) {
    switch (k) {
        case kNormal: return "normal";
        case kContiguous: return "m_grouped_contiguous";
        case kMasked: return "m_grouped_masked";
        case kPsum: return "m_grouped_contiguous_psum";
        case kKGrouped: return "k_grouped_contiguous";
    }
    return "?";
}

// Tile choice for the FP32-scale kernels. A candidate's cost is the number of
// rounds of resident workgroups it needs times the work of one tile divided by
// that candidate's relative throughput (measured MFMA efficiency of the tile
// shape and pipeline). Grouped kinds need block_m to divide the row alignment.
// Whether a block_m fits the contiguous / psum segment alignment: a block may
// not straddle two groups, except that the LDS-pipelined kernels' 256-row tile
// runs once per 128-row block when their experts differ (contiguous layout only).
bool grouped_tile_ok(GemmKind kind, int variant, int bm, int align_m) {
    if (kind == kContiguous) return align_m % bm == 0 || (variant >= 2 && bm == 256 && align_m % 128 == 0);
    if (kind == kPsum) return align_m % bm == 0;
    return true;
}

TileConfig choose_tile_1d2d(GemmKind kind, int64_t m_rows, int64_t n, int64_t k, int64_t groups, int align_m) {
    const int tv = g_tile_variant.load(), tm = g_tile_m.load(), tn = g_tile_n.load();
    // The pipelined kernel keeps one SFB value per K block in LDS (up to 1024 blocks).
    const bool pipe_ok = ceil_div(k, 128) <= 1024;
    // The 256 x 256 pipelined tile is not built for K % 128 != 0 (its K-tail
    // schedule spills registers); the other tiles give the same bits.
    const bool tile256_ok = k % 128 == 0;
    if (tv == 4) {   // persistent form of the pipelined kernel
        if (!pipe_ok || tm != 256 || tn != 256) DG_UNSUPPORTED("tile override: the persistent kernel is 256 x 256");
        if (!tile256_ok) DG_UNSUPPORTED("tile override: the 256 x 256 pipelined tile needs K % 128 == 0");
        if (!grouped_tile_ok(kind, tv, tm, align_m)) DG_UNSUPPORTED("tile override block_m does not fit the M alignment");
        return {256, 256, 4};
    }
    if (tv > 0) {
        const bool ok = tv == 1 ? fp8_1d2d_tile_supported(tm, tn) : (pipe_ok && fp8_1d2d_v2_tile_supported(tm, tn));
        if (!ok) DG_UNSUPPORTED("tile override not compiled");
        if (tv == 2 && tm == 256 && tn == 256 && !tile256_ok)
            DG_UNSUPPORTED("tile override: the 256 x 256 pipelined tile needs K % 128 == 0");
        if (!grouped_tile_ok(kind, tv, tm, align_m))
            DG_UNSUPPORTED("tile override block_m does not fit the M alignment");
        return {tm, tn, tv};
    }
    struct Cand { int variant, bm, bn, per_cu; double eff; };
    // Relative per-CU throughput of each kernel/tile, measured on MI355X at
    // M = 4096 over the DeepSeek-V3 shapes (pipelined 256 x 128 = 1.0).
    static const Cand cands[] = {
        {2, 256, 256, 1, 1.32}, {2, 256, 192, 1, 1.16}, {2, 256, 128, 1, 1.00}, {2, 128, 256, 1, 0.97},
        {2, 128, 128, 1, 0.80},
        {1, 128, 128, 2, 0.80}, {1, 128, 64, 3, 0.55}, {1, 64, 128, 3, 0.55}, {1, 64, 64, 4, 0.45}};
    int cus = 256;
    try { cus = num_sms_now(); } catch (const Error&) {}
    double best = 1e300;
    TileConfig out{64, 64, 1};
    for (const auto& c : cands) {
        if (!grouped_tile_ok(kind, c.variant, c.bm, align_m)) continue;
        if (c.variant == 2 && !pipe_ok) continue;
        // K % 128 != 0: the 256 x 256 pipelined tile has no K-tail schedule.
        if (c.variant == 2 && c.bm == 256 && c.bn == 256 && !tile256_ok) continue;
        const int64_t tiles = ceil_div(m_rows, c.bm) * ceil_div(n, c.bn) * groups;
        const int64_t slots = (int64_t)cus * c.per_cu;
        const double rounds = (double)ceil_div(tiles, slots);
        // One round runs per_cu tiles on every CU at once: its time is the work of
        // per_cu tiles at the candidate's throughput.
        const double cost = rounds * c.bm * c.bn * c.per_cu / c.eff;
        if (cost < best - 1e-9) best = cost, out = {c.bm, c.bn, c.variant};
    }
    return out;
}

// Column split of a dense call whose 256 x 256 tiles leave the last round partly
// empty (4096 x 7168: 448 tiles, 1.75 rounds on 256 CUs, so the second round
// leaves 64 CUs idle): columns [0, n1) run as 256 x 256 tiles in whole rounds
// and [n1, n) as 256 x 192 tiles (4096 x 7168: one round of each, 256 x 256
// over 4096 columns and 256 x 192 over 3072). Every tile computes its outputs
// with the same arithmetic, so the result is bitwise that of one launch.
// Returns n1, or 0 when the per-round cost model (the heuristic's measured
// tile throughputs) gains less than 5% (the second launch has a fixed cost), or
// K is under 4096. A part-empty round is cheaper than the model says: with 192
// of 256 CUs busy the clock rises (2.35 against 2.14-2.18 GHz under full MFMA
// load) and each tile runs ~22% faster, so the split measured -2.5% at
// 4096 x 7168 x 16384 (-4.6% with FP32 C) but +7% at K = 2048 with FP32 C,
// where the second launch's start and its C epilogue outweigh it.
int64_t dense_split_columns(int64_t m_rows, int64_t n, int64_t k, int cus) {
    if (k < 4096) return 0;
    constexpr double t256 = 256.0 * 256 / 1.32, t192 = 256.0 * 192 / 1.16;   // per-round cost of each tile
    const int64_t mb = ceil_div(m_rows, 256);
    auto rounds = [&](int64_t tiles) { return (double)ceil_div(tiles, (int64_t)cus); };
    const double whole = rounds(mb * ceil_div(n, 256)) * t256;
    double best = whole;
    int64_t best_n1 = 0;
    // (on equal cost the largest n1: the most work in the 256 x 256 launch)
    for (int64_t n1 = 256; n1 < n; n1 += 256) {
        const double cost = rounds(mb * (n1 / 256)) * t256 + rounds(mb * ceil_div(n - n1, 192)) * t192;
        if (cost < best - 1e-9 || (best_n1 > 0 && cost <= best + 1e-9)) best = cost, best_n1 = n1;
    }
    return best < 0.95 * whole ? best_n1 : 0;
}

// Row split of an m-grouped contiguous call (m_indices layout) whose 256 x 256
// tiles leave the last round mostly empty (8 experts, 32768 tokens, N = 4096:
// 131 M blocks x 16 = 2096 tiles, 8 full rounds and 48 tiles): rows [0, r1) run
// as 256 x 256 tiles and rows [r1, M) as smaller tiles (there 192 tiles of
// 128 x 128, each a quarter of the work). r1 is a multiple of 256 and segments
// start on the M alignment, so each part is itself an m_indices layout; every
// tile shape computes its outputs with the same arithmetic, so the result is
// bitwise that of one launch. Returns r1 and the second launch's tile, or 0 when
// the per-round cost model gains less than 5% or K is under 4096 (as for the
// column split). With 256-column tiles only (the fused SwiGLU epilogue) the bar
// is 3%: config 3's gate/up launch, 2096 tiles, split into 2048 tiles of
// 256 x 256 and 80 of 128 x 256 for a modelled 3.5% (measured 1097 -> 1083 us).
// In launches of four rounds or more the first part takes the persistent walk
// (is_persistent_route) when it still makes four rounds.
int64_t contiguous_split_rows(int64_t m_rows, int64_t n, int64_t k, int cus, int align_m, TileConfig& hi_tile,
                              bool bn256_only = false) {
    if (k < 4096) return 0;
    struct Part { int bm, bn; double eff; };
    static const Part parts[] = {{256, 128, 1.00}, {128, 256, 0.97}, {128, 128, 0.80}};   // as in choose_tile_1d2d
    constexpr double t256 = 256.0 * 256 / 1.32;
    const int64_t mb = ceil_div(m_rows, 256);
    auto rounds = [&](int64_t tiles) { return (double)ceil_div(tiles, (int64_t)cus); };
    const double whole = rounds(mb * ceil_div(n, 256)) * t256;
    double best = whole;
    int64_t best_r1 = 0;
    // (on equal cost the largest r1: the most work in the 256 x 256 launch)
    for (int64_t mb1 = mb - 1; mb1 >= 1; --mb1)
        for (const auto& p : parts) {
            if (!grouped_tile_ok(kContiguous, 2, p.bm, align_m)) continue;
            if (bn256_only && p.bn != 256) continue;
            const int64_t rows2 = m_rows - mb1 * 256;
            const double cost = rounds(mb1 * ceil_div(n, 256)) * t256 +
                                rounds(ceil_div(rows2, p.bm) * ceil_div(n, p.bn)) * (p.bm * p.bn / p.eff);
            if (cost < best - 1e-9) best = cost, best_r1 = mb1 * 256, hi_tile = TileConfig{p.bm, p.bn, 2};
        }
    return best < (bn256_only ? 0.97 : 0.95) * whole ? best_r1 : 0;
}

// Whether a dense or contiguous call on 256 x 256 tiles runs as persistent
// workgroups (variant 4): BF16 D without C, at least four rounds of tiles on
// the CUs, and for dense calls K <= 2048 (measurements in run_gemm).
bool is_persistent_route(GemmKind kind, const TileConfig& t, const Fp8GemmArgs& args, int64_t m_rows, int64_t n,
                         int64_t k) {
    if (!(kind == kContiguous || (kind == kNormal && k <= 2048))) return false;
    if (t.variant != 2 || t.block_m != 256 || t.block_n != 256 || args.out_f32 || args.c != nullptr) return false;
    return ceil_div(m_rows, 256) * ceil_div(n, 256) >= 4 * (int64_t)args.grid_limit;
}

void record_config(const char* kernel, GemmKind kind, const TileConfig& t, int64_t m, int64_t n, int64_t k,
                   int64_t g) {
    char buf[256];
    std::snprintf(buf, sizeof(buf), "%s v%d kind=%s block_m=%d block_n=%d m=%lld n=%lld k=%lld groups=%lld", kernel,
                  t.variant, kind_name(kind), t.block_m, t.block_n, (long long)m, (long long)n, (long long)k,
                  (long long)g);
    t_last_config = buf;
}

// ---------------------------------------------------------------- dispatch

struct Operands {
    View a, sfa, b, sfb, d;
    const dg_tensor* c;
    const dg_tensor* layout;
};

// FP32 SF recipe of the reference's SM90 "1D2D" kernel:
// A 1 x 128 per token, B 128 x 128 per block, both e4m3.
bool is_1d2d(const Operands& o, const Recipe& r) {
    return o.a.dtype() == DG_E4M3 && o.b.dtype() == DG_E4M3 && o.sfa.dtype() == DG_F32 &&
           o.sfb.dtype() == DG_F32 && r.gran_mn_a == 1 && r.gran_k_a == 128 && r.gran_mn_b == 128 &&
           r.gran_k_b == 128;
}

// FP32 SF recipe of the reference's SM90 "1D1D" kernel (weight gradients):
// A and B both 1 x 128 per row, both e4m3.
bool is_1d1d(const Operands& o, const Recipe& r) {
    return o.a.dtype() == DG_E4M3 && o.b.dtype() == DG_E4M3 && o.sfa.dtype() == DG_F32 &&
           o.sfb.dtype() == DG_F32 && r.gran_mn_a == 1 && r.gran_k_a == 128 && r.gran_mn_b == 1 &&
           r.gran_k_b == 128;
}

// The 1D1D kernels: the 128 x 128 LDS-pipelined one (variant 7, the default) or
// the 128-row streaming one (variant 6, by tile override).
void launch_1d1d(bool k_grouped, const Fp8GemmArgs& args, hipStream_t stream, int64_t m, int64_t n, int64_t k,
                 int64_t groups) {
    const GemmKind kind = k_grouped ? kKGrouped : kNormal;
    if (g_tile_variant.load() == 6) {
        const int waves = g_tile_n.load() / 32;
        record_config("fp8_gemm_1d1d", kind, TileConfig{128, 32 * waves, 6}, m, n, k, groups);
        launch_fp8_gemm_1d1d(k_grouped, waves, args, stream);
        return;
    }
    record_config("fp8_gemm_1d1d", kind, TileConfig{128, 128, 7}, m, n, k, groups);
    launch_fp8_gemm_1d1d_pipe(k_grouped, args, stream);
}

bool is_ue8m0_path(const Operands& o, const Recipe& r) {
    const bool fp4 = is_fp4(o.a) || is_fp4(o.b);
    const bool packed = o.sfa.dtype() == DG_I32 || o.sfb.dtype() == DG_I32;
    const bool gran_ok = (r.gran_k_a == 32 || r.gran_k_a == 128) && (r.gran_k_b == 32 || r.gran_k_b == 128) &&
                         r.gran_mn_a == 1 && (r.gran_mn_b == 1 || (r.gran_mn_b == 128 && o.sfb.dtype() == DG_F32));
    return gran_ok && (fp4 || packed || r.gran_k_a == 32 || r.gran_k_b == 32);
}

// expected_m: the masked layout's per-group row hint (tile choice only), else -1.
// Whether a dense call of at most 64 rows (K % 128 == 0, BF16 D, no C) takes the
// split-K kernel when given a workspace, and its plan. The chunk count fills
// the CUs with workgroups of 64 columns (at least two chunks). Measured on
// MI355X against the kernels the call takes without a workspace (tiny-M /
// streaming; graph replays over 8 rotating buffer sets after a cache flush, us):
//   64 x 2112 x 7168 13.5 against 22.4, 16 x 2112 x 7168 11.0 against 12.9,
//   1 x 2112 x 7168 10.8 against 9.4; 64 x 7168 x 16384 38.1 against 62.2,
//   64 x 16384 x 7168 (two chunks, two rounds) 37.1 against 42.7;
//   64 x 7168 x 2048 13.1 against 12.6, 1 x 4096 x 4096 11.0 against 7.5.
// Its two launches cost ~8 us before any work, so it pays where the single
// launch is slow: more than 8 rows and K >= 6144 (the variant-10 override
// takes it anywhere, with block_n chunks or the heuristic's count).
bool splitk_choice(int64_t m, int64_t n, int64_t k, int cus, SplitKPlan& pl) {
    const int tv = g_tile_variant.load();
    const int64_t tiles = ceil_div(n, kSplitKCols);
    int want = tv == 10 ? g_tile_n.load() : 0;
    if (tv != 10 && tiles <= cus) want = (int)std::max<int64_t>(2, cus / tiles);
    pl = plan_fp8_splitk(m, n, k, cus, want);
    if (tv == 10) return true;
    return m > 8 && k >= 6144 && tiles <= cus && pl.splits >= 2;
}

// ws / ws_bytes: a caller-provided device workspace (dense split-K), or null.
void run_gemm(GemmKind kind, const Operands& o, const Recipe& r, int64_t m, int64_t n, int64_t k, int64_t groups,
              int disable_ue8m0_cast, int zero_padding, hipStream_t stream, int expected_m = -1,
              const dg_epilogue* ep = nullptr, void* ws = nullptr, int64_t ws_bytes = 0) {
    // Epilogue classes and alpha exist on the UE8M0 path only, as in the reference
    // (csrc/apis/gemm.hpp:118-119 for its FP32-scale path); the FP8 stage is a BF16 D
    // without C (csrc/jit_kernels/impls/epilogue_class.hpp:81-84).
    if (ep) {
        DG_CHECK(ep->kind == DG_EPILOGUE_IDENTITY || ep->kind == DG_EPILOGUE_ALPHA || ep->kind == DG_EPILOGUE_FP8_STAGE);
        if (ep->kind == DG_EPILOGUE_FP8_STAGE) DG_CHECK(o.c == nullptr && o.d.dtype() == DG_BF16);
    }
    const int align_m = g_mk_alignment.load();
    const bool grouped_b = kind != kNormal;
    const bool grouped_a = kind == kMasked;

    if (is_1d2d(o, r)) {
        DG_CHECK(ep == nullptr && "alpha and epilogue classes need UE8M0 scales");
        // The kernels move K in 16-byte chunks; a partial chunk would pull in the
        // bytes past K of a padded row.
        if (k % 16 != 0) DG_UNSUPPORTED("K must be a multiple of 16 on the FP32-scale FP8 path");
        check_vector_alignment(o.a, "a");
        check_vector_alignment(o.b, "b");
        check_vector_alignment(o.d, "d");
        if (o.c) check_vector_alignment(view(o.c, "c"), "c");
        Fp8GemmArgs args{};
        args.a = static_cast<const uint8_t*>(o.a.data());
        args.b = static_cast<const uint8_t*>(o.b.data());
        args.sfa = static_cast<const float*>(o.sfa.data());
        args.sfb = static_cast<const float*>(o.sfb.data());
        args.d = const_cast<void*>(o.d.data());
        args.c = o.c ? o.c->data : nullptr;
        args.layout = o.layout ? static_cast<const int32_t*>(o.layout->data) : nullptr;
        args.m = (int32_t)m, args.n = (int32_t)n, args.k = (int32_t)k;
        args.num_groups = (int32_t)groups;
        args.out_f32 = o.d.dtype() == DG_F32;
        args.align_m = align_m;
        args.zero_padding = zero_padding;
        args.lda = o.a.stride(-2), args.ldb = o.b.stride(-2), args.ldd = o.d.stride(-2);
        args.ldc = o.c ? o.c->strides[o.c->ndim - 2] : 0;
        args.a_gs = grouped_a ? o.a.stride(0) : 0;
        args.b_gs = grouped_b ? o.b.stride(0) : 0;
        args.d_gs = grouped_a ? o.d.stride(0) : 0;
        args.c_gs = 0;
        args.sfa_sm = o.sfa.stride(-2), args.sfa_sk = o.sfa.stride(-1);
        args.sfa_gs = grouped_a ? o.sfa.stride(0) : 0;
        args.sfb_sn = o.sfb.stride(-2), args.sfb_sk = o.sfb.stride(-1);
        args.sfb_gs = grouped_b ? o.sfb.stride(0) : 0;
        args.grid_limit = 256;
        try { args.grid_limit = num_sms_now(); } catch (const Error&) {}
        const int64_t m_rows = m;
        const int tv = g_tile_variant.load();
        // Dense calls of at most 64 rows with a workspace: K split over workgroups
        // whenever that gives at least two chunks (variant 10 forces it, block_n
        // = chunks or 0 for the heuristic's count).
        if (kind == kNormal && (tv == 0 || tv == 10) && fp8_splitk_supported(args)) {
            SplitKPlan pl{};
            const bool chosen = splitk_choice(m_rows, n, k, args.grid_limit, pl);
            const bool fits = ws != nullptr && ws_bytes >= pl.workspace_bytes;
            if (tv == 10 && !fits)
                DG_UNSUPPORTED("tile override: the split-K kernel needs a workspace of "
                               "dg_fp8_gemm_nt_workspace_size bytes (dg_fp8_fp4_gemm_nt_ws)");
            if (fits && chosen) {
                record_config("fp8_gemm_1d2d", kind, TileConfig{pl.rows, kSplitKCols, 10}, m, n, k, groups);
                t_last_config += " splits=" + std::to_string(pl.splits) + "x" + std::to_string(pl.kper);
                launch_fp8_gemm_splitk(args, pl, static_cast<float*>(ws), stream);
                return;
            }
        } else if (tv == 10) {
            DG_UNSUPPORTED("tile override: the split-K kernel runs dense calls of at most 64 rows with K % 128 == 0, "
                           "BF16 D and no C");
        }
        TileConfig t;
        // Dense calls of at most kDenseStreamRows rows are weight-stream bound: they
        // run on the streaming kernel as one group (layout null), which loads only
        // the rows that exist (16 x 16 x 128 MFMAs up to 16 rows).
        const bool stream_ok = fp8_masked_stream_supported(args) &&
                               (kind == kMasked || (kind == kNormal && m_rows <= kMaskedStreamRows));
        // Dense calls of at most 64 rows (128-256 with K <= 8192): K split over the
        // waves of a workgroup, so the launch has N / 16 or N / 32 workgroups per
        // row group instead of the streaming kernel's N / 128.
        auto tinym_fits = [&] {   // above 128 rows: a small tiled launch, and one round of tiny-M workgroups
            if (m_rows <= 128) return true;
            if (ceil_div(m_rows, 128) * ceil_div(n, 128) >= kTinyMWideMaxTiles) return false;
            const TileConfig c = choose_tinym(m_rows, n, k, args.grid_limit);
            return ceil_div(n, c.block_n) * ceil_div(m_rows, c.block_m) <= args.grid_limit;
        };
        const bool tinym_ok = kind == kNormal && fp8_tinym_supported(args) &&
                              (tv == 8 || tv == 9 || m_rows <= kTinyMRows ||
                               (k <= kTinyMWideMaxK && tinym_fits()));
        if (tv == 8 || tv == 9) {   // forced: the tiny-M kernel
            if (!tinym_ok)
                DG_UNSUPPORTED("tile override: the tiny-M kernel runs dense calls of at most 256 rows with "
                               "K % 128 == 0, K <= 32768, BF16 D and no C");
            t = {g_tile_m.load(), g_tile_n.load(), tv};   // rows per workgroup, columns per workgroup
        } else if (tv == 0 && tinym_ok &&
                   (!stream_ok || (n + 32 * fp8_masked_stream_waves(n, 1, args.grid_limit) - 1) /
                                          (32 * fp8_masked_stream_waves(n, 1, args.grid_limit)) <
                                      kTinyMStreamGrid)) {
            t = choose_tinym(m_rows, n, k, args.grid_limit);
        } else if (tv == 5) {   // forced: the weight-streaming kernel
            if (!stream_ok)
                DG_UNSUPPORTED("tile override: the weight-streaming kernel runs the masked layout, or dense calls of at "
                               "most 160 rows, with K % 128 == 0, BF16 D and no C");
            t = {g_tile_m.load(), g_tile_n.load(), 5};
        } else if (tv == 0 && stream_ok &&
                   (kind == kNormal ? m_rows <= kDenseStreamRows : expected_m <= kMaskedStreamRows)) {
            // decode-sized groups: the weight-streaming kernel (one pass per group
            // when masked_m <= 160; larger groups take more passes)
            // 16 x 16 x 128 passes for groups of at most 16 rows (5-10% faster there)
            const int rows_hint = kind == kNormal ? (int)m_rows : expected_m;
            t = {rows_hint <= kStream16Rows ? kStream16Rows : kMaskedStreamRows,
                 32 * fp8_masked_stream_waves(n, groups, args.grid_limit), 5};
        } else {
            t = choose_tile_1d2d(kind, m_rows, n, k, kind == kMasked ? groups : 1, align_m);
            // Masked groups far below max_m: one workgroup per tile launches every
            // m-block of max_m, and each empty workgroup still holds a CU's LDS while
            // it starts and exits; the persistent walk visits only the m-blocks below
            // each group's masked_m. Taken when expected_m leaves at least half of
            // the m-blocks empty (reference test shapes, max_m 4096: 32 groups at
            // expected_m 192 2.5-2.7x faster, 6 groups at 1024 4-10%; with most
            // m-blocks active it is 6-13% slower).
            if (kind == kMasked && tv == 0 && t.variant == 2 && t.block_m == 256 && t.block_n == 256 &&
                ceil_div(m_rows, 256) >= 2 * ceil_div(std::max(expected_m, 1), 256))
                t.variant = 4;
            // Many rounds of tiles (BF16 D, no C): the per-tile launch pays each
            // workgroup's start and first-stage wait once per tile, the persistent
            // walk once per CU. Measured per launch (µs, per tile -> persistent):
            // 4096 x 24576 x 1536 (6 rounds) 170-173 -> 168-172 (K-major SFA 195 ->
            // 189); contiguous 33408 x 7168 x 2048 (14 rounds) 522-524 -> 509-510,
            // 33408 x 4096 x 7168 (8 rounds, per tile with the row split) 958-961 ->
            // 942-943. Dense calls with longer K are even (within 1-2% at 4-8
            // rounds) and keep the per-tile launch and its column split; at 1-3.5
            // rounds it loses (4096 x 7168 x 2048 +5%), and with FP32 C it is even.
            if (tv == 0 && is_persistent_route(kind, t, args, m_rows, n, k)) t.variant = 4;
        }
        if (!grouped_tile_ok(kind, t.variant, t.block_m, align_m))
            DG_UNSUPPORTED("M alignment for contiguous layout must be a multiple of 64");
        record_config("fp8_gemm_1d2d", kind, t, m, n, k, groups);
        if (kind == kNormal && tv == 0 && t.variant == 2 && t.block_m == 256 && t.block_n == 256) {
            const int64_t n1 = dense_split_columns(m_rows, n, k, args.grid_limit);
            if (n1 > 0) {
                t_last_config += " split_n=" + std::to_string(n1) + ":256x192";
                Fp8GemmArgs lo = args;
                lo.n = (int32_t)n1;
                launch_fp8_gemm_1d2d_v2(kind, t, lo, stream);
                // columns [n1, n): B rows, SFB rows (n1 is a multiple of 128), D and C columns
                Fp8GemmArgs hi = args;
                hi.n = (int32_t)(n - n1);
                hi.b = args.b + n1 * args.ldb;
                hi.sfb = args.sfb + (n1 / 128) * args.sfb_sn;
                const int64_t elem = args.out_f32 ? 4 : 2;
                hi.d = static_cast<uint8_t*>(args.d) + n1 * elem;
                if (args.c) hi.c = static_cast<const uint8_t*>(args.c) + n1 * elem;
                launch_fp8_gemm_1d2d_v2(kind, TileConfig{256, 192, 2}, hi, stream);
                return;
            }
        }
        // (persistent launches too: their last round is as uneven; the first rows
        // stay persistent when they still make four rounds. Measured, interleaved
        // bench runs: 33408 x 4096 x 7168 970-981 -> 954-958 us, the first 32768
        // rows 880-890 us and the 640-row tail on 128 x 128 tiles 43 us.)
        if (kind == kContiguous && tv == 0 && (t.variant == 2 || t.variant == 4) && t.block_m == 256 &&
            t.block_n == 256) {
            TileConfig ht{};
            const int64_t r1 = contiguous_split_rows(m_rows, n, k, args.grid_limit, align_m, ht);
            if (r1 > 0) {
                t_last_config += " split_m=" + std::to_string(r1) + ":" + std::to_string(ht.block_m) + "x" +
                                 std::to_string(ht.block_n);
                Fp8GemmArgs lo = args;
                lo.m = (int32_t)r1;
                TileConfig lt = t;
                if (lt.variant == 4 && !is_persistent_route(kind, TileConfig{256, 256, 2}, args, r1, n, k))
                    lt.variant = 2;
                launch_fp8_gemm_1d2d_v2(kind, lt, lo, stream);
                // rows [r1, m): A rows, SFA rows (K- or MN-major: sfa_sm is the row
                // stride), m_indices entries and D rows
                Fp8GemmArgs hi = args;
                hi.m = (int32_t)(m_rows - r1);
                hi.a = args.a + r1 * args.lda;
                hi.sfa = args.sfa + r1 * args.sfa_sm;
                hi.layout = args.layout + r1;
                const int64_t elem = args.out_f32 ? 4 : 2;
                hi.d = static_cast<uint8_t*>(args.d) + r1 * args.ldd * elem;
                if (args.c) hi.c = static_cast<const uint8_t*>(args.c) + r1 * args.ldc * elem;
                launch_fp8_gemm_1d2d_v2(kind, ht, hi, stream);
                return;
            }
        }
        if (t.variant == 8 || t.variant == 9)
            launch_fp8_gemm_tinym(args, t.variant == 8 ? 8 : 4, t.block_n, t.block_m, stream);
        else if (t.variant == 5)
            launch_fp8_gemm_masked_stream(args, t.block_n / 32, t.block_m == kStream16Rows, stream);
        else if (t.variant >= 2)
            launch_fp8_gemm_1d2d_v2(kind, t, args, stream);
        else
            launch_fp8_gemm_1d2d(kind, t, args, stream);
        return;
    }

    if (is_ue8m0_path(o, r)) {
        // csrc/apis/layout.hpp:46-47: FP32 SFs are cast to UE8M0 on this path.
        if (o.sfa.dtype() == DG_F32 || o.sfb.dtype() == DG_F32) DG_CHECK(!disable_ue8m0_cast);
        if (o.sfa.dtype() == DG_I32) check_packed_sf_strides(o.sfa, m);
        if (o.sfb.dtype() == DG_I32) check_packed_sf_strides(o.sfb, n);
        check_vector_alignment(o.a, "a");
        check_vector_alignment(o.b, "b");
        check_vector_alignment(o.d, "d");
        if (o.c) check_vector_alignment(view(o.c, "c"), "c");
        Fp8Fp4GemmArgs args{};
        args.a = static_cast<const uint8_t*>(o.a.data());
        args.b = static_cast<const uint8_t*>(o.b.data());
        args.sfa = o.sfa.data();
        args.sfb = o.sfb.data();
        args.d = const_cast<void*>(o.d.data());
        args.c = o.c ? o.c->data : nullptr;
        args.layout = o.layout ? static_cast<const int32_t*>(o.layout->data) : nullptr;
        args.m = (int32_t)m, args.n = (int32_t)n, args.k = (int32_t)k;
        args.num_groups = (int32_t)groups;
        args.out_f32 = o.d.dtype() == DG_F32;
        args.align_m = align_m;
        args.zero_padding = zero_padding;
        args.a_fp4 = is_fp4(o.a), args.b_fp4 = is_fp4(o.b);
        args.sfa_packed = o.sfa.dtype() == DG_I32, args.sfb_packed = o.sfb.dtype() == DG_I32;
        args.gran_k_a = r.gran_k_a, args.gran_k_b = r.gran_k_b;
        args.lda = o.a.stride(-2), args.ldb = o.b.stride(-2), args.ldd = o.d.stride(-2);
        args.ldc = o.c ? o.c->strides[o.c->ndim - 2] : 0;
        args.a_gs = grouped_a ? o.a.stride(0) : 0;
        args.b_gs = grouped_b ? o.b.stride(0) : 0;
        args.d_gs = grouped_a ? o.d.stride(0) : 0;
        args.c_gs = 0;
        // gran_mn_b == 128 with FP32 SFB: the row index is n / 128 (the reference
        // broadcasts rows before packing, csrc/apis/layout.hpp:48-49).
        args.sfa_sm = o.sfa.stride(-2), args.sfa_sk = o.sfa.stride(-1);
        args.sfa_gs = grouped_a ? o.sfa.stride(0) : 0;
        args.sfb_sn = o.sfb.stride(-2), args.sfb_sk = o.sfb.stride(-1);
        args.sfb_gs = grouped_b ? o.sfb.stride(0) : 0;
        args.sfb_row_shift = r.gran_mn_b == 128 ? 7 : 0;
        args.alpha = (ep && ep->kind == DG_EPILOGUE_ALPHA) ? ep->alpha : 1.0f;
        // The 256 x 256 pipelined kernel takes packed scale words and K % 128 == 0;
        // everything else runs on the 128 x 128 kernel. A tile override selects
        // the kernel by its variant (1: 128 x 128, 2: pipelined).
        const int tv = g_tile_variant.load();
        const bool pipe_ok = fp8_fp4_pipe_supported(args) && grouped_tile_ok(kind, 2, 256, align_m);
        if (tv == 2 && !pipe_ok) DG_UNSUPPORTED("tile override: the pipelined UE8M0 kernel does not take these inputs");
        if (pipe_ok && tv != 1) {
            const TileConfig t{256, 256, 2};
            record_config("fp8_fp4_gemm_ue8m0_pipe", kind, t, m, n, k, groups);
            launch_fp8_fp4_gemm_pipe(kind, args, stream);
            return;
        }
        const TileConfig t{128, 128, 1};
        if ((kind == kContiguous || kind == kPsum) && align_m % t.block_m != 0)
            DG_UNSUPPORTED("M alignment for contiguous layout must be a multiple of 128 on the UE8M0 path");
        record_config("fp8_fp4_gemm_ue8m0", kind, t, m, n, k, groups);
        launch_fp8_fp4_gemm(kind, t, args, stream);
        return;
    }

    if (is_1d1d(o, r)) {
        DG_CHECK(ep == nullptr && "alpha and epilogue classes need UE8M0 scales");
        // csrc/jit_kernels/impls/sm90_fp8_gemm_1d1d.hpp:91: FP32 D, accumulating into C
        DG_CHECK(o.c != nullptr && o.d.dtype() == DG_F32);
        if (kind != kNormal) DG_UNSUPPORTED("the 1D1D recipe runs the dense and K-grouped GEMMs only");
        if (k % 128 != 0) DG_UNSUPPORTED("the 1D1D recipe needs K to be a multiple of 128 here");
        check_vector_alignment(o.a, "a");
        check_vector_alignment(o.b, "b");
        check_vector_alignment(o.d, "d");
        check_vector_alignment(view(o.c, "c"), "c");
        const View cv = view(o.c, "c");
        Fp8GemmArgs args{};
        args.a = static_cast<const uint8_t*>(o.a.data());
        args.b = static_cast<const uint8_t*>(o.b.data());
        args.sfa = static_cast<const float*>(o.sfa.data());
        args.sfb = static_cast<const float*>(o.sfb.data());
        args.d = const_cast<void*>(o.d.data());
        args.c = cv.data();
        args.m = (int32_t)m, args.n = (int32_t)n, args.k = (int32_t)k;
        args.num_groups = 1;
        args.out_f32 = 1;
        args.lda = o.a.stride(-2), args.ldb = o.b.stride(-2), args.ldd = o.d.stride(-2), args.ldc = cv.stride(-2);
        args.sfa_sm = o.sfa.stride(-2), args.sfa_sk = o.sfa.stride(-1);
        args.sfb_sn = o.sfb.stride(-2), args.sfb_sk = o.sfb.stride(-1);
        launch_1d1d(false, args, stream, m, n, k, 1);
        return;
    }
    DG_UNSUPPORTED("Unsupported architecture or scaling factor types");
}

// ---------------------------------------------------------------- the three GEMMs

void gemm_nt_impl(const dg_tensor* a_, const dg_tensor* sfa_, const dg_tensor* b_, const dg_tensor* sfb_,
                  const dg_tensor* d_, const dg_tensor* c, const dg_recipe* recipe, int disable_ue8m0_cast,
                  const dg_epilogue* ep, hipStream_t stream, const dg_tensor* ws_ = nullptr) {
    const View a = view(a_, "a"), sfa = view(sfa_, "sfa"), b = view(b_, "b"), sfb = view(sfb_, "sfb"),
               d = view(d_, "d");
    // Shape must be [M, K] @ [N, K].T; the gfx950 kernels need K-major operands
    // (as the reference's SM90 path does, csrc/apis/gemm.hpp:93-97).
    DG_CHECK(is_k_major(a));
    DG_CHECK(is_k_major(b));
    check_major_type_cd(d);
    const auto [m, k] = check_ab(a);
    const auto [n, k_] = check_ab(b);
    check_shape(d, 2);
    const int64_t m_ = d.size(0), n_ = d.size(1);
    DG_CHECK(m == m_ && n == n_ && k == k_);
    DG_CHECK(d.dtype() == DG_BF16 || d.dtype() == DG_F32);
    if (early_return(m, n, k, d, c, stream)) return;
    const Recipe r = resolve_recipe(recipe, sfa, sfb);
    check_sf_layout(sfa, m, k, r.gran_mn_a, r.gran_k_a, -1);
    check_sf_layout(sfb, n, k, r.gran_mn_b, r.gran_k_b, -1);
    void* ws = nullptr;
    int64_t ws_bytes = 0;
    if (ws_) {
        const View w = view(ws_, "workspace");
        DG_CHECK(w.on_device() && w.dim() == 1 && (w.size(0) <= 1 || w.stride(0) == 1));
        ws = const_cast<void*>(w.data());
        ws_bytes = w.size(0) * elem_size(w.dtype());
        DG_CHECK(reinterpret_cast<uintptr_t>(ws) % 16 == 0);
    }
    run_gemm(kNormal, Operands{a, sfa, b, sfb, d, c, nullptr}, r, m, n, k, 1, disable_ue8m0_cast, 0, stream, -1, ep,
             ws, ws_bytes);
}

// Bytes of the workspace dg_fp8_fp4_gemm_nt_ws uses for an m x n x k call on the
// FP32-scale path with a BF16 D and no C (0: the call takes no workspace).
int64_t dense_workspace_bytes(int64_t m, int64_t n, int64_t k) {
    if (m <= 0 || n <= 0 || k <= 0 || m > kSplitKMaxRows || k % 128 != 0) return 0;
    int cus = 256;
    try { cus = num_sms_now(); } catch (const Error&) {}
    const int tv = g_tile_variant.load();
    if (tv != 0 && tv != 10) return 0;
    SplitKPlan pl{};
    return splitk_choice(m, n, k, cus, pl) ? pl.workspace_bytes : 0;
}

void contiguous_impl(const dg_tensor* a_, const dg_tensor* sfa_, const dg_tensor* b_, const dg_tensor* sfb_,
                     const dg_tensor* d_, const dg_tensor* layout_, const dg_recipe* recipe, int disable_ue8m0_cast,
                     int use_psum_layout, int ensure_zero_padding, int expected_m_for_psum_layout,
                     const dg_epilogue* ep, hipStream_t stream) {
    const View a = view(a_, "a"), sfa = view(sfa_, "sfa"), b = view(b_, "b"), sfb = view(sfb_, "sfb"),
               d = view(d_, "d"), gl = view(layout_, "grouped_layout");
    // Shape must be [M, K] @ [G, N, K].mT (csrc/apis/gemm.hpp:195-218)
    DG_CHECK(is_k_major(a));
    DG_CHECK(is_k_major(b));
    DG_CHECK(gl.dim() == 1 && (gl.size(0) <= 1 || gl.stride(0) == 1));
    const auto [m, k] = check_ab(a);
    int64_t groups, n, k_;
    check_grouped_ab(b, groups, n, k_);
    check_shape(d, 2);
    const int64_t m_ = d.size(0), n_ = d.size(1);
    DG_CHECK(m == m_ && n == n_ && k == k_);
    DG_CHECK(n > 0 && k > 0 && groups > 0);
    DG_CHECK(d.dtype() == DG_BF16);
    DG_CHECK(gl.dtype() == DG_I32);
    check_shape(gl, 1);
    if (use_psum_layout) {
        DG_CHECK(gl.size(0) == groups);
    } else {
        DG_CHECK(gl.size(0) == m);
        DG_CHECK(expected_m_for_psum_layout < 0);
    }
    check_major_type_cd(d);
    if (m == 0) return;
    const Recipe r = resolve_recipe(recipe, sfa, sfb);
    check_sf_layout(sfa, m, k, r.gran_mn_a, r.gran_k_a, -1);
    check_sf_layout(sfb, n, k, r.gran_mn_b, r.gran_k_b, groups);
    run_gemm(use_psum_layout ? kPsum : kContiguous, Operands{a, sfa, b, sfb, d, nullptr, layout_}, r, m, n, k, groups,
             disable_ue8m0_cast, use_psum_layout && ensure_zero_padding, stream, -1, ep);
}

void masked_impl(const dg_tensor* a_, const dg_tensor* sfa_, const dg_tensor* b_, const dg_tensor* sfb_,
                 const dg_tensor* d_, const dg_tensor* masked_m_, int expected_m, const dg_recipe* recipe,
                 int disable_ue8m0_cast, const dg_epilogue* ep, hipStream_t stream) {
    const View a = view(a_, "a"), sfa = view(sfa_, "sfa"), b = view(b_, "b"), sfb = view(sfb_, "sfb"),
               d = view(d_, "d"), mm = view(masked_m_, "masked_m");
    // Shape must be [G, M, K] @ [G, N, K].mT (csrc/apis/gemm.hpp:282-297)
    DG_CHECK(is_k_major(a) && is_k_major(b));
    DG_CHECK(mm.dim() == 1 && (mm.size(0) <= 1 || mm.stride(0) == 1));
    int64_t g, m, k, g_, n, k_;
    check_grouped_ab(a, g, m, k);
    check_grouped_ab(b, g_, n, k_);
    check_shape(d, 3);
    const int64_t g__ = d.size(0), m_ = d.size(1), n_ = d.size(2);
    const int64_t g___ = mm.size(0);
    DG_CHECK(g == g_ && g == g__ && g == g___);
    DG_CHECK(m == m_ && n == n_ && k == k_);
    DG_CHECK(expected_m > 0 && m > 0 && n > 0 && k > 0 && g > 0);
    DG_CHECK(d.dtype() == DG_BF16);
    DG_CHECK(mm.dtype() == DG_I32);
    DG_CHECK(mm.on_device());
    check_major_type_cd(d);
    const Recipe r = resolve_recipe(recipe, sfa, sfb);
    check_sf_layout(sfa, m, k, r.gran_mn_a, r.gran_k_a, g);
    check_sf_layout(sfb, n, k, r.gran_mn_b, r.gran_k_b, g);
    run_gemm(kMasked, Operands{a, sfa, b, sfb, d, nullptr, masked_m_}, r, m, n, k, g, disable_ue8m0_cast, 0, stream,
             expected_m, ep);
}

// ---------------------------------------------------------------- fused L1 (SwiGLU epilogue)

// The L1 grouped GEMM of an MoE layer with the SwiGLU x routing weight -> FP8
// step in its epilogue: no BF16 intermediate goes through HBM. The reference
// fuses the same step into its SM100 Mega-MoE kernel's L1 epilogue
// (deep_gemm/include/deep_gemm/impls/sm100_fp8_fp4_mega_moe.cuh:1066-1130) and
// runs it unfused between two grouped GEMMs on SM90 (tests/test_mega_moe.py:296-330).
// Checks: the m-grouped GEMM's (contiguous_impl / masked_impl) for A, B and the
// layout; B has N = 2I rows with gate and up interleaved in 128-row blocks;
// q e4m3 [.., rows, I] with unit stride along I and 8-byte aligned rows; sf f32
// [.., rows, I/128] in any strides; row weights f32 [.., rows] contiguous or null.
bool contiguous_view(const View& t);

void swiglu_l1_impl(GemmKind kind, const dg_tensor* a_, const dg_tensor* sfa_, const dg_tensor* b_,
                    const dg_tensor* sfb_, const dg_tensor* layout_, int expected_m, const dg_tensor* w_, float clamp,
                    const dg_tensor* q_, const dg_tensor* sfq_, int ensure_zero_padding, hipStream_t stream) {
    const View a = view(a_, "a"), sfa = view(sfa_, "sfa"), b = view(b_, "b"), sfb = view(sfb_, "sfb"),
               gl = view(layout_, kind == kMasked ? "masked_m" : "grouped_layout"), q = view(q_, "q"),
               sfq = view(sfq_, "sf");
    const bool masked = kind == kMasked;
    DG_CHECK(is_k_major(a) && is_k_major(b));
    DG_CHECK(a.dtype() == DG_E4M3 && b.dtype() == DG_E4M3);
    DG_CHECK(gl.dim() == 1 && (gl.size(0) <= 1 || gl.stride(0) == 1));
    DG_CHECK(gl.dtype() == DG_I32 && gl.on_device());
    int64_t g = 1, m, k, n, k_;
    if (masked) {
        check_grouped_ab(a, g, m, k);
        int64_t g_;
        check_grouped_ab(b, g_, n, k_);
        DG_CHECK(g == g_ && gl.size(0) == g);
        DG_CHECK(expected_m > 0);
    } else {
        std::tie(m, k) = check_ab(a);
        check_grouped_ab(b, g, n, k_);
        DG_CHECK(gl.size(0) == (kind == kPsum ? g : m));
    }
    DG_CHECK(k == k_ && n > 0 && k > 0 && g > 0 && m >= 0);
    if (n % 256 != 0) DG_UNSUPPORTED("fused SwiGLU: N = 2 * intermediate must be a multiple of 256");
    const int64_t inter = n / 2;
    // q and sf: [rows, I] / [G, max_m, I]
    check_shape(q, masked ? 3 : 2);
    DG_CHECK(q.dtype() == DG_E4M3 && q.stride(-1) == 1 && q.size(-1) == inter && q.size(-2) == m);
    if (masked) DG_CHECK(q.size(0) == g);
    const int64_t ldq = q.stride(-2), q_gs = masked ? q.stride(0) : 0;
    DG_CHECK(reinterpret_cast<uintptr_t>(q.data()) % 8 == 0 && (m <= 1 || ldq % 8 == 0) && q_gs % 8 == 0);
    check_shape(sfq, masked ? 3 : 2);
    DG_CHECK(sfq.dtype() == DG_F32 && sfq.size(-1) == inter / 128 && sfq.size(-2) == m);
    if (masked) DG_CHECK(sfq.size(0) == g);
    const float* w = nullptr;
    int64_t w_gs = 0;
    if (w_) {
        const View wv = view(w_, "row_weights");
        DG_CHECK(wv.dtype() == DG_F32 && wv.on_device() && contiguous_view(wv));
        if (masked) {
            DG_CHECK((wv.dim() == 2 && wv.size(0) == g && wv.size(1) == m) || (wv.dim() == 1 && wv.size(0) == g * m));
            w_gs = m;
        } else {
            DG_CHECK(wv.dim() == 1 && wv.size(0) == m);
        }
        w = static_cast<const float*>(wv.data());
    }
    if (m == 0) return;
    const Recipe r = resolve_recipe(nullptr, sfa, sfb);
    const Operands o{a, sfa, b, sfb, q, nullptr, layout_};
    if (!is_1d2d(o, r)) DG_UNSUPPORTED("fused SwiGLU: FP32 scales of the (1, 128, 128) recipe");
    check_sf_layout(sfa, m, k, 1, 128, masked ? g : -1);
    check_sf_layout(sfb, n, k, 128, 128, g);
    if (k % 16 != 0) DG_UNSUPPORTED("K must be a multiple of 16 on the FP32-scale FP8 path");
    check_vector_alignment(a, "a");
    check_vector_alignment(b, "b");
    const int align_m = g_mk_alignment.load();
    Fp8GemmArgs args{};
    args.a = static_cast<const uint8_t*>(a.data());
    args.b = static_cast<const uint8_t*>(b.data());
    args.sfa = static_cast<const float*>(sfa.data());
    args.sfb = static_cast<const float*>(sfb.data());
    args.layout = static_cast<const int32_t*>(gl.data());
    args.m = (int32_t)m, args.n = (int32_t)n, args.k = (int32_t)k;
    args.num_groups = (int32_t)g;
    args.align_m = align_m;
    args.zero_padding = kind == kPsum && ensure_zero_padding;
    args.lda = a.stride(-2), args.ldb = b.stride(-2);
    args.a_gs = masked ? a.stride(0) : 0;
    args.b_gs = b.stride(0);
    args.sfa_sm = sfa.stride(-2), args.sfa_sk = sfa.stride(-1);
    args.sfa_gs = masked ? sfa.stride(0) : 0;
    args.sfb_sn = sfb.stride(-2), args.sfb_sk = sfb.stride(-1), args.sfb_gs = sfb.stride(0);
    args.grid_limit = 256;
    try { args.grid_limit = num_sms_now(); } catch (const Error&) {}
    args.sw_q = static_cast<uint8_t*>(const_cast<void*>(q.data()));
    args.sw_ldq = ldq, args.sw_q_gs = q_gs;
    args.sw_sf = static_cast<float*>(const_cast<void*>(sfq.data()));
    args.sw_sf_sm = sfq.stride(-2), args.sw_sf_sk = sfq.stride(-1), args.sw_sf_gs = masked ? sfq.stride(0) : 0;
    args.sw_w = w, args.sw_w_gs = w_gs;
    args.sw_clamp = clamp > 0.f ? clamp : 0.f;

    // Tile: the 256-column tiles of the pipelined kernel (256 rows when K % 128 == 0
    // and the layout allows, else 128; for masked groups far below max_m the
    // persistent 256 x 256 walk), or for masked decode groups the weight-streaming
    // kernel with 8 waves (256 columns).
    const int tv = g_tile_variant.load(), tm = g_tile_m.load(), tn = g_tile_n.load();
    const bool ktail = k % 128 != 0;
    if (ceil_div(k, 128) > 1024) DG_UNSUPPORTED("fused SwiGLU: K up to 131072");
    TileConfig t{256, 256, 2};
    if (kind == kPsum && (align_m % 256 != 0 || ktail)) t.block_m = 128;
    if (kind == kContiguous && ktail) t.block_m = 128;
    if (masked && ktail) t.block_m = 128;
    const bool stream_ok = masked && fp8_masked_stream_supported(args);
    if (tv == 5) {
        if (!stream_ok || tn != 256)
            DG_UNSUPPORTED("tile override: the fused SwiGLU epilogue takes the streaming kernel with 8 waves, "
                           "masked layout, K % 128 == 0");
        t = {kMaskedStreamRows, 256, 5};
    } else if (tv == 2) {
        if (tn != 256 || (tm != 256 && tm != 128) || (tm == 256 && ktail))
            DG_UNSUPPORTED("tile override: the fused SwiGLU epilogue takes 256 x 256 (K % 128 == 0) or 128 x 256 tiles");
        t = {tm, 256, 2};
    } else if (tv != 0) {
        DG_UNSUPPORTED("tile override: the fused SwiGLU epilogue runs variants 2 and 5");
    } else if (stream_ok && expected_m <= kMaskedStreamRows) {
        t = {kMaskedStreamRows, 256, 5};
    } else if (masked && t.block_m == 256 && ceil_div(m, 256) >= 2 * ceil_div(std::max(expected_m, 1), 256)) {
        t.variant = 4;   // the persistent group walk, as for the plain masked launch (run_gemm)
    } else if (kind == kContiguous && is_persistent_route(kind, t, args, m, n, k)) {
        t.variant = 4;   // many rounds of tiles: persistent, as the plain contiguous launch (run_gemm)
    }
    if (t.variant == 2 && !grouped_tile_ok(kind, 2, t.block_m, align_m))
        DG_UNSUPPORTED("M alignment for contiguous layout must be a multiple of 128 for the fused SwiGLU epilogue");
    record_config("fp8_gemm_1d2d_swiglu", kind, t, m, n, k, g);
    if (t.variant == 5) {
        launch_fp8_gemm_masked_stream(args, 8, false, stream);
        return;
    }
    if (kind == kContiguous && tv == 0 && (t.variant == 2 || t.variant == 4) && t.block_m == 256) {
        // the row split of the plain contiguous launch, with a 256-column second tile
        TileConfig ht{};
        const int64_t r1 = contiguous_split_rows(m, n, k, args.grid_limit, align_m, ht, true);
        if (r1 > 0) {
            t_last_config += " split_m=" + std::to_string(r1) + ":" + std::to_string(ht.block_m) + "x" +
                             std::to_string(ht.block_n);
            Fp8GemmArgs lo = args;
            lo.m = (int32_t)r1;
            TileConfig lt = t;
            if (lt.variant == 4 && !is_persistent_route(kind, TileConfig{256, 256, 2}, args, r1, n, k))
                lt.variant = 2;
            launch_fp8_gemm_1d2d_v2(kind, lt, lo, stream);
            Fp8GemmArgs hi = args;
            hi.m = (int32_t)(m - r1);
            hi.a = args.a + r1 * args.lda;
            hi.sfa = args.sfa + r1 * args.sfa_sm;
            hi.layout = args.layout + r1;
            hi.sw_q = args.sw_q + r1 * args.sw_ldq;
            hi.sw_sf = args.sw_sf + r1 * args.sw_sf_sm;
            if (args.sw_w) hi.sw_w = args.sw_w + r1;
            launch_fp8_gemm_1d2d_v2(kind, ht, hi, stream);
            return;
        }
    }
    launch_fp8_gemm_1d2d_v2(kind, t, args, stream);
}

// ---------------------------------------------------------------- SF layouts

// csrc/apis/layout.hpp:11-58 (planning half).
int plan_sf(const dg_tensor* sf_, int32_t mn, int32_t k, const int32_t* recipe3, const int32_t* recipe2,
            int32_t num_groups, int32_t is_sfa, int32_t disable_ue8m0_cast) {
    const View sf = view(sf_, "sf");
    int gran_mn, gran_k;
    if (recipe3) {
        DG_CHECK(is_sfa == 0 || is_sfa == 1);
        gran_mn = is_sfa ? recipe3[0] : recipe3[1];
        gran_k = recipe3[2];
    } else if (recipe2) {
        DG_CHECK(is_sfa < 0);
        gran_mn = recipe2[0];
        gran_k = recipe2[1];
    } else {
        DG_UNSUPPORTED("Invalid recipe");
    }
    check_sf_layout(sf, mn, k, gran_mn, gran_k, num_groups);
    // (FP32, 1, 128): MN-major TMA-aligned copy, as the reference's SM90 path.
    if (sf.dtype() == DG_F32 && gran_mn == 1 && gran_k == 128) return 1;
    // (FP32, 128, 128): used as is (reference checks contiguity, layout.hpp:132-138).
    if (sf.dtype() == DG_F32 && gran_mn == 128 && gran_k == 128) {
        if (num_groups >= 0) DG_CHECK(sf.stride(-3) == sf.size(-2) * sf.size(-1));
        DG_CHECK((sf.stride(-1) == 1 && sf.stride(-2) == sf.size(-1)) ||
                 (sf.stride(-1) == sf.size(-2) && sf.stride(-2) == 1));
        return 0;
    }
    // (FP32, x, 32): UE8M0 pack (the reference's SM100 path, layout.hpp:45-51).
    if (sf.dtype() == DG_F32 && gran_k == 32) {
        DG_CHECK(!disable_ue8m0_cast);
        return 2;
    }
    // (INT, 1, 32/128): already packed; check TMA-aligned MN-major strides.
    if (sf.dtype() == DG_I32 && gran_mn == 1 && (gran_k == 32 || gran_k == 128)) {
        if (num_groups >= 0) DG_CHECK(sf.stride(-3) == sf.stride(-1) * sf.size(-1));
        check_packed_sf_strides(sf, mn);
        DG_CHECK(sf.stride(-1) % 4 == 0);
        return 0;
    }
    DG_UNSUPPORTED("Unknown SF transformation");
}

void sf3(const View& v, int64_t& g, int64_t& mn, int64_t& k, int64_t& sg, int64_t& smn, int64_t& sk) {
    DG_CHECK(v.dim() == 2 || v.dim() == 3);
    g = v.dim() == 3 ? v.size(0) : 1;
    sg = v.dim() == 3 ? v.stride(0) : 0;
    mn = v.size(-2), k = v.size(-1), smn = v.stride(-2), sk = v.stride(-1);
}

void transpose_impl(const dg_tensor* sf_, const dg_tensor* out_, hipStream_t stream) {
    const View sf = view(sf_, "sf"), out = view(out_, "out");
    DG_CHECK(sf.dtype() == DG_F32 && out.dtype() == DG_F32);
    DG_CHECK(sf.on_device() && out.on_device());
    int64_t g, mn, k, sg, smn, sk, g2, mn2, k2, og, omn, ok;
    sf3(sf, g, mn, k, sg, smn, sk);
    sf3(out, g2, mn2, k2, og, omn, ok);
    DG_CHECK(g == g2 && mn == mn2 && k == k2);
    const int64_t amn = align_up(mn, 4);
    DG_CHECK(omn == 1 && ok == amn);
    if (g > 1) DG_CHECK(og == amn * k);
    SfTransposeArgs args{static_cast<const float*>(sf.data()), static_cast<float*>(const_cast<void*>(out.data())),
                         (int32_t)g, (int32_t)mn, (int32_t)k, sg, smn, sk, og, ok};
    launch_sf_transpose(args, stream);
}

void pack_impl(const dg_tensor* sf_, const dg_tensor* out_, hipStream_t stream) {
    const View sf = view(sf_, "sf"), out = view(out_, "out");
    DG_CHECK(sf.dtype() == DG_F32 && out.dtype() == DG_I32);
    DG_CHECK(sf.on_device() && out.on_device());
    int64_t g, mn, k, sg, smn, sk, g2, mn2, pk, og, omn, ok;
    sf3(sf, g, mn, k, sg, smn, sk);
    sf3(out, g2, mn2, pk, og, omn, ok);
    DG_CHECK(g == g2 && mn == mn2 && pk == ceil_div(k, 4));
    const int64_t amn = align_up(mn, 4);
    DG_CHECK(omn == 1 && ok == amn);
    if (g > 1) DG_CHECK(og == amn * pk);
    SfPackArgs args{static_cast<const float*>(sf.data()), static_cast<int32_t*>(const_cast<void*>(out.data())),
                    (int32_t)g, (int32_t)mn, (int32_t)k, (int32_t)pk, sg, smn, sk, og, ok};
    launch_sf_pack_ue8m0(args, stream);
}

void cast_impl(const dg_tensor* x_, const dg_tensor* q_, const dg_tensor* sf_, int32_t gran_k, int32_t use_ue8m0,
               hipStream_t stream) {
    const View x = view(x_, "x"), q = view(q_, "q"), sf = view(sf_, "sf");
    DG_CHECK(x.dim() == 2 && q.dim() == 2 && sf.dim() == 2);
    DG_CHECK(x.dtype() == DG_BF16 && q.dtype() == DG_E4M3);
    DG_CHECK(x.on_device() && q.on_device() && sf.on_device());
    DG_CHECK(gran_k == 32 || gran_k == 64 || gran_k == 128);
    const int64_t m = x.size(0), n = x.size(1);
    DG_CHECK(q.size(0) == m && q.size(1) == n);
    DG_CHECK(x.stride(-1) == 1 && q.stride(-1) == 1);
    const int64_t groups = ceil_div(n, (int64_t)gran_k);
    const bool packed = sf.dtype() == DG_I32;
    if (packed) {
        DG_CHECK(use_ue8m0);
        DG_CHECK(sf.size(0) == m && sf.size(1) == ceil_div(groups, (int64_t)4));
    } else {
        DG_CHECK(sf.dtype() == DG_F32);
        DG_CHECK(sf.size(0) == m && sf.size(1) == groups);
    }
    DG_CHECK(m < ((int64_t)1 << 31) && n < ((int64_t)1 << 27));
    CastArgs a{};
    a.x = static_cast<const uint16_t*>(x.data());
    a.ldx = x.stride(0);
    a.q = static_cast<uint8_t*>(const_cast<void*>(q.data()));
    a.ldq = q.stride(0);
    a.sf = const_cast<void*>(sf.data());
    a.sf_sm = sf.stride(0), a.sf_sk = sf.stride(1);
    a.m = (int32_t)m, a.n = (int32_t)n, a.gran = gran_k, a.ue8m0 = use_ue8m0 != 0, a.packed = packed;
    launch_per_token_cast(a, stream);
    char buf[160];
    std::snprintf(buf, sizeof(buf), "per_token_cast kind=%s gran_k=%d ue8m0=%d m=%lld n=%lld",
                  packed ? "packed" : "f32", gran_k, (int)a.ue8m0, (long long)m, (long long)n);
    t_last_config = buf;
}

// ---------------------------------------------------------------- MoE plumbing
// The layer around the grouped GEMMs on one GPU, as the reference's MoE baseline
// runs it (tests/test_mega_moe.py:296-330): dispatch into the grouped layouts,
// SwiGLU x routing weight -> FP8 (third-party/tilelang_ops/swiglu_apply_weight_to_fp8.py),
// combine.

bool contiguous_view(const View& t) {
    int64_t want = 1;
    for (int i = t.dim() - 1; i >= 0; --i) {
        if (t.size(i) != 1 && t.stride(i) != want) return false;
        want *= t.size(i);
    }
    return true;
}

int64_t moe_worst_rows(int64_t tokens, int64_t topk, int64_t experts, int64_t alignment) {
    return align_up(tokens * topk + experts * (alignment - 1), alignment);
}

void moe_dispatch_impl(const dg_tensor* x_, const dg_tensor* x_sf_, const dg_tensor* topk_idx_,
                       const dg_tensor* topk_w_, int32_t num_experts, int32_t layout, int32_t alignment,
                       const dg_tensor* a_, const dg_tensor* sf_, const dg_tensor* meta_, const dg_tensor* pos_,
                       const dg_tensor* w_out_, int32_t* workspace, int64_t workspace_ints, hipStream_t stream) {
    const View x = view(x_, "x"), xs = view(x_sf_, "x_sf"), ti = view(topk_idx_, "topk_idx"), a = view(a_, "a"),
               sf = view(sf_, "sf"), meta = view(meta_, "grouped_layout"), pos = view(pos_, "pos");
    DG_CHECK(layout == kMoeContiguous || layout == kMoePsum || layout == kMoeMasked);
    DG_CHECK(num_experts > 0 && num_experts <= kMoeMaxExperts);
    DG_CHECK(x.dim() == 2 && x.dtype() == DG_E4M3 && x.stride(-1) == 1 && x.on_device());
    const int64_t t = x.size(0), kdim = x.size(1), sfk = ceil_div(kdim, (int64_t)128);
    DG_CHECK(kdim % 16 == 0 && t < ((int64_t)1 << 30));
    check_vector_alignment(x, "x");
    DG_CHECK(xs.dim() == 2 && xs.dtype() == DG_F32 && xs.on_device() && xs.size(0) == t && xs.size(1) == sfk);
    DG_CHECK(ti.dim() == 2 && (ti.dtype() == DG_I32 || ti.dtype() == DG_I64) && ti.on_device() && ti.size(0) == t);
    const int64_t k = ti.size(1);
    DG_CHECK(k > 0 && k <= kMoeMaxTopk);
    if (topk_w_) {
        const View tw = view(topk_w_, "topk_weights");
        DG_CHECK(tw.dim() == 2 && tw.dtype() == DG_F32 && tw.on_device() && tw.size(0) == t && tw.size(1) == k);
    }
    DG_CHECK(pos.dim() == 2 && pos.dtype() == DG_I32 && pos.on_device() && pos.size(0) == t && pos.size(1) == k &&
             contiguous_view(pos));
    DG_CHECK(a.dtype() == DG_E4M3 && a.on_device() && a.stride(-1) == 1 && a.size(-1) == kdim);
    DG_CHECK(sf.dtype() == DG_F32 && sf.on_device() && sf.size(-1) == sfk);
    DG_CHECK(meta.dtype() == DG_I32 && meta.on_device() && meta.dim() == 1 && contiguous_view(meta));
    check_vector_alignment(a, "a");
    int64_t cap = 0, max_m = 0;
    if (layout == kMoeMasked) {
        DG_CHECK(a.dim() == 3 && a.size(0) == num_experts && sf.dim() == 3 && sf.size(0) == num_experts);
        max_m = a.size(1);
        DG_CHECK(max_m > 0 && sf.size(1) == max_m && meta.size(0) == num_experts);
        cap = num_experts * max_m;
    } else {
        DG_CHECK(alignment > 0 && alignment % 16 == 0);
        DG_CHECK(a.dim() == 2 && sf.dim() == 2 && sf.size(0) == a.size(0));
        cap = a.size(0);
        // every routing must fit: the segments take at most T*k + E*(alignment - 1) rows
        DG_CHECK(cap >= moe_worst_rows(t, k, num_experts, alignment));
        DG_CHECK(meta.size(0) == (layout == kMoeContiguous ? cap : (int64_t)num_experts));
    }
    DG_CHECK(cap < ((int64_t)1 << 31));
    float* w_out = nullptr;
    if (w_out_) {
        const View wo = view(w_out_, "row_weights");
        DG_CHECK(wo.dtype() == DG_F32 && wo.on_device() && contiguous_view(wo));
        int64_t numel = 1;
        for (int i = 0; i < wo.dim(); ++i) numel *= wo.size(i);
        DG_CHECK(numel == cap);
        w_out = static_cast<float*>(const_cast<void*>(wo.data()));
    }
    DG_CHECK(workspace != nullptr && workspace_ints >= moe_dispatch_workspace_ints(t, num_experts));
    MoeDispatchArgs p{};
    p.x = static_cast<const uint8_t*>(x.data()), p.ldx = x.stride(0);
    p.x_sf = static_cast<const float*>(xs.data()), p.sf_st = xs.stride(0), p.sf_sk = xs.stride(1);
    p.topk = ti.data(), p.topk_i64 = ti.dtype() == DG_I64, p.topk_st = ti.stride(0), p.topk_sk = ti.stride(1);
    if (topk_w_) {
        const View tw = view(topk_w_, "topk_weights");
        p.topk_w = static_cast<const float*>(tw.data()), p.w_st = tw.stride(0), p.w_sk = tw.stride(1);
    }
    p.t = (int32_t)t, p.k = (int32_t)k, p.kdim = (int32_t)kdim, p.sfk = (int32_t)sfk;
    p.num_experts = num_experts, p.layout = layout, p.alignment = alignment, p.max_m = (int32_t)max_m;
    p.chunks = moe_dispatch_chunks(t);
    p.a = static_cast<uint8_t*>(const_cast<void*>(a.data()));
    p.lda = a.stride(-2), p.a_gs = a.dim() == 3 ? a.stride(0) : 0;
    p.sf = static_cast<float*>(const_cast<void*>(sf.data()));
    p.sf_sm = sf.stride(-2), p.sf_sk_o = sf.stride(-1), p.sf_gs = sf.dim() == 3 ? sf.stride(0) : 0;
    p.meta = static_cast<int32_t*>(const_cast<void*>(meta.data()));
    p.cap_rows = cap;
    p.w_out = w_out;
    p.pos = static_cast<int32_t*>(const_cast<void*>(pos.data()));
    p.ws = workspace;
    launch_moe_dispatch(p, stream);
    char buf[160];
    std::snprintf(buf, sizeof(buf), "moe_dispatch layout=%s experts=%d t=%lld k=%lld kdim=%lld",
                  layout == kMoeContiguous ? "contiguous" : layout == kMoePsum ? "psum" : "masked", num_experts,
                  (long long)t, (long long)k, (long long)kdim);
    t_last_config = buf;
}

void moe_swiglu_impl(const dg_tensor* x_, const dg_tensor* w_, const dg_tensor* rl_, float clamp, const dg_tensor* q_,
                     const dg_tensor* sf_, int32_t gran_k, hipStream_t stream) {
    const View x = view(x_, "x"), q = view(q_, "q"), sf = view(sf_, "sf");
    DG_CHECK(x.dim() == 2 && x.dtype() == DG_BF16 && x.on_device() && x.stride(-1) == 1);
    DG_CHECK(q.dim() == 2 && q.dtype() == DG_E4M3 && q.on_device() && q.stride(-1) == 1);
    DG_CHECK(gran_k == 32 || gran_k == 128);
    const int64_t m = x.size(0), n = x.size(1) / 2;
    DG_CHECK(x.size(1) % 2 == 0 && n % gran_k == 0);
    DG_CHECK(q.size(0) == m && q.size(1) == n);
    DG_CHECK(sf.dim() == 2 && sf.dtype() == DG_F32 && sf.on_device() && sf.size(0) == m && sf.size(1) == n / gran_k);
    check_vector_alignment(x, "x");
    DG_CHECK(reinterpret_cast<uintptr_t>(q.data()) % 8 == 0 && q.stride(0) % 8 == 0);
    SwigluCastArgs p{};
    if (w_) {
        const View w = view(w_, "row_weights");
        DG_CHECK(w.dtype() == DG_F32 && w.on_device() && contiguous_view(w));
        int64_t numel = 1;
        for (int i = 0; i < w.dim(); ++i) numel *= w.size(i);
        DG_CHECK(numel == m);
        p.row_weight = static_cast<const float*>(w.data());
    }
    if (rl_) {
        const View rl = view(rl_, "row_layout");
        DG_CHECK(rl.dtype() == DG_I32 && rl.on_device() && rl.dim() == 1 && rl.size(0) == m && contiguous_view(rl));
        p.row_layout = static_cast<const int32_t*>(rl.data());
    }
    DG_CHECK(m < ((int64_t)1 << 31));
    p.x = static_cast<const uint16_t*>(x.data()), p.ldx = x.stride(0);
    p.clamp = clamp;
    p.q = static_cast<uint8_t*>(const_cast<void*>(q.data())), p.ldq = q.stride(0);
    p.sf = static_cast<float*>(const_cast<void*>(sf.data())), p.sf_sm = sf.stride(0), p.sf_sk = sf.stride(1);
    p.m = (int32_t)m, p.n = (int32_t)n, p.gran = gran_k;
    launch_moe_swiglu_cast(p, stream);
    char buf[128];
    std::snprintf(buf, sizeof(buf), "moe_swiglu_cast gran_k=%d m=%lld n=%lld", gran_k, (long long)m, (long long)n);
    t_last_config = buf;
}

void moe_combine_impl(const dg_tensor* y_, const dg_tensor* pos_, const dg_tensor* w_, const dg_tensor* out_,
                      hipStream_t stream) {
    const View y = view(y_, "y"), pos = view(pos_, "pos"), out = view(out_, "out");
    DG_CHECK(y.dtype() == DG_BF16 && y.on_device() && y.stride(-1) == 1 && (y.dim() == 2 || y.dim() == 3));
    DG_CHECK(out.dim() == 2 && out.dtype() == DG_BF16 && out.on_device() && out.stride(-1) == 1);
    DG_CHECK(pos.dim() == 2 && pos.dtype() == DG_I32 && pos.on_device() && contiguous_view(pos));
    const int64_t t = pos.size(0), k = pos.size(1), n = y.size(-1);
    DG_CHECK(out.size(0) == t && out.size(1) == n && n % 8 == 0 && k > 0);
    check_vector_alignment(y, "y");
    check_vector_alignment(out, "out");
    CombineArgs p{};
    p.y = static_cast<const uint16_t*>(y.data());
    p.ldy = y.stride(-2);
    p.y_gs = y.dim() == 3 ? y.stride(0) : 0;
    p.max_m = y.dim() == 3 ? (int32_t)y.size(1) : 0;
    p.rows = y.dim() == 3 ? y.size(0) * y.size(1) : y.size(0);
    p.pos = static_cast<const int32_t*>(pos.data());
    if (w_) {
        const View w = view(w_, "topk_weights");
        DG_CHECK(w.dim() == 2 && w.dtype() == DG_F32 && w.on_device() && w.size(0) == t && w.size(1) == k);
        p.topk_w = static_cast<const float*>(w.data()), p.w_st = w.stride(0), p.w_sk = w.stride(1);
    }
    p.out = static_cast<uint16_t*>(const_cast<void*>(out.data())), p.ldo = out.stride(0);
    DG_CHECK(t < ((int64_t)1 << 31));
    p.t = (int32_t)t, p.k = (int32_t)k, p.n = (int32_t)n;
    launch_moe_combine(p, stream);
    char buf[128];
    std::snprintf(buf, sizeof(buf), "moe_combine t=%lld k=%lld n=%lld", (long long)t, (long long)k, (long long)n);
    t_last_config = buf;
}

// csrc/apis/gemm.hpp:369-425 (k_grouped_fp8_gemm_nt_contiguous), with
// check_k_grouped_args (:55-76) and early_return (:17-53).
void k_grouped_impl(const dg_tensor* a_, const dg_tensor* sfa_, const dg_tensor* b_, const dg_tensor* sfb_,
                    const dg_tensor* d_, const int32_t* ks, int32_t num_ks, const dg_tensor* layout_,
                    const dg_tensor* c, const int32_t* recipe, int32_t use_psum_layout, hipStream_t stream) {
    const View a = view(a_, "a"), sfa = view(sfa_, "sfa"), b = view(b_, "b"), sfb = view(sfb_, "sfb"),
               d = view(d_, "d"), gl = view(layout_, "grouped_layout");
    const int r0 = recipe ? recipe[0] : 1, r1 = recipe ? recipe[1] : 1, r2 = recipe ? recipe[2] : 128;
    DG_CHECK(r0 == 1 && r1 == 1 && r2 == 128);   // recipe == std::make_tuple(1, 1, 128)
    DG_CHECK(!use_psum_layout && ks != nullptr && num_ks > 0);
    check_shape(d, 3);
    const int64_t g = d.size(0), m = d.size(1), n = d.size(2);
    auto numel = [](const View& t) {
        int64_t e = 1;
        for (int i = 0; i < t.dim(); ++i) e *= t.size(i);
        return e;
    };
    auto contiguous = [](const View& t) {
        int64_t want = 1;
        for (int i = t.dim() - 1; i >= 0; --i) {
            if (t.size(i) != 1 && t.stride(i) != want) return false;
            want *= t.size(i);
        }
        return true;
    };
    DG_CHECK(contiguous(gl));
    DG_CHECK(gl.dtype() == DG_I32);
    DG_CHECK(numel(gl) == g);
    DG_CHECK(gl.on_device());
    DG_CHECK((int64_t)num_ks == g);
    int64_t sum_k = 0;
    for (int32_t i = 0; i < num_ks; ++i) {
        DG_CHECK(ks[i] >= 0 && ks[i] % 128 == 0);
        sum_k += ks[i];
    }
    DG_CHECK(numel(a) == sum_k * m);
    DG_CHECK(numel(b) == sum_k * n);
    DG_CHECK(contiguous(a));
    DG_CHECK(contiguous(b));
    DG_CHECK(contiguous(d));
    DG_CHECK(c != nullptr && contiguous(view(c, "c")));
    DG_CHECK(a.dtype() == DG_E4M3 && b.dtype() == DG_E4M3);
    DG_CHECK(a.on_device() && b.on_device());
    // csrc/jit_kernels/impls/sm90_fp8_gemm_1d1d.hpp:153: FP32 D, accumulating into C
    DG_CHECK(d.dtype() == DG_F32);
    const View cv = view(c, "c");
    DG_CHECK(cv.dtype() == DG_F32 && cv.on_device() && cv.dim() == 3);
    for (int i = 0; i < 3; ++i) DG_CHECK(cv.size(i) == d.size(i));
    if (m == 0 || n == 0) return;
    if (sum_k == 0) {   // D = C
        if (cv.data() != d.data())
            launch_fill_or_copy(const_cast<void*>(d.data()), cv.data(), (int)m, (int)n, (int)g, n, m * n, n, m * n,
                                4, stream);
        return;
    }
    // SF: [M, sum_k / 128] and [N, sum_k / 128], FP32, any strides (the kernel
    // reads them in place; the reference makes them MN-major TMA-aligned first)
    DG_CHECK(sfa.dim() == 2 && sfb.dim() == 2 && sfa.dtype() == DG_F32 && sfb.dtype() == DG_F32);
    DG_CHECK(sfa.on_device() && sfb.on_device());
    DG_CHECK(sfa.size(0) == m && sfa.size(1) == sum_k / 128);
    DG_CHECK(sfb.size(0) == n && sfb.size(1) == sum_k / 128);
    check_vector_alignment(d, "d");
    check_vector_alignment(cv, "c");
    DG_CHECK(reinterpret_cast<uintptr_t>(a.data()) % 16 == 0 && reinterpret_cast<uintptr_t>(b.data()) % 16 == 0);
    Fp8GemmArgs args{};
    args.a = static_cast<const uint8_t*>(a.data());
    args.b = static_cast<const uint8_t*>(b.data());
    args.sfa = static_cast<const float*>(sfa.data());
    args.sfb = static_cast<const float*>(sfb.data());
    args.d = const_cast<void*>(d.data());
    args.c = cv.data();
    args.layout = static_cast<const int32_t*>(gl.data());
    args.m = (int32_t)m, args.n = (int32_t)n, args.k = 0;
    args.num_groups = (int32_t)g;
    args.out_f32 = 1;
    args.ldd = n, args.ldc = n, args.d_gs = m * n, args.c_gs = m * n;
    args.sfa_sm = sfa.stride(0), args.sfa_sk = sfa.stride(1);
    args.sfb_sn = sfb.stride(0), args.sfb_sk = sfb.stride(1);
    launch_1d1d(true, args, stream, m, n, sum_k, g);
}

}  // namespace
}  // namespace dgm

using namespace dgm;

extern "C" {

const char* dg_last_error(void) { return t_last_error.c_str(); }

const char* dg_version(void) { return "deepgemm-mi355x 0.1 (gfx950; DeepGEMM 2.8.1 FP8 GEMM API)"; }

int dg_init(void) {
    return guarded([] {
        g_num_sms = 0;
        g_mk_alignment = kDefaultMKAlignment;
        g_tile_variant = 0;
        g_tile_m = 0;
        g_tile_n = 0;
    });
}

int dg_shutdown(void) { return guarded([] {}); }

int dg_fp8_fp4_gemm_nt(const dg_tensor* a, const dg_tensor* sfa, const dg_tensor* b, const dg_tensor* sfb,
                       const dg_tensor* d, const dg_tensor* c, const dg_recipe* recipe, int32_t disable_ue8m0_cast,
                       const dg_epilogue* epilogue, void* stream) {
    return guarded([&] {
        gemm_nt_impl(a, sfa, b, sfb, d, c, recipe, disable_ue8m0_cast, epilogue, static_cast<hipStream_t>(stream));
    });
}

int dg_fp8_fp4_gemm_nt_ws(const dg_tensor* a, const dg_tensor* sfa, const dg_tensor* b, const dg_tensor* sfb,
                          const dg_tensor* d, const dg_tensor* c, const dg_recipe* recipe, int32_t disable_ue8m0_cast,
                          const dg_epilogue* epilogue, const dg_tensor* workspace, void* stream) {
    return guarded([&] {
        gemm_nt_impl(a, sfa, b, sfb, d, c, recipe, disable_ue8m0_cast, epilogue, static_cast<hipStream_t>(stream),
                     workspace);
    });
}

int64_t dg_fp8_gemm_nt_workspace_size(int64_t m, int64_t n, int64_t k) {
    int64_t out = -1;
    if (guarded([&] { out = dense_workspace_bytes(m, n, k); }) != DG_OK) return -1;
    return out;
}

int dg_m_grouped_fp8_fp4_gemm_nt_contiguous(const dg_tensor* a, const dg_tensor* sfa, const dg_tensor* b,
                                            const dg_tensor* sfb, const dg_tensor* d, const dg_tensor* grouped_layout,
                                            const dg_recipe* recipe, int32_t disable_ue8m0_cast,
                                            int32_t use_psum_layout, int32_t ensure_zero_padding,
                                            int32_t expected_m_for_psum_layout, const dg_epilogue* epilogue,
                                            void* stream) {
    return guarded([&] {
        contiguous_impl(a, sfa, b, sfb, d, grouped_layout, recipe, disable_ue8m0_cast, use_psum_layout,
                        ensure_zero_padding, expected_m_for_psum_layout, epilogue, static_cast<hipStream_t>(stream));
    });
}

int dg_k_grouped_fp8_gemm_nt_contiguous(const dg_tensor* a, const dg_tensor* sfa, const dg_tensor* b,
                                        const dg_tensor* sfb, const dg_tensor* d, const int32_t* ks_cpu,
                                        int32_t num_ks, const dg_tensor* grouped_layout, const dg_tensor* c,
                                        const int32_t* recipe, int32_t use_psum_layout, void* stream) {
    return guarded([&] {
        k_grouped_impl(a, sfa, b, sfb, d, ks_cpu, num_ks, grouped_layout, c, recipe, use_psum_layout,
                       static_cast<hipStream_t>(stream));
    });
}

int dg_k_grouped_fp8_gemm_tn_contiguous(const dg_tensor* a, const dg_tensor* sfa, const dg_tensor* b,
                                        const dg_tensor* sfb, const dg_tensor* d, const int32_t* ks_cpu,
                                        int32_t num_ks, const dg_tensor* grouped_layout, const dg_tensor* c,
                                        const int32_t* recipe, int32_t use_psum_layout, void* stream) {
    (void)a, (void)sfa, (void)b, (void)sfb, (void)d, (void)ks_cpu, (void)num_ks, (void)grouped_layout, (void)c;
    (void)recipe, (void)use_psum_layout, (void)stream;
    // The reference runs the MN-major (TN) form only with its SM100 kernel
    // (csrc/apis/gemm.hpp:360-367); like its SM90 build, this one does not.
    return guarded([&] { DG_UNSUPPORTED("Unsupported architecture: k_grouped_fp8_gemm_tn_contiguous"); });
}

int dg_m_grouped_fp8_fp4_gemm_nt_masked(const dg_tensor* a, const dg_tensor* sfa, const dg_tensor* b,
                                        const dg_tensor* sfb, const dg_tensor* d, const dg_tensor* masked_m,
                                        int32_t expected_m, const dg_recipe* recipe, int32_t disable_ue8m0_cast,
                                        const dg_epilogue* epilogue, void* stream) {
    return guarded([&] {
        masked_impl(a, sfa, b, sfb, d, masked_m, expected_m, recipe, disable_ue8m0_cast, epilogue,
                    static_cast<hipStream_t>(stream));
    });
}

int dg_m_grouped_fp8_gemm_nt_contiguous_swiglu(const dg_tensor* a, const dg_tensor* sfa, const dg_tensor* b,
                                               const dg_tensor* sfb, const dg_tensor* grouped_layout,
                                               const dg_tensor* row_weights, float clamp_value, const dg_tensor* q,
                                               const dg_tensor* sf, int32_t use_psum_layout,
                                               int32_t ensure_zero_padding, void* stream) {
    return guarded([&] {
        swiglu_l1_impl(use_psum_layout ? kPsum : kContiguous, a, sfa, b, sfb, grouped_layout, -1, row_weights,
                       clamp_value, q, sf, ensure_zero_padding, static_cast<hipStream_t>(stream));
    });
}

int dg_m_grouped_fp8_gemm_nt_masked_swiglu(const dg_tensor* a, const dg_tensor* sfa, const dg_tensor* b,
                                           const dg_tensor* sfb, const dg_tensor* masked_m, int32_t expected_m,
                                           const dg_tensor* row_weights, float clamp_value, const dg_tensor* q,
                                           const dg_tensor* sf, void* stream) {
    return guarded([&] {
        swiglu_l1_impl(kMasked, a, sfa, b, sfb, masked_m, expected_m, row_weights, clamp_value, q, sf, 0,
                       static_cast<hipStream_t>(stream));
    });
}

int dg_get_tma_aligned_size(int32_t x, int32_t element_size, int32_t* out) {
    return guarded([&] {
        DG_CHECK(out != nullptr);
        DG_CHECK(element_size > 0 && 16 % element_size == 0);
        *out = (int32_t)align_up(x, 16 / element_size);
    });
}

int dg_get_mn_major_tma_aligned_tensor(const dg_tensor* sf, const dg_tensor* out, void* stream) {
    return guarded([&] { transpose_impl(sf, out, static_cast<hipStream_t>(stream)); });
}

int dg_get_mn_major_tma_aligned_packed_ue8m0_tensor(const dg_tensor* sf, const dg_tensor* out, void* stream) {
    return guarded([&] { pack_impl(sf, out, static_cast<hipStream_t>(stream)); });
}

int dg_plan_sf_transform(const dg_tensor* sf, int32_t mn, int32_t k, const int32_t* recipe3, const int32_t* recipe2,
                         int32_t num_groups, int32_t is_sfa, int32_t disable_ue8m0_cast, int32_t* kind) {
    return guarded([&] {
        DG_CHECK(kind != nullptr);
        *kind = plan_sf(sf, mn, k, recipe3, recipe2, num_groups, is_sfa, disable_ue8m0_cast);
    });
}

int dg_per_token_cast_to_fp8(const dg_tensor* x, const dg_tensor* q, const dg_tensor* sf, int32_t gran_k,
                             int32_t use_ue8m0, void* stream) {
    return guarded([&] { cast_impl(x, q, sf, gran_k, use_ue8m0, static_cast<hipStream_t>(stream)); });
}

int64_t dg_moe_dispatch_workspace_size(int64_t num_tokens, int32_t num_experts) {
    if (num_tokens < 0 || num_experts <= 0) return -1;
    return moe_dispatch_workspace_ints(num_tokens, num_experts) * 4;
}

int64_t dg_moe_dispatch_max_rows(int64_t num_tokens, int32_t num_topk, int32_t num_experts, int32_t alignment) {
    if (num_tokens < 0 || num_topk <= 0 || num_experts <= 0 || alignment <= 0) return -1;
    return moe_worst_rows(num_tokens, num_topk, num_experts, alignment);
}

int dg_moe_dispatch(const dg_tensor* x, const dg_tensor* x_sf, const dg_tensor* topk_idx, const dg_tensor* topk_weights,
                    int32_t num_experts, int32_t layout, int32_t alignment, const dg_tensor* a, const dg_tensor* sf,
                    const dg_tensor* grouped_layout, const dg_tensor* pos, const dg_tensor* row_weights,
                    const dg_tensor* workspace, void* stream) {
    return guarded([&] {
        const View ws = view(workspace, "workspace");
        DG_CHECK(ws.dtype() == DG_I32 && ws.on_device() && contiguous_view(ws));
        int64_t numel = 1;
        for (int i = 0; i < ws.dim(); ++i) numel *= ws.size(i);
        moe_dispatch_impl(x, x_sf, topk_idx, topk_weights, num_experts, layout, alignment, a, sf, grouped_layout, pos,
                          row_weights, static_cast<int32_t*>(const_cast<void*>(ws.data())), numel,
                          static_cast<hipStream_t>(stream));
    });
}

int dg_moe_dispatch_noalloc(const dg_tensor* x, const dg_tensor* x_sf, const dg_tensor* topk_idx,
                            const dg_tensor* topk_weights, int32_t num_experts, int32_t layout, int32_t alignment,
                            const dg_tensor* a, const dg_tensor* sf, const dg_tensor* grouped_layout,
                            const dg_tensor* pos, const dg_tensor* row_weights, void* stream) {
    return guarded([&] {
        const View xv = view(x, "x");
        DG_CHECK(xv.dim() == 2 && num_experts > 0);
        int dev = -1;   // the scratch used is the current device's copy
        DG_HIP_CHECK(hipGetDevice(&dev));
        DG_CHECK(xv.on_device() && x->device == dev);
        const int64_t need = moe_dispatch_workspace_ints(xv.size(0), num_experts);
        if (need > kMoeScratchInts)
            throw Error(DG_ERR_INVALID, "Assertion", __FILE__, __LINE__,
                        "the allocation-free dispatch needs " + std::to_string(need) +
                            " int32 of scratch, more than its fixed " + std::to_string(kMoeScratchInts) +
                            "; use dg_moe_dispatch with a workspace");
        moe_dispatch_impl(x, x_sf, topk_idx, topk_weights, num_experts, layout, alignment, a, sf, grouped_layout, pos,
                          row_weights, moe_scratch_device_ptr(), kMoeScratchInts, static_cast<hipStream_t>(stream));
    });
}

int dg_moe_swiglu_apply_weight_to_fp8(const dg_tensor* x, const dg_tensor* row_weights, const dg_tensor* row_layout,
                                      float clamp_value, const dg_tensor* q, const dg_tensor* sf, int32_t gran_k,
                                      void* stream) {
    return guarded([&] {
        moe_swiglu_impl(x, row_weights, row_layout, clamp_value, q, sf, gran_k, static_cast<hipStream_t>(stream));
    });
}

int dg_moe_combine(const dg_tensor* y, const dg_tensor* pos, const dg_tensor* topk_weights, const dg_tensor* out,
                   void* stream) {
    return guarded([&] { moe_combine_impl(y, pos, topk_weights, out, static_cast<hipStream_t>(stream)); });
}

int dg_set_num_sms(int32_t num_sms) {
    return guarded([&] {
        DG_CHECK(num_sms > 0);
        g_num_sms = num_sms;
    });
}

int dg_get_num_sms(int32_t* out) {
    return guarded([&] {
        DG_CHECK(out != nullptr);
        *out = num_sms_now();
    });
}

int dg_set_mk_alignment_for_contiguous_layout(int32_t alignment) {
    return guarded([&] {
        DG_CHECK(alignment > 0);
        g_mk_alignment = alignment;
    });
}

int32_t dg_get_mk_alignment_for_contiguous_layout(void) { return g_mk_alignment.load(); }

int32_t dg_get_theoretical_mk_alignment_for_contiguous_layout(int32_t expected_m) {
    // The gfx950 kernels use M blocks of at most 128 rows; 128 keeps every
    // compiled block_m a divisor (csrc/jit_kernels/heuristics/runtime.hpp:57-64).
    (void)expected_m;
    return kDefaultMKAlignment;
}

int dg_set_tile_override(int32_t variant, int32_t block_m, int32_t block_n) {
    return guarded([&] {
        if (variant == 0) {
            g_tile_variant = 0, g_tile_m = 0, g_tile_n = 0;
            return;
        }
        const bool ok = variant == 1   ? fp8_1d2d_tile_supported(block_m, block_n)
                        : variant == 2 ? fp8_1d2d_v2_tile_supported(block_m, block_n)
                        : variant == 5 ? ((block_m == kMaskedStreamRows || block_m == kStream16Rows) &&
                                          block_n % 32 == 0 && block_n >= 128 &&
                                          block_n <= 256)
                        : variant == 6 ? (block_m == 128 && (block_n == 128 || block_n == 192 || block_n == 256))
                        : variant == 7 ? (block_m == 128 && block_n == 128)
                        : variant == 8 || variant == 9
                            ? ((block_m == 16 || block_m == 32 || block_m == kTinyMRows) &&
                               (block_n == 16 || block_n == 32 || block_n == 64))
                        : variant == 10 ? (block_m == 0 && block_n >= 0 && block_n <= 1024)
                                       : (variant == 4 && block_m == 256 && block_n == 256);
        if (!ok) DG_UNSUPPORTED("tile shape not compiled");
        g_tile_m = block_m, g_tile_n = block_n;
        g_tile_variant = variant;
    });
}

int dg_last_config(char* buf, int32_t cap) {
    return guarded([&] {
        DG_CHECK(buf != nullptr && cap > 0);
        std::snprintf(buf, (size_t)cap, "%s", t_last_config.c_str());
    });
}

}  // extern "C"
