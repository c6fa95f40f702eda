// ffn_mi355x.hip -- host side of libffn_mi355x.so: tile planning, Stream-K schedule,
// launch sequencing and the extern "C" entry points declared in include/ffn_mi355x.h.
//
// The reference builds one artifact per FFN with tla.compile and launches it once
// (ops/host/dispatch.py:97-116, ops/api.py:37-45); here the kernels are compiled ahead
// of time for gfx950 and an FFN is two stream-ordered launches of the GEMM engine:
// up-projection + GELU epilogue, then the Basic or Stream-K down-projection.  The
// kernel boundary is the stage barrier that the reference builds from cross-core flags
// (ops/kernel/ffn.py:371-376, 582-585).
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <atomic>
#include <mutex>
#include <string>

#include "ffn_gemm.hpp"
#include "ffn_mi355x.h"
#include "ffn_variants.hpp"

#ifndef FFN_MI355X_REVISION
#define FFN_MI355X_REVISION "unversioned"
#endif

typedef hipError_t (*ffn_launch_fn)(int role, const ffn::GemmParams* p, int grid, hipStream_t stream);

#define FFN_DECLARE_LAUNCHERS(id, bm, bn, bk, wgm, wgn, st, ...)                                    \
    extern "C" hipError_t ffn_launch_d0_v##id(int, const ffn::GemmParams*, int, hipStream_t); \
    extern "C" hipError_t ffn_launch_d1_v##id(int, const ffn::GemmParams*, int, hipStream_t);
FFN_VARIANTS(FFN_DECLARE_LAUNCHERS)
#undef FFN_DECLARE_LAUNCHERS

typedef hipError_t (*ffn_fused_fn)(int role, const ffn::GemmParams* pu, const ffn::GemmParams* pd,
                                   const ffn::FusedParams* f, int grid, hipStream_t stream);
#define FFN_DECLARE_FUSED(u, d)                                                                          \
    extern "C" hipError_t ffn_fused_d0_u##u##_n##d(int, const ffn::GemmParams*, const ffn::GemmParams*, \
                                                   const ffn::FusedParams*, int, hipStream_t);          \
    extern "C" hipError_t ffn_fused_d1_u##u##_n##d(int, const ffn::GemmParams*, const ffn::GemmParams*, \
                                                   const ffn::FusedParams*, int, hipStream_t);
FFN_FUSED_PAIRS(FFN_DECLARE_FUSED)
#undef FFN_DECLARE_FUSED

namespace {

struct Variant {
    int bm, bn, bk, wgm, wgn, stages;
    int lds_bytes;            // LDS of one workgroup: the stages plus any epilogue staging beyond
    int nw;                   // waves holding wave tiles
    int wgk;                  // waves along K (K-sliced tile when > 1)
    int prod;                 // waves that only refill the LDS stages
    int mf;                   // MFMA block edge: 32 (32x32x16) or 16 (16x16x32)
    ffn_launch_fn launch[2];  // [dtype]
    int waves() const { return nw + prod; }
    int lds() const { return lds_bytes; }
};

#define FFN_VARIANT_ROW(id, bm, bn, bk, wgm, wgn, st, ...)                                     \
    {bm, bn, bk, wgm, wgn, st, ffn::TileCfg<bm, bn, bk, wgm, wgn, st, ##__VA_ARGS__>::LDS_USE, \
     ffn::TileCfg<bm, bn, bk, wgm, wgn, st, ##__VA_ARGS__>::NW,                                \
     ffn::TileCfg<bm, bn, bk, wgm, wgn, st, ##__VA_ARGS__>::WGK,                               \
     ffn::TileCfg<bm, bn, bk, wgm, wgn, st, ##__VA_ARGS__>::PROD,                              \
     ffn::TileCfg<bm, bn, bk, wgm, wgn, st, ##__VA_ARGS__>::MF,                                \
     {ffn_launch_d0_v##id, ffn_launch_d1_v##id}},
const Variant kVariants[] = {FFN_VARIANTS(FFN_VARIANT_ROW)};
#undef FFN_VARIANT_ROW
constexpr int kNumVariants = (int)(sizeof(kVariants) / sizeof(kVariants[0]));
static_assert(kNumVariants == FFN_NUM_VARIANTS, "variant table");

// Single-launch FFN kernels of the compiled (up, down) variant pairs (ffn_fused.hip).
struct FusedPair {
    int up, down;
    ffn_fused_fn launch[2];  // [dtype]
};
#define FFN_FUSED_ROW(u, d) {u, d, {ffn_fused_d0_u##u##_n##d, ffn_fused_d1_u##u##_n##d}},
const FusedPair kFusedPairs[] = {FFN_FUSED_PAIRS(FFN_FUSED_ROW)};
#undef FFN_FUSED_ROW
const FusedPair* fused_pair(int up, int down) {
    for (const FusedPair& f : kFusedPairs)
        if (f.up == up && f.down == down) return &f;
    return nullptr;
}

thread_local std::string g_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

int ok() {
    g_error.clear();
    return FFN_MI355X_OK;
}

long long cdiv(long long a, long long b) { return (a + b - 1) / b; }

// ---- planning -------------------------------------------------------------------------
// A small time model picks the tile: per-workgroup time = work units x per-iteration time,
// where an iteration is bounded by the tile's MFMA rate and by the loads the workgroup can
// keep in flight ((S-1) stages over the memory latency), and the whole GEMM by streaming
// its operands from HBM once.  Rates are measured on MI355X (sustained clock ~1.8-2 GHz).
constexpr double kCuMfmaRate = 4.8e12;     // FLOP/s per CU a 256x256 tile sustains
constexpr double kCuLoadRate = 60e9;       // B/s per CU of LDS-DMA alongside MFMA work
constexpr double kLoadLatency = 0.8e-6;    // s, L2/MALL load latency under load
constexpr double kHbmRate = 6.5e12;        // B/s sustained HBM read rate
constexpr double kFinishLatency = 1.2e-6;  // s, one dependent step of a split tile's finish:
                                           // partial write-through, arrival count, partial reads
constexpr double kUnitOverhead = 2.5e-6;   // s per unit: DMA prologue latency + epilogue

// Relative MFMA efficiency of each macro tile (measured on the FFN shapes, 256x256 = 1): the
// fragment reads per MFMA grow as the wave tile shrinks.  A K-sliced 128x128 tile has 128x64
// wave tiles (and pays an LDS exchange of half its partials per tile); with two waves per SIMD
// (eight tile waves, or four beside four refill waves) one wave's work covers the other's waits.
// The K-sliced 64x64 tile (64x32 wave tiles, two MFMAs per k-step) is a little ahead of the
// plain one.  A tile whose refill is issued by waves of its own (no wave tile) keeps its tile
// waves off the texture unit: 1.6-18% ahead of the same tile without them on the Basic downs
// and unaligned up it serves.  A tile of 16x16x32 blocks runs at a higher clock for the same
// power: the DiT-size up GEMM 7% and its Stream-K down 4% faster than on the same tile of
// 32x32x16 blocks.
double tile_eff(const Variant& v, bool up = false) {
    const int a = v.bm < v.bn ? v.bm : v.bn, b = v.bm < v.bn ? v.bn : v.bm;
    const double refill = (v.prod > 0 ? 1.03 : 1.0) * (v.mf == 16 ? 1.05 : 1.0);
    // The K-sliced 32x32 decode tile (32x32 wave tiles, one MFMA per k-step and wave) reads the
    // most fragments per MFMA: 0.15, from the 512x1024 -> 4096 -> 1024 FFN's Basic down, where its
    // 512 tiles took 30.7 us against 27.0 us for 128 K-sliced 64x64 tiles (one tuning run).
    if (v.wgk > 1) return refill * (a >= 128 ? (v.nw + v.prod >= 8 ? 0.9 : 0.85) : a >= 64 ? 0.3 : 0.15);
    if (a >= 256) return refill * 1.0;
    // 256x192 (16x16 blocks): 0.92 per FLOP of the 256x256 tile, from the DiT-size up at eight
    // tiles per CU (493.5 against 453.0 us at six of 256x256) and its H/8 shard at one wave of
    // tiles (62.6 against 74.5 us on 192 of 256x256)
    if (a == 192 && b == 256) return refill * 0.92;
    // The 256x128 and 128x256 tiles as the up GEMM (GELU epilogue, short K): 0.88.  On
    // 16384x1152 -> 4608, 4096x8192 -> 21824 and 8192x1024 -> 2752 the automatic up on the
    // 256x128 tile ran 2-6% behind the 256x192 or 256x256 tile that a rating of 0.88 picks; as
    // the down GEMM it keeps 0.95, where the same change lost 5-9% (512x4096 -> 16384 Stream-K,
    // 4096x5120 -> 13632 Basic).
    if (a == 128 && b == 256) return refill * (up ? 0.88 : 0.95);
    if (a == 128) return refill * 0.6;
    if (a == 64 && b >= 128) return refill * 0.42;
    return refill * 0.25;
}

// Seconds per BK-deep iteration of one workgroup on a tile with `rows` data-bearing rows.
double iter_time(const Variant& v, long long rows, bool up = false) {
    const double flops = 2.0 * v.bm * v.bn * v.bk;
    const double t_mfma = flops / (kCuMfmaRate * tile_eff(v, up));
    const double bytes = (double)(rows + v.bn) * v.bk * 2.0;
    const double inflight = (double)(v.stages - 1) * (double)(v.bm + v.bn) * v.bk * 2.0;
    // refill-only waves take the texture unit's stalls off the tile waves, where the refill
    // bounds the iteration too: the K-sliced 128x128 tile with them (v24) against the one
    // without (v10), both load-bound here, took the 3000x1000 -> 4000 -> 1000 fp16 FFN's Basic
    // down 7% faster
    const double rate = std::min(kCuLoadRate, inflight / kLoadLatency) * (v.prod > 0 ? 1.03 : 1.0);
    return std::max(t_mfma, bytes / rate);
}

long long rows_in_tile(const Variant& v, long long m_valid) { return std::min<long long>(v.bm, m_valid); }

// Estimated seconds of a data-parallel GEMM [M x N] (m_valid data rows), depth K.
double cost_basic(const Variant& v, long long M, long long m_valid, long long N, long long K, int G,
                  bool up = false) {
    (void)M;
    const long long T = cdiv(m_valid, v.bm) * cdiv(N, v.bn);
    const long long waves = cdiv(T, G);
    const double t = (double)waves * ((double)cdiv(K, v.bk) * iter_time(v, rows_in_tile(v, m_valid), up) +
                                      kUnitOverhead);
    const double hbm = (double)(N * K + m_valid * K) * 2.0 / kHbmRate;
    return std::max(t, hbm);
}

struct SkShape {
    long long tiles, k_iters, grid, dp, sk, q, r, slots;
    long long pieces;  // pieces per tile of a reduced grid; 0 when the grid is block_num
};

// Stream-K grid: block_num workgroups, or fewer when every tile is split (fewer tiles than
// workgroups): p pieces per tile, p a divisor of the tile's iterations where one exists (each
// workgroup then covers exactly one piece of one tile, none straddles two tiles and needs a
// second partial slot), p at most kMaxPieces: the last piece of a tile reads the others' partials
// in a chain of dependent loads that grows with p.  On the 16x5120 -> 13824 -> 5120 decode down,
// 240 workgroups (80 tiles x 3 pieces of 72 iterations) measured 6% faster than 256 with pieces
// of 67.5; on the smallest FFN's down (8 tiles), 16 one-iteration pieces per tile measured 24%
// slower than a separate reduction launch.
constexpr long long kMaxPieces = 4;
long long sk_pieces(long long tiles, long long k_iters, int G) {
    const long long pmax = std::min<long long>({(long long)G / std::max<long long>(1, tiles), kMaxPieces, k_iters});
    if (tiles >= G || pmax < 2) return 0;
    for (long long p = pmax; p >= 2; --p)
        if (k_iters % p == 0) return p;
    return pmax;
}
long long sk_grid(long long tiles, long long k_iters, int G) {
    const long long p = sk_pieces(tiles, k_iters, G);
    return p ? tiles * p : G;
}

// Tiles of a GEMM whose rows [m_valid, M) are zero padding: only tile rows holding data are
// computed (the kernel zero-fills the rows past them).
// Arrival counters of split tiles (one per tile and wave) live in a fixed region at the start
// of the workspace; a split schedule needing more than it holds is not used.
constexpr size_t kCounterBytes = FFN_MI355X_WORKSPACE_COUNTER_BYTES;
bool counters_fit(long long split_tiles, const Variant& v) { return split_tiles * v.nw * 4 <= (long long)kCounterBytes; }

bool sk_shape(const Variant& v, long long m_valid, long long N, long long K, int block_num, SkShape& s) {
    s.tiles = cdiv(m_valid, v.bm) * cdiv(N, v.bn);
    s.k_iters = cdiv(K, v.bk);
    s.pieces = sk_pieces(s.tiles, s.k_iters, block_num);
    const long long G = s.pieces ? s.tiles * s.pieces : block_num;
    s.grid = G;
    s.sk = s.tiles % G;
    s.dp = s.tiles - s.sk;
    const long long total = s.sk * s.k_iters;
    s.q = total / G;
    s.r = total % G;
    const long long span = s.q + (s.r ? 1 : 0);
    // a range of `span` iterations touches at most ceil(span / k_iters) + 1 tiles
    s.slots = cdiv(span, s.k_iters) + 1;
    return s.sk > 0 && s.k_iters >= 2 && counters_fit(s.sk, v);
}

double cost_streamk(const Variant& v, const SkShape& s, long long m_valid, long long N, long long K,
                    bool up = false) {
    const long long G = s.grid;
    const double it = iter_time(v, rows_in_tile(v, m_valid), up);
    const long long dp_waves = cdiv(s.dp, G);
    const long long sk_iters = s.q + (s.r ? 1 : 0);
    // Pieces that start at scattered depths of their tiles (a grid of block_num workgroups over
    // a number of split tiles that does not divide it, so a tile holds a fractional number of
    // pieces): neighbouring workgroups of an XCD read different K slices at any moment, so no
    // panel slice is shared in L2 and the split iterations stream at the chip's HBM rate.  On the
    // 1024x5120 -> 13824 -> 5120 fp16 FFN the 256x128 down's 160 tiles so split (1.6 pieces a
    // tile) took ~270 us, against ~150 us for 80 tiles of 256x256 in three aligned pieces.
    // A whole number of pieces a tile keeps their offsets within an iteration of K / pieces.
    const bool scattered = s.pieces == 0 && s.sk > 0 && (G % s.sk) != 0;
    double it_split = it;
    if (scattered)
        it_split = std::max(it, (double)(rows_in_tile(v, m_valid) + v.bn) * v.bk * 2.0 * (double)G / kHbmRate);
    double t = it * (double)dp_waves * s.k_iters + it_split * (double)sk_iters +
               kUnitOverhead * (double)(dp_waves + 1);
    // shared split tiles: each piece writes its FP32 partial through to memory and counts in;
    // the last reads the others (several at a time when its waves hold at most two 32x32
    // blocks, one at a time otherwise) and stores the tile
    const long long pieces_per_tile = std::min<long long>(G, cdiv(s.k_iters, std::max<long long>(1, s.q)) + 1);
    if (s.k_iters > sk_iters) {
        const double tile_bytes = (double)v.bm * v.bn * 4.0;
        const long long per_read = (long long)v.bm * v.bn / v.nw <= 2048 ? 4 : 1;
        t += kFinishLatency * (double)(2 + cdiv(pieces_per_tile - 1, per_read)) +
             (double)pieces_per_tile * tile_bytes / kCuLoadRate;
    }
    const double hbm = (double)(N * K + m_valid * K) * 2.0 / kHbmRate;
    return std::max(t, hbm);
}

// A candidate replaces the best so far when it is cheaper by more than 0.1%, or within 0.1% on a
// tile of higher MFMA efficiency: where the load or HBM term bounds every candidate alike (a
// load-bound 128x128 down, scattered split pieces), the tile that computes faster wins the tie
// instead of the lower variant number (aligned mid-size down at 2048 rows: v24 133.3 us, v18
// 147.7, v10 155.0, one tuning run).  Not where the tiles are taller than the rows holding data:
// a decode-size GEMM at the HBM bound gains nothing from a tall tile's efficiency (16 x 8192 ->
// 21824: the 128x128 tile 4% behind the 32x32 one).
bool better(double c, const Variant& v, double best_cost, const Variant& best, long long m_valid) {
    return c < best_cost * 0.999 || (c <= best_cost * 1.001 && v.bm <= m_valid && best.bm <= m_valid &&
                                     tile_eff(v) > tile_eff(best));
}

int pick_basic(long long M, long long m_valid, long long N, long long K, int G) {
    int best = 0;
    double best_cost = 1e300;
    for (int i = 0; i < kNumVariants; ++i) {
        const double c = cost_basic(kVariants[i], M, m_valid, N, K, G);
        if (better(c, kVariants[i], best_cost, kVariants[best], m_valid)) best_cost = c, best = i;
    }
    return best;
}

// The 256x192 tile is not an automatic Stream-K down: it would make Stream-K applicable where
// every power-of-two tiling divides the grid, and there lost to the Basic down it competes with
// (8192x4096 -> 8192: 877.9 against 774.7 us), its split form holding more work per workgroup
// than the whole tiles it replaces.  A forced down_variant still takes it.
bool sk_candidate(const Variant& v) { return !(v.mf == 16 && v.bn == 192); }

int pick_streamk(long long M, long long m_valid, long long N, long long K, int G) {
    int best = -1;
    double best_cost = 1e300;
    for (int i = 0; i < kNumVariants; ++i) {
        if (!sk_candidate(kVariants[i])) continue;
        SkShape s;
        if (!sk_shape(kVariants[i], m_valid, N, K, G, s)) continue;
        const double c = cost_streamk(kVariants[i], s, m_valid, N, K);
        if (best < 0 || better(c, kVariants[i], best_cost, kVariants[best], m_valid)) best_cost = c, best = i;
    }
    return best;
}

// Split up GEMM: taken when the up's tiles would leave at least half of the workgroups idle and
// the reduction is deep enough to split (a decode-size FFN with a narrow H, e.g. one GPU's H/8
// share of a 16x5120 -> 13824 FFN, whose few tiles would stream W1 on a few CUs).  Every tile is
// then cut into p equal pieces (sk_grid); the last piece of a tile to finish sums the partials
// and applies the activation.  On that decode shard (54 tiles of 32x32, 4 pieces of 10
// iterations on 216 workgroups) the split up takes 10.6-10.8 us.
constexpr int kUpSplitMinIters = 16;
bool split_up(const Variant& v, long long m_valid, long long N, long long K, int G, SkShape& s) {
    const long long tiles = cdiv(m_valid, v.bm) * cdiv(N, v.bn), k_iters = cdiv(K, v.bk);
    if (tiles * 2 > G || k_iters < kUpSplitMinIters) return false;
    const long long grid = sk_grid(tiles, k_iters, G);
    if (!sk_shape(v, m_valid, N, K, (int)grid, s) || s.grid != grid || s.dp != 0 || s.sk != tiles) return false;
    const long long kI = s.k_iters, big = (s.q + 1) * s.r;
    auto owner = [&](long long x) { return s.q == 0 ? x : x < big ? x / (s.q + 1) : s.r + (x - big) / s.q; };
    for (long long t = 0; t < tiles; ++t)
        if (owner(t * kI) == owner(t * kI + kI - 1)) return false;
    return true;
}

// Up-GEMM tile when none is forced: every variant is priced as the plan it would get, split
// along K (Stream-K cost, the finish of split tiles included) or one workgroup per tile.
// A SwiGLU up GEMM (N = 2 x the hidden width, gate and up rows interleaved in 32-row blocks)
// needs wave tiles of whole block pairs, and is never split: no split role is compiled for it.
bool swiglu_tile(const Variant& v) { return (v.bn / v.wgn) % 64 == 0; }

// A tile that would be split competes only when no tiling of 64x64 or more fills more than half
// of the grid with whole tiles: at 128 rows (128 x 4096 -> 16384) the 128x128 tile split in two
// pieces priced ahead of 256 whole 64x128 tiles and measured 9-15% slower on the FFN; at 64 rows
// and H 8192 only the 32x32 decode tiles fill the grid, and the split 64x64 tile stays 10%
// ahead of them.
int pick_up(long long M, long long m_valid, long long N, long long K, int G, bool swiglu) {
    int best = -1;
    double best_cost = 1e300;
    bool fills = false;
    for (int i = 0; i < kNumVariants; ++i)
        fills |= (!swiglu || swiglu_tile(kVariants[i])) && kVariants[i].bm * kVariants[i].bn >= 64 * 64 &&
                 cdiv(m_valid, kVariants[i].bm) * cdiv(N, kVariants[i].bn) * 2 > G;
    for (int i = 0; i < kNumVariants; ++i) {
        if (swiglu && !swiglu_tile(kVariants[i])) continue;
        SkShape s;
        const bool split = !swiglu && split_up(kVariants[i], m_valid, N, K, G, s);
        if (split && fills) continue;
        const double c = split ? cost_streamk(kVariants[i], s, m_valid, N, K, true)
                               : cost_basic(kVariants[i], M, m_valid, N, K, G, true);
        if (best < 0 || better(c, kVariants[i], best_cost, kVariants[best], m_valid)) best_cost = c, best = i;
    }
    return best;
}

// Tile-row group of the tile order (tile_coords): consecutive tiles walk 4 tile rows column by
// column.  Whole-FFN runs, interleaved, two boxes: against groups of 8, the aligned
// 4096x1024 -> 4096 FFN -0.8% and -1.4%, the DiT-size FFN -0.7% and -0.3%; groups of 2 and 16
// were slower.
int group_m_for(long long tiles_m) { return (int)(tiles_m < 4 ? tiles_m : 4); }

// Refill DMA addressing (GemmParams::fast_dma).  The SALU-addressed path takes the vector
// offset arithmetic out of the MFMA stream and measured 2-5% faster on reductions up to 8192
// deep (every up GEMM, and the down GEMM of hidden widths up to 8192); on the 12288- and
// 13824-deep down GEMMs it measured up to 20% slower than the checked path, which they keep.
constexpr int kFastDmaMaxK = 8192;
int fast_dma_for(int k) { return k <= kFastDmaMaxK ? 1 : 0; }

// Depth of the down GEMM's reduction: the logical H when hidden rows can be read to it in
// whole 16-byte chunks, else the padded H (W2 then spans hp columns, zero past h).
int down_depth(const ffn_mi355x_plan* p) { return p->h % 8 == 0 ? p->h : p->hp; }

// Largest operand row pitch (elements).  The kernels address a macro tile's rows with 32-bit
// buffer offsets: up to 256 rows of a pitch plus the K offset, (256 + 1) * pitch * 2 bytes,
// must stay below 2^31, the offset that marks a zero-filled chunk.
constexpr int kMaxPitch = FFN_MI355X_MAX_PITCH;
static_assert((256LL + 1) * kMaxPitch * 2 < (1LL << 31), "a tile's row offsets stay below 2^31");

bool pitch_ok(int ld) { return ld % 8 == 0 && ld <= kMaxPitch; }

// Bytes from X's base to the end of the furthest row element the up GEMM reads, for gathered
// rows (ffn_mi355x_set_x_rows); -1 for a grid that does not tile the m rows.
long long x_grid_span(const ffn_mi355x_plan* p) {
    if (p->x_d1 < 1 || p->x_d2 < 1 || p->m % ((long long)p->x_d1 * p->x_d2) != 0) return -1;
    if (p->x_s0 < 0 || p->x_s1 < 0 || p->x_s2 < 0 || p->x_s0 % 8 || p->x_s1 % 8 || p->x_s2 % 8) return -1;
    const long long d0 = p->m / ((long long)p->x_d1 * p->x_d2);
    return ((d0 - 1) * p->x_s0 + (long long)(p->x_d1 - 1) * p->x_s1 + (long long)(p->x_d2 - 1) * p->x_s2 + p->k) * 2;
}

// Gathered rows are addressed with 32-bit buffer offsets below 2^31, the zero-fill offset.
constexpr long long kMaxGatherSpan = 1LL << 31;

bool layout_ok(const ffn_mi355x_plan* p) {
    const bool x_ok = p->x_d1 == 0 ? p->x_d2 == 0 && p->x_s0 == 0 && p->x_s1 == 0 && p->x_s2 == 0
                                   : x_grid_span(p) > 0 && x_grid_span(p) <= kMaxGatherSpan;
    return p->k >= 1 && p->k <= p->kp && (p->k % 8 == 0 || p->k == p->kp) && p->h >= 1 && p->h <= p->hp &&
           p->n >= 1 && p->n <= p->np && p->ldx >= p->k && pitch_ok(p->ldx) && p->ldw1 >= p->k &&
           pitch_ok(p->ldw1) && p->ldw2 >= down_depth(p) && pitch_ok(p->ldw2) && x_ok;
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

// Bytes of a row-major buffer the kernels touch: `rows` rows at `pitch` elements, of which the
// last is read or written only to `width` elements.
size_t span_bytes(long long rows, long long pitch, long long width) {
    return rows <= 0 ? 0 : (size_t)((rows - 1) * pitch + width) * 2u;
}

// [ptr, ptr + bytes) must lie inside one HIP allocation: a host pointer or a buffer too short
// for the plan is refused before any launch instead of faulting the GPU.  The runtime is asked
// on every call (a map lookup, well under a microsecond): a cached answer would go stale when a
// buffer is freed and a smaller one allocated at the same address.  The check sees HIP
// allocations, not sub-blocks of a caching allocator: a span that runs past a torch tensor into
// another block of the same segment passes.
bool in_allocation(const void* ptr, size_t bytes) {
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    if (hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)ptr) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    const uintptr_t b = (uintptr_t)base, q = (uintptr_t)ptr;
    return q >= b && bytes <= size && q - b <= size - bytes;
}

int check_span(const char* name, const void* ptr, size_t bytes) {
    if (in_allocation(ptr, bytes)) return FFN_MI355X_OK;
    return fail(FFN_MI355X_EINVAL, "buffer %s at %p: %zu bytes needed are not inside one device allocation",
                name, ptr, bytes);
}

// Check word of a plan: FNV-1a (64-bit) over every field but the stamp, seeded with a constant
// of this library.  Fields are hashed by value, so struct padding never enters it.
unsigned long long plan_stamp(const ffn_mi355x_plan* p) {
    unsigned long long h = 0xcbf29ce484222325ull ^ 0x6666e6d69333535ull;
    auto mix = [&h](unsigned long long v) {
        for (int i = 0; i < 8; ++i) {
            h ^= (v >> (8 * i)) & 0xffu;
            h *= 0x100000001b3ull;
        }
    };
    const int ints[] = {p->m, p->mp, p->kp, p->hp, p->np, p->dtype, p->down_impl, p->activation, p->block_num,
                        p->up_variant, p->down_variant, p->up_bm, p->up_bn, p->up_bk, p->down_bm, p->down_bn,
                        p->down_bk, p->up_tiles, p->up_grid, p->down_tiles, p->down_grid, p->down_k_iters,
                        p->down_dp_tiles, p->down_sk_tiles, p->down_slots_per_wg, p->k, p->h, p->n, p->ldx,
                        p->ldw1, p->ldw2, p->up_k_iters, p->up_sk_tiles, p->up_slots_per_wg,
                        p->x_d1, p->x_d2, p->x_s0, p->x_s1, p->x_s2, p->single_launch};
    for (int v : ints) mix((unsigned long long)(unsigned)v);
    mix((unsigned long long)p->workspace_bytes);
    return h;
}

// A plan is used only as ffn_mi355x_make_plan (and ffn_mi355x_set_operands) left it: the grids,
// tile counts, Stream-K split and workspace size it carries decide which memory the kernels
// touch.  Both entry points derive them and stamp the plan; a plan whose fields no longer match
// its stamp is refused.  (The stamp catches accidental edits of a plan, not forgery.)
bool valid_plan(const ffn_mi355x_plan* p) {
    return p && p->stamp == plan_stamp(p) && p->m >= 1 && p->m <= p->mp && layout_ok(p) && p->up_variant >= 0 &&
           p->up_variant < kNumVariants && p->down_variant >= 0 && p->down_variant < kNumVariants &&
           (p->dtype == 0 || p->dtype == 1) &&
           (p->down_impl == FFN_MI355X_DOWN_BASIC || p->down_impl == FFN_MI355X_DOWN_STREAMK) &&
           p->activation >= FFN_MI355X_GELU_ERF && p->activation <= FFN_MI355X_SWIGLU && p->block_num >= 1;
}

// Workspace layout: a fixed region of arrival counters first (one per split tile and wave, for
// the split up GEMM and the Stream-K down alike, which run one after the other; every launch
// leaves them zero), then the FP32 partial-tile slots.  The region has the same size for every
// plan, so one zero-filled workspace serves any plans in turn: no plan's slots overlap another
// plan's counters.
size_t flags_bytes(const ffn_mi355x_plan*) { return kCounterBytes; }

// Arrival counters (one word per split tile and wave): the Stream-K down's from the start of the
// counter region, a split up GEMM's from its end, so that each GEMM's launch can clear the
// other's (GemmParams::clear_words) without touching its own.
// Each split tile's counters take a 128-byte line of their own (FFN_MI355X_SPLIT_COUNTER_WORDS
// words) when both GEMMs' split tiles fit the region that way, else they are packed (the tile's
// waves only).  Atomics on one line are serialised (~11 ns apiece), and every piece of every
// split tile counts in at about the same time, at the end of a launch: packed, the decode FFN's
// Stream-K down put 96 arrivals (8 tiles x 3 pieces x 4 waves) on each line.
constexpr int kSplitWords = FFN_MI355X_SPLIT_COUNTER_WORDS;
bool spread_counters(long long up_sk, long long down_sk) {
    return (up_sk + down_sk) * kSplitWords <= (long long)(kCounterBytes / 4);
}
long long down_split_tiles(const ffn_mi355x_plan* p) {
    return p->down_impl == FFN_MI355X_DOWN_STREAMK ? p->down_sk_tiles : 0;
}
int counter_stride(const ffn_mi355x_plan* p, const Variant& v) {
    return spread_counters(p->up_sk_tiles, down_split_tiles(p)) ? kSplitWords : v.nw;
}
size_t down_counter_words(const ffn_mi355x_plan* p) {
    return (size_t)down_split_tiles(p) * (size_t)counter_stride(p, kVariants[p->down_variant]);
}
size_t up_counter_words(const ffn_mi355x_plan* p) {
    return p->up_sk_tiles > 0 ? (size_t)p->up_sk_tiles * (size_t)counter_stride(p, kVariants[p->up_variant]) : 0;
}
unsigned* up_counters(const ffn_mi355x_plan* p, void* ws) {
    return (unsigned*)ws + (kCounterBytes / 4 - up_counter_words(p));
}


// A plan can run as one launch (ffn_fused.hip): a compiled kernel for its tile pair, a Basic down,
// an unsplit up GEMM with the GELU epilogue (its K within the SALU-addressed refill), at least one
// up row block per XCD and whole down row blocks per up row block, and room in the counter
// region for the queues and the row-block counters.
bool fused_ok(const ffn_mi355x_plan* p) {
    if (!fused_pair(p->up_variant, p->down_variant)) return false;
    const Variant& U = kVariants[p->up_variant];
    const Variant& D = kVariants[p->down_variant];
    const long long rbs = cdiv(p->m, U.bm);
    return p->down_impl == FFN_MI355X_DOWN_BASIC && p->up_sk_tiles == 0 &&
           (p->activation == FFN_MI355X_GELU_ERF || p->activation == FFN_MI355X_GELU_RATIONAL) &&
           U.nw + U.prod == D.nw + D.prod && U.bm % D.bm == 0 && rbs >= 8 &&
           ffn::kFusedReady + rbs * ffn::kFusedStride <= (long long)(kCounterBytes / 4) && fast_dma_for(p->kp);
}

int launch(const Variant& v, int dtype, int role, const ffn::GemmParams& gp, int grid,
           void* stream) {
    const hipError_t e = v.launch[dtype](role, &gp, grid, (hipStream_t)stream);
    if (e != hipSuccess)
        return fail(FFN_MI355X_EHIP, "kernel launch failed: %s", hipGetErrorString(e));
    return ok();
}

}  // namespace

extern "C" {

int ffn_mi355x_query(int device, int* cu_count, char* arch, int arch_len) {
    hipDeviceProp_t prop;
    const hipError_t e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess)
        return fail(FFN_MI355X_EHIP, "hipGetDeviceProperties(%d): %s", device, hipGetErrorString(e));
    if (cu_count) *cu_count = prop.multiProcessorCount;
    if (arch && arch_len > 0) {
        strncpy(arch, prop.gcnArchName, (size_t)arch_len - 1);
        arch[arch_len - 1] = '\0';
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(FFN_MI355X_EDEVICE, "This implementation targets gfx950 (MI355X) only, got %s",
                    prop.gcnArchName);
    return ok();
}

int ffn_mi355x_make_plan(int m, int mp, int kp, int hp, int np, int dtype, int down_impl, int activation,
                         int block_num, int up_variant, int down_variant, ffn_mi355x_plan* plan) {
    if (!plan) return fail(FFN_MI355X_EINVAL, "plan must not be NULL");
    if (m <= 0 || m > mp)
        return fail(FFN_MI355X_EINVAL, "logical rows m must be in [1, mp] (got m=%d mp=%d)", m, mp);
    if (dtype != FFN_MI355X_FP16 && dtype != FFN_MI355X_BF16)
        return fail(FFN_MI355X_EINVAL, "dtype must be float16 or bfloat16");
    if (activation < FFN_MI355X_GELU_ERF || activation > FFN_MI355X_SWIGLU)
        return fail(FFN_MI355X_EINVAL, "activation must be erf GELU, rational GELU, SiLU or SwiGLU");
    const bool swiglu = activation == FFN_MI355X_SWIGLU;
    if (down_impl == FFN_MI355X_DOWN_FULL_LOAD_A || down_impl == FFN_MI355X_DOWN_FULL_LOAD_B)
        return fail(FFN_MI355X_EUNAVAILABLE, "%s: no gfx950 kernel is provided for this down variant; no fallback",
                    down_impl == FFN_MI355X_DOWN_FULL_LOAD_A ? "full_load_a" : "full_load_b");
    if (down_impl != FFN_MI355X_DOWN_BASIC && down_impl != FFN_MI355X_DOWN_STREAMK)
        return fail(FFN_MI355X_EINVAL, "Unknown down_impl: %d", down_impl);
    if (block_num < 1 || block_num > 65535)
        return fail(FFN_MI355X_EINVAL,
                    "block_num must be a positive integer; hardware limit checked before launch");
    if (mp <= 0 || kp <= 0 || hp <= 0 || np <= 0 || mp % 64 || hp % 64 || np % 64 || kp % 16)
        return fail(FFN_MI355X_EINVAL,
                    "padded extents must be positive, M/H/N multiples of 64 and K a multiple of 16 "
                    "(got mp=%d kp=%d hp=%d np=%d)", mp, kp, hp, np);
    if (kp > 65536 || hp > 65536 || np > 65536 || mp > INT_MAX - 256)
        return fail(FFN_MI355X_EINVAL, "Shape exceeds the supported bounds");
    if (up_variant >= kNumVariants || down_variant >= kNumVariants)
        return fail(FFN_MI355X_EINVAL, "tile variant out of range (0..%d)", kNumVariants - 1);

    memset(plan, 0, sizeof *plan);
    plan->m = m;
    plan->mp = mp, plan->kp = kp, plan->hp = hp, plan->np = np;
    plan->dtype = dtype, plan->down_impl = down_impl, plan->activation = activation, plan->block_num = block_num;
    const int G = block_num;

    // up: [mp x hp], depth kp (SwiGLU: [mp x 2hp], gate and up column blocks interleaved)
    const long long un = swiglu ? 2LL * hp : hp;
    if (swiglu && up_variant >= 0 && !swiglu_tile(kVariants[up_variant]))
        return fail(FFN_MI355X_EINVAL, "SwiGLU needs an up tile whose wave tiles are multiples of 64 columns "
                    "(variant %d is not)", up_variant);
    const int uv = up_variant >= 0 ? up_variant : pick_up(mp, m, un, kp, G, swiglu);
    const Variant& U = kVariants[uv];
    plan->up_variant = uv;
    plan->up_bm = U.bm, plan->up_bn = U.bn, plan->up_bk = U.bk;
    plan->up_tiles = (int)(cdiv(m, U.bm) * cdiv(un, U.bn));
    plan->up_grid = plan->up_tiles < G ? plan->up_tiles : G;
    plan->up_k_iters = (int)cdiv(kp, U.bk);
    size_t up_ws = 0;
    SkShape su;
    if (!swiglu && split_up(U, m, hp, kp, G, su)) {
        plan->up_sk_tiles = (int)su.sk;
        plan->up_slots_per_wg = (int)su.slots;
        plan->up_grid = (int)su.grid;
        up_ws = (size_t)su.grid * (size_t)su.slots * (size_t)U.bm * (size_t)U.bn * 4u;
    }

    // down: [mp x np], depth hp
    int dv;
    if (down_impl == FFN_MI355X_DOWN_STREAMK) {
        if (down_variant >= 0) {
            SkShape s;
            if (!sk_shape(kVariants[down_variant], m, np, hp, G, s)) {
                if (s.k_iters < 2)
                    return fail(FFN_MI355X_ENOT_APPLICABLE,
                                "Stream-K candidate requires at least two K tiles along H");
                if (s.sk > 0)
                    return fail(FFN_MI355X_ENOT_APPLICABLE,
                                "Stream-K candidate splits more tiles (%lld) than the workspace counters "
                                "hold for this block_num", s.sk);
                return fail(FFN_MI355X_ENOT_APPLICABLE,
                            "Stream-K candidate has no remainder tiles for this block_num");
            }
            dv = down_variant;
        } else {
            dv = pick_streamk(mp, m, np, hp, G);
            if (dv < 0) {
                bool any_two = false;
                for (int i = 0; i < kNumVariants; ++i) any_two |= cdiv(hp, kVariants[i].bk) >= 2;
                if (!any_two)
                    return fail(FFN_MI355X_ENOT_APPLICABLE,
                                "Stream-K candidate requires at least two K tiles along H");
                return fail(FFN_MI355X_ENOT_APPLICABLE,
                            "Stream-K candidate has no remainder tiles for this block_num");
            }
        }
    } else {
        dv = down_variant >= 0 ? down_variant : pick_basic(mp, m, np, hp, G);
    }
    const Variant& D = kVariants[dv];
    plan->down_variant = dv;
    plan->down_bm = D.bm, plan->down_bn = D.bn, plan->down_bk = D.bk;
    plan->down_tiles = (int)(cdiv(m, D.bm) * cdiv(np, D.bn));
    plan->down_k_iters = (int)cdiv(hp, D.bk);
    if (down_impl == FFN_MI355X_DOWN_STREAMK) {
        SkShape s;
        sk_shape(D, m, np, hp, G, s);
        plan->down_dp_tiles = (int)s.dp;
        plan->down_sk_tiles = (int)s.sk;
        plan->down_slots_per_wg = (int)s.slots;
        plan->down_grid = (int)s.grid;
        plan->workspace_bytes = (size_t)s.grid * (size_t)s.slots * (size_t)D.bm * (size_t)D.bn * 4u;
    } else {
        plan->down_dp_tiles = plan->down_tiles;
        plan->down_grid = plan->down_tiles < G ? plan->down_tiles : G;
        plan->workspace_bytes = 0;
    }
    if (up_ws > plan->workspace_bytes) plan->workspace_bytes = up_ws;
    if (plan->workspace_bytes > 0) plan->workspace_bytes += flags_bytes(plan);
    // The single launch is opt-in (ffn_mi355x_set_single_launch): measured against the two launches
    // of the same tile pair it was slower on every workload it serves (aligned mid-size 78.6
    // against 72.0 us, unaligned 45.4 against 30.2, DiT-size 1065 against 979).  A plan that can
    // take it reserves the counter region, so its workspace serves either form.
    plan->single_launch = 0;
    if (fused_ok(plan) && plan->workspace_bytes < flags_bytes(plan)) plan->workspace_bytes = flags_bytes(plan);
    if (up_counter_words(plan) + down_counter_words(plan) > kCounterBytes / 4)
        return fail(FFN_MI355X_ENOT_APPLICABLE, "the split tiles of the two GEMMs need more arrival counters "
                    "(%zu) than the workspace holds (%zu)", up_counter_words(plan) + down_counter_words(plan),
                    kCounterBytes / 4);
    // the kernels address partial slots with 32-bit buffer offsets
    if (plan->workspace_bytes >= (size_t)1 << 31)
        return fail(FFN_MI355X_EINVAL, "workspace of %zu bytes exceeds 2 GiB", plan->workspace_bytes);
    plan->k = kp, plan->h = hp, plan->n = np;
    plan->ldx = kp, plan->ldw1 = kp, plan->ldw2 = hp;
    plan->x_d1 = plan->x_d2 = plan->x_s0 = plan->x_s1 = plan->x_s2 = 0;
    if (!layout_ok(plan))
        return fail(FFN_MI355X_EINVAL, "padded extents exceed the largest row pitch (%d elements)", kMaxPitch);
    plan->stamp = plan_stamp(plan);
    return ok();
}

int ffn_mi355x_set_operands(ffn_mi355x_plan* plan, int k, int h, int n, int ldx, int ldw1, int ldw2) {
    if (!plan) return fail(FFN_MI355X_EINVAL, "plan must not be NULL");
    if (!valid_plan(plan)) return fail(FFN_MI355X_EINVAL, "invalid plan");
    ffn_mi355x_plan t = *plan;
    t.k = k, t.h = h, t.n = n, t.ldx = ldx, t.ldw1 = ldw1, t.ldw2 = ldw2;
    if (!layout_ok(&t))
        return fail(FFN_MI355X_EINVAL,
                    "operand layout k=%d h=%d n=%d ldx=%d ldw1=%d ldw2=%d does not fit the plan "
                    "(kp=%d hp=%d np=%d): k a multiple of 8 or kp, pitches multiples of 8 covering "
                    "the widths and at most %d, W2 spanning hp columns when h is not a multiple of 8",
                    k, h, n, ldx, ldw1, ldw2, plan->kp, plan->hp, plan->np, kMaxPitch);
    t.stamp = plan_stamp(&t);
    *plan = t;
    return ok();
}

int ffn_mi355x_set_x_rows(ffn_mi355x_plan* plan, int d1, int d2, int s0, int s1, int s2) {
    if (!plan) return fail(FFN_MI355X_EINVAL, "plan must not be NULL");
    if (!valid_plan(plan)) return fail(FFN_MI355X_EINVAL, "invalid plan");
    ffn_mi355x_plan t = *plan;
    if (d1 == 0) t.x_d1 = t.x_d2 = t.x_s0 = t.x_s1 = t.x_s2 = 0;
    else t.x_d1 = d1, t.x_d2 = d2, t.x_s0 = s0, t.x_s1 = s1, t.x_s2 = s2;
    if (!layout_ok(&t))
        return fail(FFN_MI355X_EINVAL,
                    "row grid d1=%d d2=%d strides (%d, %d, %d) does not fit m=%d k=%d: d1*d2 must divide m, "
                    "strides be non-negative multiples of 8 and the rows lie within 2^31 bytes",
                    d1, d2, s0, s1, s2, plan->m, plan->k);
    t.stamp = plan_stamp(&t);
    *plan = t;
    return ok();
}

int ffn_mi355x_set_single_launch(ffn_mi355x_plan* plan, int on) {
    if (!plan) return fail(FFN_MI355X_EINVAL, "plan must not be NULL");
    if (!valid_plan(plan)) return fail(FFN_MI355X_EINVAL, "invalid plan");
    if (on && !fused_ok(plan))
        return fail(FFN_MI355X_ENOT_APPLICABLE, "no single-launch kernel for this plan (tile pair %d/%d, %s down)",
                    plan->up_variant, plan->down_variant,
                    plan->down_impl == FFN_MI355X_DOWN_BASIC ? "Basic" : "Stream-K");
    ffn_mi355x_plan t = *plan;
    t.single_launch = on ? 1 : 0;
    t.stamp = plan_stamp(&t);
    *plan = t;
    return ok();
}

int ffn_mi355x_workspace_bytes(const ffn_mi355x_plan* plan, size_t* bytes) {
    if (!plan || !bytes) return fail(FFN_MI355X_EINVAL, "NULL argument");
    *bytes = plan->workspace_bytes;
    return ok();
}

int ffn_mi355x_workspace_counter_bytes(const ffn_mi355x_plan* plan, size_t* bytes) {
    if (!plan || !bytes) return fail(FFN_MI355X_EINVAL, "NULL argument");
    if (!valid_plan(plan)) return fail(FFN_MI355X_EINVAL, "invalid plan");
    *bytes = plan->workspace_bytes > 0 ? flags_bytes(plan) : 0;
    return ok();
}

}  // extern "C"

namespace {

void set_workspace(ffn::GemmParams& gp, const ffn_mi355x_plan* plan, void* ws, bool up) {
    const size_t f = flags_bytes(plan);
    gp.sk_flags = up ? up_counters(plan, ws) : (unsigned*)ws;
    gp.sk_stride = counter_stride(plan, kVariants[up ? plan->up_variant : plan->down_variant]);
    gp.ws = (float*)((char*)ws + f);
    gp.ws_bytes = (unsigned)(plan->workspace_bytes - f);
}

// Up GEMM of a plan.  ws_scratch: ws is this library's scratch array (its size is known, and it
// is not a HIP allocation of its own to look up).
// Rows of W1 a plan reads: the logical H, or for SwiGLU the 2 hp interleaved gate and up rows.
long long w1_rows(const ffn_mi355x_plan* p) { return p->activation == FFN_MI355X_SWIGLU ? 2LL * p->hp : p->h; }

// built: fill *built and *role_out with the launch of an unsplit up GEMM instead of launching it.
int run_up(const ffn_mi355x_plan* plan, const void* x, const void* w1, const void* b1, void* hidden, void* ws,
           bool ws_scratch, void* hip_stream, ffn::GemmParams* built = nullptr, int* role_out = nullptr) {
    if (!valid_plan(plan)) return fail(FFN_MI355X_EINVAL, "invalid plan");
    if (!x || !w1 || !hidden) return fail(FFN_MI355X_EINVAL, "NULL device buffer");
    if (!aligned16(x) || !aligned16(w1) || !aligned16(hidden) || (ws && !aligned16(ws)) || (b1 && !aligned16(b1)))
        return fail(FFN_MI355X_EINVAL, "device buffers must be 16-byte aligned");
    const bool split = plan->up_sk_tiles > 0;
    const bool swiglu = plan->activation == FFN_MI355X_SWIGLU;
    if (split && !ws)
        return fail(FFN_MI355X_EINVAL, "the split up GEMM needs a workspace of %zu bytes", plan->workspace_bytes);
    const long long rows = w1_rows(plan);
    int rc;
    const bool gather = plan->x_d1 != 0;
    const size_t x_span = gather ? (size_t)x_grid_span(plan) : span_bytes(plan->m, plan->ldx, plan->k);
    if ((rc = check_span("x", x, x_span)) != FFN_MI355X_OK ||
        (rc = check_span("w1", w1, span_bytes(rows, plan->ldw1, plan->k))) != FFN_MI355X_OK ||
        (b1 && (rc = check_span("bias1", b1, (size_t)rows * 2u)) != FFN_MI355X_OK) ||
        (rc = check_span("hidden", hidden, span_bytes(plan->mp, plan->hp, plan->hp))) != FFN_MI355X_OK ||
        (split && !ws_scratch && (rc = check_span("ws", ws, plan->workspace_bytes)) != FFN_MI355X_OK) ||
        (!split && ws && !ws_scratch && down_counter_words(plan) > 0 &&
         (rc = check_span("ws", ws, flags_bytes(plan))) != FFN_MI355X_OK))
        return rc;
    const Variant& U = kVariants[plan->up_variant];
    ffn::GemmParams gp;
    memset(&gp, 0, sizeof gp);
    gp.a = x, gp.b = w1, gp.c = hidden;
    // all hp hidden columns are written: those past h from zero rows of W1 (act(0) = 0 for every
    // activation, and a bias reads as zero past h)
    gp.M = plan->mp, gp.N = (int)(swiglu ? 2LL * plan->hp : plan->hp), gp.K = plan->k;
    gp.c_cols = plan->hp;
    gp.m_valid = plan->m, gp.n_valid = (int)rows;
    gp.lda = plan->ldx, gp.ldb = plan->ldw1, gp.ldc = plan->hp;
    gp.tiles_m = (int)cdiv(plan->m, U.bm), gp.tiles_n = (int)cdiv(gp.N, U.bn);
    gp.zero_row0 = (int)std::min<long long>(plan->mp, (long long)gp.tiles_m * U.bm);
    gp.k_iters = plan->up_k_iters;
    gp.dp_tiles = gp.tiles_m * gp.tiles_n;
    gp.group_m = group_m_for(gp.tiles_m);
    gp.fast_dma = fast_dma_for(gp.K);
    gp.bias = b1, gp.bias_n = b1 ? (int)rows : 0;
    if (gather) {
        gp.a_gather = 1;
        gp.a_d1 = plan->x_d1, gp.a_d2 = plan->x_d2;
        gp.a_s0 = plan->x_s0, gp.a_s1 = plan->x_s1, gp.a_s2 = plan->x_s2;
        gp.a_bytes = (unsigned)x_span;
    }
    if (ws && down_counter_words(plan) > 0) {
        // the Stream-K down that follows counts on zero counters: clear them here
        gp.clear_words = (unsigned*)ws;
        gp.clear_count = (int)down_counter_words(plan);
    }
    if (split && built) return fail(FFN_MI355X_EINVAL, "a split up GEMM does not run in a single launch");
    if (split) {
        // every tile split (no whole tiles): FP32 partials; the last piece of a tile applies the
        // activation
        const long long total = (long long)plan->up_sk_tiles * plan->up_k_iters;
        gp.dp_tiles = 0;
        gp.sk_tiles = plan->up_sk_tiles;
        gp.sk_q = (int)(total / plan->up_grid);
        gp.sk_r = (int)(total % plan->up_grid);
        gp.slots_per_wg = plan->up_slots_per_wg;
        set_workspace(gp, plan, ws, true);
        const int role = plan->activation == FFN_MI355X_GELU_ERF        ? FFN_ROLE_UP_SPLIT_ERF
                         : plan->activation == FFN_MI355X_GELU_RATIONAL ? FFN_ROLE_UP_SPLIT_RATIONAL
                                                                        : FFN_ROLE_UP_SPLIT_SILU;
        return launch(U, plan->dtype, role, gp, plan->up_grid, hip_stream);
    }
    const int role = plan->activation == FFN_MI355X_GELU_ERF        ? FFN_ROLE_UP_ERF
                     : plan->activation == FFN_MI355X_GELU_RATIONAL ? FFN_ROLE_UP_RATIONAL
                     : plan->activation == FFN_MI355X_SILU          ? FFN_ROLE_UP_SILU
                                                                    : FFN_ROLE_UP_SWIGLU;
    if (built) {
        *built = gp, *role_out = role;
        return ok();
    }
    return launch(U, plan->dtype, role, gp, plan->up_grid, hip_stream);
}

// Down GEMM of a plan (ws_scratch as for run_up).
// built: fill *built with the launch of a Basic down GEMM instead of launching it.
int run_down(const ffn_mi355x_plan* plan, const void* hidden, const void* w2, const void* b2, void* out, void* ws,
             bool ws_scratch, void* hip_stream, ffn::GemmParams* built = nullptr) {
    if (!valid_plan(plan)) return fail(FFN_MI355X_EINVAL, "invalid plan");
    if (!hidden || !w2 || !out) return fail(FFN_MI355X_EINVAL, "NULL device buffer");
    if (!aligned16(hidden) || !aligned16(w2) || !aligned16(out) || (ws && !aligned16(ws)) || (b2 && !aligned16(b2)))
        return fail(FFN_MI355X_EINVAL, "device buffers must be 16-byte aligned");
    int rc;
    if ((rc = check_span("hidden", hidden, span_bytes(plan->m, plan->hp, down_depth(plan)))) != FFN_MI355X_OK ||
        (rc = check_span("w2", w2, span_bytes(plan->n, plan->ldw2, down_depth(plan)))) != FFN_MI355X_OK ||
        (b2 && (rc = check_span("bias2", b2, (size_t)plan->n * 2u)) != FFN_MI355X_OK) ||
        (rc = check_span("out", out, span_bytes(plan->mp, plan->np, plan->np))) != FFN_MI355X_OK ||
        (plan->down_impl == FFN_MI355X_DOWN_STREAMK && ws && !ws_scratch &&
         (rc = check_span("ws", ws, plan->workspace_bytes)) != FFN_MI355X_OK) ||
        (plan->down_impl != FFN_MI355X_DOWN_STREAMK && ws && !ws_scratch && up_counter_words(plan) > 0 &&
         (rc = check_span("ws", ws, flags_bytes(plan))) != FFN_MI355X_OK))
        return rc;
    const Variant& D = kVariants[plan->down_variant];
    ffn::GemmParams gp;
    memset(&gp, 0, sizeof gp);
    gp.a = hidden, gp.b = w2, gp.c = out;
    gp.M = plan->mp, gp.N = plan->np, gp.K = down_depth(plan);
    gp.c_cols = plan->np;
    gp.bias = b2, gp.bias_n = b2 ? plan->n : 0;
    gp.m_valid = plan->m, gp.n_valid = plan->n;
    gp.lda = plan->hp, gp.ldb = plan->ldw2, gp.ldc = plan->np;
    gp.tiles_m = (int)cdiv(plan->m, D.bm), gp.tiles_n = (int)cdiv(plan->np, D.bn);
    gp.zero_row0 = (int)std::min<long long>(plan->mp, (long long)gp.tiles_m * D.bm);
    gp.k_iters = plan->down_k_iters;
    gp.group_m = group_m_for(gp.tiles_m);
    gp.fast_dma = fast_dma_for(gp.K);
    // the up GEMM writes hidden tile row after tile row: starting from its last rows finds
    // more of hidden in the last-level cache (DiT-size FFN step: 1044 -> 1037 us Basic,
    // 1056 -> 1043 us Stream-K)
    gp.rev_m = 1;
    if (ws && up_counter_words(plan) > 0) {
        // the split up GEMM of the next call counts on zero counters: clear them here
        gp.clear_words = up_counters(plan, ws);
        gp.clear_count = (int)up_counter_words(plan);
    }
    if (plan->down_impl == FFN_MI355X_DOWN_STREAMK) {
        if (!ws) return fail(FFN_MI355X_EINVAL, "Stream-K needs a workspace of %zu bytes", plan->workspace_bytes);
        const int G = plan->down_grid;
        gp.dp_tiles = plan->down_dp_tiles;
        gp.sk_tiles = plan->down_sk_tiles;
        const long long total = (long long)plan->down_sk_tiles * plan->down_k_iters;
        gp.sk_q = (int)(total / G);
        gp.sk_r = (int)(total % G);
        gp.slots_per_wg = plan->down_slots_per_wg;
        set_workspace(gp, plan, ws, false);
        return launch(D, plan->dtype, FFN_ROLE_DOWN_STREAMK, gp, G, hip_stream);
    }
    gp.dp_tiles = plan->down_tiles;
    if (built) {
        *built = gp;
        return ok();
    }
    return launch(D, plan->dtype, FFN_ROLE_DOWN_BASIC, gp, plan->down_grid, hip_stream);
}

// The whole FFN of a plan: one launch when the plan says so and X is not read as gathered rows
// (ffn_fused.hip, counters in the workspace's counter region), else up then down.
int run_ffn(const ffn_mi355x_plan* plan, const void* x, const void* w1, const void* b1, const void* w2,
            const void* b2, void* hidden, void* out, void* ws, bool ws_scratch, void* hip_stream) {
    if (!valid_plan(plan)) return fail(FFN_MI355X_EINVAL, "invalid plan");
    int rc;
    if (plan->single_launch && plan->x_d1 == 0) {
        if (!ws) return fail(FFN_MI355X_EINVAL, "the single launch needs a workspace of %zu bytes", plan->workspace_bytes);
        if (!ws_scratch && (rc = check_span("ws", ws, flags_bytes(plan))) != FFN_MI355X_OK) return rc;
        ffn::GemmParams pu, pd;
        int role = 0;
        if ((rc = run_up(plan, x, w1, b1, hidden, nullptr, false, hip_stream, &pu, &role)) != FFN_MI355X_OK) return rc;
        if ((rc = run_down(plan, hidden, w2, b2, out, nullptr, false, hip_stream, &pd)) != FFN_MI355X_OK) return rc;
        const Variant& U = kVariants[plan->up_variant];
        const Variant& D = kVariants[plan->down_variant];
        ffn::FusedParams f;
        f.ctr = (unsigned*)ws, f.ratio = U.bm / D.bm, f.spin_limit = 1 << 20;
        const FusedPair* fp = fused_pair(plan->up_variant, plan->down_variant);
        const hipError_t e = fp->launch[plan->dtype](role, &pu, &pd, &f, plan->block_num, (hipStream_t)hip_stream);
        if (e != hipSuccess) return fail(FFN_MI355X_EHIP, "kernel launch failed: %s", hipGetErrorString(e));
        return ok();
    }
    if ((rc = run_up(plan, x, w1, b1, hidden, ws, ws_scratch, hip_stream)) != FFN_MI355X_OK) return rc;
    return run_down(plan, hidden, w2, b2, out, ws, ws_scratch, hip_stream);
}

// ---- scratch of the entry point that allocates nothing ----------------------------------
// The FP32 partial tiles of a Stream-K down or a split up GEMM, for callers that cannot
// allocate: device memory of this library's own code object.  Each GPU the library is loaded
// on holds its own copy of FFN_MI355X_NOALLOC_SCRATCH_BYTES until the process ends.  In host
// code `scratch` only names the symbol: its device address, per device, comes from
// hipGetSymbolAddress and is what the kernels are given.
static __device__ __align__(256) unsigned char scratch[FFN_MI355X_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];
std::mutex g_scratch_mutex;

// Device address of `scratch` on the device of `stream`, looked up once per device with that
// device current.
int scratch_address(void* hip_stream, void** out) {
    int dev = -1;
    hipError_t e = hip_stream ? hipStreamGetDevice((hipStream_t)hip_stream, &dev) : hipGetDevice(&dev);
    if (e != hipSuccess) return fail(FFN_MI355X_EHIP, "device of the stream: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return fail(FFN_MI355X_EINVAL, "device %d out of range", dev);
    void* p = g_scratch[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_scratch_mutex);
        p = g_scratch[dev].load(std::memory_order_relaxed);
        if (!p) {
            int cur = -1;
            if ((e = hipGetDevice(&cur)) != hipSuccess)
                return fail(FFN_MI355X_EHIP, "hipGetDevice: %s", hipGetErrorString(e));
            if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess)
                return fail(FFN_MI355X_EHIP, "hipSetDevice(%d): %s", dev, hipGetErrorString(e));
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            const hipError_t e2 = cur != dev ? hipSetDevice(cur) : hipSuccess;
            if (e != hipSuccess || !p)
                return fail(FFN_MI355X_EHIP, "scratch address on device %d: %s", dev, hipGetErrorString(e));
            if (e2 != hipSuccess)
                return fail(FFN_MI355X_EHIP, "hipSetDevice(%d): %s", cur, hipGetErrorString(e2));
            g_scratch[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return FFN_MI355X_OK;
}

}  // namespace

extern "C" {

int ffn_mi355x_up(const ffn_mi355x_plan* plan, const void* x, const void* w1, void* hidden,
                  void* ws, void* hip_stream) {
    return run_up(plan, x, w1, nullptr, hidden, ws, false, hip_stream);
}

int ffn_mi355x_down(const ffn_mi355x_plan* plan, const void* hidden, const void* w2, void* out,
                    void* ws, void* hip_stream) {
    return run_down(plan, hidden, w2, nullptr, out, ws, false, hip_stream);
}

int ffn_mi355x_run(const ffn_mi355x_plan* plan, const void* x, const void* w1, const void* w2,
                   void* hidden, void* out, void* ws, void* hip_stream) {
    return run_ffn(plan, x, w1, nullptr, w2, nullptr, hidden, out, ws, false, hip_stream);
}

int ffn_mi355x_up_ex(const ffn_mi355x_plan* plan, const void* x, const void* w1, const void* b1, void* hidden,
                     void* ws, void* hip_stream) {
    return run_up(plan, x, w1, b1, hidden, ws, false, hip_stream);
}

int ffn_mi355x_down_ex(const ffn_mi355x_plan* plan, const void* hidden, const void* w2, const void* b2,
                       void* out, void* ws, void* hip_stream) {
    return run_down(plan, hidden, w2, b2, out, ws, false, hip_stream);
}

int ffn_mi355x_run_ex(const ffn_mi355x_plan* plan, const void* x, const void* w1, const void* b1,
                      const void* w2, const void* b2, void* hidden, void* out, void* ws, void* hip_stream) {
    if ((b1 == nullptr) != (b2 == nullptr))
        return fail(FFN_MI355X_EINVAL, "bias1 and bias2 are given together or not at all");
    return run_ffn(plan, x, w1, b1, w2, b2, hidden, out, ws, false, hip_stream);
}

int ffn_mi355x_run_noalloc(const ffn_mi355x_plan* plan, const void* x, const void* w1, const void* w2,
                           void* hidden, void* out, void* hip_stream) {
    if (!valid_plan(plan)) return fail(FFN_MI355X_EINVAL, "invalid plan");
    if (plan->workspace_bytes > (size_t)FFN_MI355X_NOALLOC_SCRATCH_BYTES)
        return fail(FFN_MI355X_EINVAL,
                    "plan needs %zu bytes of workspace, more than the %zu bytes of scratch of "
                    "ffn_mi355x_run_noalloc; run it with ffn_mi355x_run and a workspace",
                    plan->workspace_bytes, (size_t)FFN_MI355X_NOALLOC_SCRATCH_BYTES);
    void* ws = nullptr;
    if (plan->workspace_bytes > 0) {
        const int rc = scratch_address(hip_stream, &ws);
        if (rc != FFN_MI355X_OK) return rc;
    }
    return run_ffn(plan, x, w1, nullptr, w2, nullptr, hidden, out, ws, true, hip_stream);
}

int ffn_mi355x_num_variants(void) { return kNumVariants; }

int ffn_mi355x_variant_refill_waves(int variant) {
    if (variant < 0 || variant >= kNumVariants)
        return fail(FFN_MI355X_EINVAL, "tile variant out of range (0..%d)", kNumVariants - 1);
    ok();
    return kVariants[variant].prod;
}

int ffn_mi355x_variant_mfma_edge(int variant) {
    if (variant < 0 || variant >= kNumVariants)
        return fail(FFN_MI355X_EINVAL, "tile variant out of range (0..%d)", kNumVariants - 1);
    ok();
    return kVariants[variant].mf;
}

int ffn_mi355x_variant_info(int variant, int* bm, int* bn, int* bk, int* waves, int* stages,
                            int* lds_bytes) {
    if (variant < 0 || variant >= kNumVariants)
        return fail(FFN_MI355X_EINVAL, "tile variant out of range (0..%d)", kNumVariants - 1);
    const Variant& v = kVariants[variant];
    if (bm) *bm = v.bm;
    if (bn) *bn = v.bn;
    if (bk) *bk = v.bk;
    if (waves) *waves = v.waves();
    if (stages) *stages = v.stages;
    if (lds_bytes) *lds_bytes = v.lds();
    return ok();
}

const char* ffn_mi355x_last_error(void) { return g_error.c_str(); }

const char* ffn_mi355x_strerror(int code) {
    switch (code) {
        case FFN_MI355X_OK: return "ok";
        case FFN_MI355X_EINVAL: return "invalid argument";
        case FFN_MI355X_ENOT_APPLICABLE: return "not applicable";
        case FFN_MI355X_EUNAVAILABLE: return "unavailable";
        case FFN_MI355X_EHIP: return "HIP runtime error";
        case FFN_MI355X_EDEVICE: return "unsupported device";
        default: return "unknown error";
    }
}

const char* ffn_mi355x_version(void) { return "ffn_mi355x gfx950 " FFN_MI355X_REVISION; }

}  // extern "C"
