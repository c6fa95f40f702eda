// ffn_gemm.hpp -- CDNA4 (gfx950) MFMA GEMM engine behind the fused FFN.
//
// One kernel template serves the three GEMM roles of the FFN
//     up   : hidden[m,h] = GELU( sum_k X[m,k]  * W1[h,k] )   (ops/kernel/ffn.py:207-360, 540-581)
//     down : out[m,n]    =       sum_h hid[m,h] * W2[n,h]     (Basic ops/kernel/ffn.py:377-529,
//                                                              Stream-K ops/kernel/ffn.py:951-1423)
// Both are "NT" products: the two operands are row-major with the reduction
// dimension contiguous, which is exactly what an MFMA lane wants (8 consecutive
// K elements = one 16-byte register quad per lane).
//
// Data path of one macro tile (BM x BN, reduction step BK):
//   HBM/L2 --buffer_load_dwordx4 ... lds--> LDS stage s  (no VGPR staging)
//   LDS --ds_read_b128--> A/B fragments --v_mfma_f32_32x32x16 or 16x16x32_{bf16,f16}--> FP32 acc
// LDS rows are BK*2 bytes; the 16-byte chunk c of row r lives at c ^ ((r / R256) mod CH),
// R256 = rows per 256-byte line of the 64 LDS banks: the 16 lanes of one ds_read_b128 cycle
// (16 consecutive rows, one chunk) then cover all 64 banks exactly once.  That holds for both
// fragment shapes: a 32x32x16 fragment gives lanes 0-31 rows 0-31 and lanes 32-63 the next
// chunk of the same rows, a 16x16x32 fragment gives each 16 lanes rows 0-15 and one of four
// consecutive chunks.  Out-of-range
// rows and the K tail read as zero through the buffer descriptor's range check,
// so tiles may overhang the matrices and no load can leave its buffer.
//
// The MFMA is issued with the weight fragment as operand A and the activation
// fragment as operand B, so an accumulator holds D[n][m]; each lane then owns
// groups of four consecutive n of one row m, which the epilogue packs into 8 bytes and pairs
// across lanes into 16-byte stores.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ffn {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((__vector_size__(16)));
typedef _Float16 f16x8 __attribute__((__vector_size__(16)));
typedef __attribute__((address_space(3))) char lds_char;

enum { DT_F16 = 0, DT_BF16 = 1 };
// Epilogue of a GEMM role: the activation applied to the FP32 sum (plus bias) before the cast.
// EPI_SWIGLU pairs 32-column blocks: block 2k holds gate columns, block 2k+1 the up columns of the
// same 32 hidden columns (the weight rows are interleaved so), and SiLU(gate) * up is stored.
enum { EPI_GELU_ERF = 0, EPI_GELU_RATIONAL = 1, EPI_STORE = 2, EPI_SILU = 3, EPI_SWIGLU = 4 };

// Launch-time description of one GEMM.  All extents are in elements.
struct GemmParams {
    const void* a;        // [M][lda]   activations (X or hidden)
    const void* b;        // [N][ldb]   weights (W1 or W2)
    void* c;              // [M][ldc]   hidden or out
    float* ws;            // Stream-K partial-tile slots (FP32), ws_bytes long
    unsigned* sk_flags;   // per split tile and wave: arrivals of the tile's pieces (zero between launches)
    int sk_stride;        // words from one split tile's counters to the next's (at least the tile waves)
    unsigned ws_bytes;
    int M, N, K;
    int m_valid;          // rows of A holding data; rows [m_valid, M) are zero padding
    int n_valid;          // rows of B holding data; rows [n_valid, N) read as zero
    int lda, ldb, ldc;
    int tiles_m, tiles_n;
    int k_iters;          // ceil(K / BK)
    int dp_tiles;         // tiles [0, dp_tiles) are reduced whole by one workgroup
    int sk_tiles;         // tiles [dp_tiles, dp_tiles + sk_tiles) are split along K
    int sk_q, sk_r;       // split iterations per workgroup: q, plus one for the first r
    int slots_per_wg;     // partial-tile slots owned by each workgroup
    int group_m;          // tile-order swizzle: tiles walk group_m tile-rows column by column
    int fast_dma;         // 1: launch the kernel whose interior tiles refill through the SALU-addressed DMA path
    int rev_m;            // 1: tile rows are walked last-first
    int zero_row0;        // rows [zero_row0, M) of C lie past every tile holding data: written as zeros
    int c_cols;           // columns of C (N, or N / 2 for SwiGLU, whose column pairs make one output)
    const void* bias;     // per-column bias in the storage type, added in FP32 before the activation
    int bias_n;           // bias values present; columns at or past bias_n add zero (NULL bias: none)
    // Gathered rows of A (a strided activation read in place): row r = (i0, i1, i2) in a
    // [d0, a_d1, a_d2] grid starts at element i0*a_s0 + i1*a_s1 + i2*a_s2; K is contiguous and
    // the rows lie within a_bytes of a.  a_gather = 0: row r starts at r*lda.
    int a_gather, a_d1, a_d2, a_s0, a_s1, a_s2;
    unsigned a_bytes;
    // Arrival counters of the FFN's other GEMM (the Stream-K down's, in an up launch; a split up
    // GEMM's, in a down launch), written as zeros ahead of any tile: a counter region left dirty
    // (never cleared, or by an interrupted or overlapping call) is repaired by the launch before
    // the one that counts on it.
    unsigned* clear_words;
    int clear_count;
};

// Counter words of a single-launch FFN (ffn_fused.hip), in the workspace's counter region; zero
// between launches (the last workgroup to leave clears them) but for the error word.  Each
// counter has a 256-byte line of its own (kFusedStride words): atomics on one line are
// serialised, ~11 ns apiece, so with every workgroup's tickets, arrivals and polls on a single
// line each ticket waited ~3 us (256 workgroups, one fetch-add each, measured), against ~0.35 us
// on lines of their own.
//   x * S              ticket queue of XCD x (x < 8)
//   8 * S              workgroups that have left
//   9 * S              error word: set when a down tile gave up waiting for its row block
//   (10 + r) * S       up tiles stored, of up row block r
constexpr int kFusedStride = 64;
constexpr int kFusedLeft = 8 * kFusedStride, kFusedError = 9 * kFusedStride, kFusedReady = 10 * kFusedStride;
struct FusedParams {
    unsigned* ctr;
    int ratio;       // down row blocks per up row block (BM_up / BM_down)
    int spin_limit;  // polls of a row-block counter before a down tile gives up
};

// SYNCQ_: MFMA slot of a stage's last k-step after which the stage wait + barrier is placed
// (-1: end of the first block of B).  DMAKS_: with two stages, the k-steps at the start of an
// iteration carrying the refill DMA (-1: the first half); with more, DMAKS_ equal to the k-steps
// per stage spreads it over the whole iteration.  WGK_: waves along K -- each wave computes its whole
// WTM x WTN wave tile over its own BK/WGK slice of every stage, and the WGK partial tiles are
// summed through LDS after the main loop.
template <int BM_, int BN_, int BK_, int WGM_, int WGN_, int STAGES_, int SYNCQ_ = -1, int DMAKS_ = -1,
          int WGK_ = 1, int DMAW_ = 0, int PROD_ = 0, int EARLY_ = 0, int MF_ = 32>
struct TileCfg {
    static constexpr int BM = BM_, BN = BN_, BK = BK_;
    static constexpr int WGM = WGM_, WGN = WGN_, WGK = WGK_, STAGES = STAGES_;
    static constexpr int SYNCQ = SYNCQ_, DMAKS = DMAKS_;
    static constexpr int NW = WGM * WGN * WGK;     // waves holding wave tiles
    // PROD_ > 0: that many more waves (numbered first) only refill the LDS stages; the NW
    // tile waves then issue no DMA.
    static constexpr int PROD = PROD_;
    static constexpr int NT = (NW + PROD) * 64;    // threads per workgroup
    static constexpr int WTM = BM / WGM, WTN = BN / WGN;  // wave tile
    // MFMA block edge: 32 (v_mfma_f32_32x32x16, 16 accumulators per lane) or 16
    // (v_mfma_f32_16x16x32, 4 per lane).  Same FLOPs per LDS byte for a given wave tile; the
    // 16x16x32 form takes less energy per FLOP, which counts where the clock is held down by
    // the activity of the whole chip.
    static constexpr int MF = MF_;
    static_assert(MF_ == 32 || MF_ == 16, "MFMA blocks are 32x32x16 or 16x16x32");
    static constexpr int KSTEP_K = 512 / MF;       // reduction depth of one MFMA
    static constexpr int FM = WTM / MF, FN = WTN / MF;    // MFMA blocks per wave
    static_assert(MF == 32 || (FM % 2 == 0 && FN % 2 == 0), "16x16 blocks go in pairs");
    static constexpr int ROWB = BK * 2;            // bytes of one LDS row
    static constexpr int CH = ROWB / 16;           // 16-byte chunks per row
    static constexpr int RPB = 1024 / ROWB;        // rows per 1 KiB DMA block (64 lanes x 16 B)
    static constexpr int R256 = (ROWB >= 256) ? 1 : 256 / ROWB; // rows per 256-byte bank line
    // The swizzle of a row depends on (row / R256) mod CH; seen from a 1 KiB DMA block it
    // repeats every SWZ_PERIOD blocks.
    static constexpr int SWZ_PERIOD = (CH * R256 > RPB) ? (CH * R256) / RPB : 1;
    static constexpr int A_BYTES = BM * ROWB, B_BYTES = BN * ROWB;
    static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
    static constexpr int A_BLKS = A_BYTES / 1024, B_BLKS = B_BYTES / 1024;
    // Waves issuing the refill DMA: all of them (DMAW_ = 0) or waves [0, DMAW_).  A workgroup's
    // waves w and w + 4 share a SIMD (HW_REG_HW_ID read back on gfx950), so with eight waves
    // and DMAW_ = 4 every SIMD holds one wave that refills and one that only reads LDS and
    // issues MFMAs: while the first waits on the texture unit, the second keeps the matrix
    // core busy.
    static constexpr int DW = PROD > 0 ? PROD : DMAW_ == 0 ? NW : DMAW_;
    static_assert(PROD == 0 || DMAW_ == 0, "refill-only waves issue the whole refill");
    static constexpr int A_PW = A_BLKS / DW, B_PW = B_BLKS / DW;  // DMA blocks per issuing wave
    static constexpr int LOADS = A_PW + B_PW;      // DMA instructions per issuing wave per stage
    // EARLY_ > 0 (two stages only): the first EARLY_ of an iteration's LOADS go out in the slots
    // after the previous iteration's stage barrier -- the moment the stage they fill is free --
    // instead of in the iteration before the data is used: a full iteration of lead for them.
    static constexpr int EARLY = EARLY_;
    static_assert(EARLY_ == 0 || (STAGES_ == 2 && WGK_ == 1 && EARLY_ < A_PW + B_PW),
                  "early refill: two stages, no K slices, part of the refill");
    static constexpr int LDS_BYTES = STAGES * STAGE_BYTES;
    static constexpr int KSTEPS = BK / KSTEP_K / WGK;  // MFMA k-steps per stage and wave
    // Output staging of the epilogue: from stage STAGES-1 (which the next unit's DMA prologue
    // leaves free) up to EPI_AVAIL bytes.  A workgroup whose stages take more than half of the
    // LDS runs alone on its CU, so it may use all 160 KiB; a smaller one keeps to one stage and
    // does not cut the number of workgroups per CU.  ER output rows are staged at a time: ER/WGM
    // rows of every wave row (whole 32-row blocks), so that every wave writes every chunk.
    static constexpr int LDS_MAX = 160 * 1024;
    static constexpr int EPI_OFF = (STAGES - 1) * STAGE_BYTES;
    static constexpr int EPI_AVAIL = (LDS_BYTES > LDS_MAX / 2) ? LDS_MAX - EPI_OFF : STAGE_BYTES;
    static constexpr int OUT_ROWB = BN * 2;        // bytes of one staged output row (unpadded)
    // The staged rows' chunk XOR keeps a row's 16-byte pieces inside the row only when their
    // number is a power of two; other tile widths store from registers.
    static constexpr bool OUT_POW2 = ((BN / 8) & (BN / 8 - 1)) == 0;
    static constexpr int er_pick() {
        for (int er = BM; er >= 32 * WGM; er /= 2)
            if (BM % er == 0 && (er / WGM) % 32 == 0 && er * OUT_ROWB <= EPI_AVAIL) return er;
        return 0;
    }
    static constexpr int ER = er_pick();
    static constexpr int LDS_ALLOC = (EPI_OFF + ER * OUT_ROWB > LDS_BYTES) ? EPI_OFF + ER * OUT_ROWB : LDS_BYTES;
    // LDS a workgroup allocates at most (a K-sliced tile exchanges its partials through the
    // whole staging area)
    static constexpr int LDS_USE = WGK > 1 ? EPI_OFF + EPI_AVAIL : LDS_ALLOC;
    static_assert(ER > 0, "no output chunk of whole 32-row blocks fits the staging area");
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32");
    static_assert(ROWB % 16 == 0 && CH >= 2, "BK must be a multiple of 16");
    static_assert(BK % (KSTEP_K * WGK) == 0, "every wave takes whole k-steps of a stage");
    static_assert(NW % DW == 0 && A_BLKS % DW == 0 && B_BLKS % DW == 0,
                  "DMA blocks must split evenly over the issuing waves");
    static_assert(MF % (CH * R256) == 0, "fragment rows start on a swizzle period");
    // DMA offset sets a lane keeps: one per block of the swizzle period (at least two)
    static constexpr int NPAR = SWZ_PERIOD > 2 ? SWZ_PERIOD : 2;
    static_assert(SWZ_PERIOD <= 4, "at most four DMA offset sets");
    static_assert(SWZ_PERIOD == 1 || (A_PW % SWZ_PERIOD == 0 && B_PW % SWZ_PERIOD == 0),
                  "the swizzle phase of every DMA instruction must be known at compile time");
    static_assert(LDS_ALLOC <= LDS_MAX && LDS_USE <= LDS_MAX, "gfx950 has 160 KiB of LDS per CU");
};

// ---------------------------------------------------------------------------
// small device helpers
// ---------------------------------------------------------------------------

// Buffer descriptor of `bytes` bytes at `base`; both must be uniform over the wave.  They are
// passed through readfirstlane so the descriptor is built in SGPRs: a descriptor the compiler
// holds in VGPRs costs a waterfall loop (readfirstlane, compare, exec mask, branch) around every
// load that uses it, which also splits the hand-interleaved MFMA schedule into basic blocks.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = (uint64_t)(uintptr_t)base;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
    const int n = __builtin_amdgcn_readfirstlane((int)bytes);
    void* ptr = (void*)(uintptr_t)(((uint64_t)hi << 32) | lo);
    // word3 0x00020000: raw (untyped) 32-bit data format, range-checked against `bytes`
    return __builtin_amdgcn_make_buffer_rsrc(ptr, (short)0, n, 0x00020000);
}

// Device-scope (SC1) 16-byte store and load of FP32 partials.  The eight XCDs have L2 caches of
// their own: an SC1 store is written through to memory and an SC1 load reads past a stale L2
// line, so a partial stored by one XCD and read by another after the arrival counter (below)
// needs no cache writeback or invalidation.  These are the forms an agent-scope atomic store /
// load takes on this target.
constexpr int kCpolDevice = 16;  // SC1
__device__ __forceinline__ void store_coherent(const __amdgpu_buffer_rsrc_t& r, uint32_t off, f32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, (int)off, 0, kCpolDevice);
}
__device__ __forceinline__ f32x4 load_coherent(const __amdgpu_buffer_rsrc_t& r, uint32_t off) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kCpolDevice));
}

// s_waitcnt vmcnt(n) with lgkm/exp counters left alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

template <int DT>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    if constexpr (DT == DT_BF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}
template <int DT>
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    if constexpr (DT == DT_BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}
// accumulator of one MFMA block: 16 FP32 per lane for 32x32, 4 for 16x16
template <int MF>
struct AccOf {
    using type = f32x16;
};
template <>
struct AccOf<16> {
    using type = f32x4;
};

// Bit reinterpretation of one 32-bit value, taken by value: __builtin_bit_cast applied
// directly to an element of an ext_vector_type (v.y, acc[k]) reads element 0 of the vector
// instead, so elements always go through these.
__device__ __forceinline__ float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }
__device__ __forceinline__ uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }

// Round-to-nearest-even FP32 -> storage type, four values packed into 8 bytes; each pair is
// one v_cvt_pk_{bf16,f16}_f32.
template <int DT>
__device__ __forceinline__ u32x2 pack4(float a, float b, float c, float d) {
    const f32x2 lo = {a, b}, hi = {c, d};
    u32x2 r;
    if constexpr (DT == DT_BF16) {
        r.x = __builtin_bit_cast(uint32_t, __builtin_convertvector(lo, bf16x2));
        r.y = __builtin_bit_cast(uint32_t, __builtin_convertvector(hi, bf16x2));
    } else {
        r.x = __builtin_bit_cast(uint32_t, __builtin_convertvector(lo, f16x2));
        r.y = __builtin_bit_cast(uint32_t, __builtin_convertvector(hi, f16x2));
    }
    return r;
}

// ---------------------------------------------------------------------------
// GELU forms (applied to the FP32 accumulator before the cast)
// ---------------------------------------------------------------------------

// Exact-form GELU, z * Phi(z) = 0.5*z*(1+erf(z/sqrt2)) -- F.gelu(approximate='none').
// With h = Phi(-|z|) = 0.5*erfc(|z|/sqrt2), GELU(z) = max(z, 0) - |z|*h for either sign of z
// (z >= 0: z*(1-h); z < 0: z*h), so one max and one FMA replace the sign select, and erfc
// is only ever needed on the non-negative axis, where it has no cancellation.
// erfc uses the form of the Chebyshev fit of Press, Teukolsky, Vetterling & Flannery,
// "Numerical Recipes in C" (2nd ed., sec. 6.2, erfcc):
//     erfc(x) = t*exp(-x*x + P(t)),  t = 1/(1 + x/2),
// with P of degree 5 fitted here (Lawson-reweighted least squares of log(erfc(x)/t) + x^2 in t
// over x in [0, 10.5]; past that erfc is below the FP32 subnormals): relative error 7.6e-6 in
// float64 and 1.1e-5 in FP32 evaluation, forty times below half an fp16 ulp.  (Degree 7 reaches
// 4.6e-6 in FP32, where the rounding of x*x dominates, for two more FMAs per element: 1-3%
// of an up GEMM.)  1/sqrt2, the factor 1/2 of h and the change to base 2 are folded into the
// constants: one v_rcp_f32, one v_exp_f32 and about 10 full-rate VALU ops.  NaN gives NaN,
// as in torch; so do z = +inf (|z| * h is inf * 0; torch gives +inf) and z = -inf (torch: NaN).
__device__ __forceinline__ float gelu_erf(float z) {
    constexpr float L2E = 1.4426950408889634f;                  // log2(e)
    const float a = __builtin_fabsf(z);
    const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(a, 0.35355339059327376f, 1.0f));  // 1/(1+|z|/(2 sqrt2))
    float p = __builtin_fmaf(t, 0.2287914322f * L2E, -0.7091943583f * L2E);
    p = __builtin_fmaf(t, p, 0.4744972994f * L2E);
    p = __builtin_fmaf(t, p, 0.2544409355f * L2E);
    p = __builtin_fmaf(t, p, 1.0180141158f * L2E);
    p = __builtin_fmaf(t, p, -1.2665418100f * L2E - 1.0f);     // -1: the factor 1/2 of h
    const float h = t * __builtin_amdgcn_exp2f(__builtin_fmaf(-a, a * (0.5f * L2E), p));  // -x^2 = -z^2/2
    // max(z, 0) as med3(z, 0, FLT_MAX): no NaN canonicalisation is needed, a NaN z already
    // makes |z| and the result NaN
    return __builtin_fmaf(-a, h, __builtin_amdgcn_fmed3f(z, 0.0f, 3.402823466e38f));
}

// Rational erf GELU: t = clamp(z/sqrt2, +-3.92), erf(t) ~ t*P5(t^2)/Q5(t^2), coefficients and
// operation order of validation/reference.py:5-13 (= ops/kernel/ffn.py:548-572); the division
// is a v_rcp_f32 (1 ulp) and a multiply.
__device__ __forceinline__ float gelu_rational(float z) {
    float t = z * 0.70710678118654752f;
    t = __builtin_fminf(__builtin_fmaxf(t, -3.92f), 3.92f);
    const float t2 = t * t;
    float p = t2 * 0.053443748819f + 7.5517016694f;
    p = p * t2 + 101.62808918f;
    p = p * t2 + 1393.8061484f;
    p = p * t2 + 5063.7915060f;
    p = p * t2 + 29639.384698f;
    p = p * t;
    float q = t2 + 31.212858877f;
    q = q * t2 + 398.56963806f;
    q = q * t2 + 3023.1248150f;
    q = q * t2 + 13243.365831f;
    q = q * t2 + 26267.224157f;
    return (z * 0.5f) * (p * __builtin_amdgcn_rcpf(q) + 1.0f);
}

// SiLU(z) = z / (1 + e^-z) (analysis doc of the EagleFFN baseline, :52-56): one v_exp_f32 and one
// v_rcp_f32.  For z -> -inf, e^-z overflows to inf and the result is -0; for z -> +inf it is z.
__device__ __forceinline__ float silu(float z) {
    constexpr float L2E = 1.4426950408889634f;
    return z * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-z * L2E));
}

template <int EPI>
__device__ __forceinline__ float activate(float z) {
    if constexpr (EPI == EPI_GELU_ERF) return gelu_erf(z);
    else if constexpr (EPI == EPI_GELU_RATIONAL) return gelu_rational(z);
    else if constexpr (EPI == EPI_SILU) return silu(z);
    else return z;
}

// Storage value -> FP32 (exact).
template <int DT>
__device__ __forceinline__ float to_f32(uint32_t bits16) {
    if constexpr (DT == DT_BF16) return __builtin_bit_cast(float, bits16 << 16);
    else return (float)__builtin_bit_cast(_Float16, (unsigned short)bits16);
}

// Bias of columns n..n+3 (n a multiple of 4) in FP32; zero past bias_n.  Only called by the
// epilogue bodies instantiated for a bias (p.bias set): the kernels test p.bias once per tile and
// run a body without bias terms otherwise, so the bias-free epilogue is branch-free.
template <int DT>
__device__ __forceinline__ f32x4 bias4(const GemmParams& p, int n) {
    f32x4 b = {0.0f, 0.0f, 0.0f, 0.0f};
    if (n + 4 <= p.bias_n) {
        const u32x2 w = *(const u32x2*)((const char*)p.bias + (size_t)n * 2);
        b = f32x4{to_f32<DT>(w.x & 0xffffu), to_f32<DT>(w.x >> 16), to_f32<DT>(w.y & 0xffffu),
                  to_f32<DT>(w.y >> 16)};
    } else if (n < p.bias_n) {
        // the last values: element loads, none past the bias
        const unsigned short* e = (const unsigned short*)p.bias + n;
        b.x = to_f32<DT>(e[0]);
        if (n + 1 < p.bias_n) b.y = to_f32<DT>(e[1]);
        if (n + 2 < p.bias_n) b.z = to_f32<DT>(e[2]);
    }
    return b;
}

// tile index -> (tile row, tile column); tiles walk `group_m` tile-rows column by column so
// that consecutive tiles share weight panels (columns) and activation panels (rows).  With
// rev_m the tile rows go last-first: the down GEMM then starts on the hidden rows the up GEMM
// wrote last, the ones most likely still held by the 256 MiB last-level cache.
__device__ __forceinline__ void tile_coords(const GemmParams& p, int t, int& tm, int& tn) {
    const int per_group = p.group_m * p.tiles_n;
    const int gidx = t / per_group;
    const int first_m = gidx * p.group_m;
    const int rows = min(p.tiles_m - first_m, p.group_m);
    const int r = t - gidx * per_group;
    tm = first_m + r % rows;
    tn = r / rows;
    if (p.rev_m) tm = p.tiles_m - 1 - tm;
}

// Split-region bookkeeping: split iteration x (0-based inside the split region) belongs to
// workgroup sk_owner(x); workgroup v starts at sk_start(v).
__host__ __device__ __forceinline__ int sk_owner(const GemmParams& p, int x) {
    if (p.sk_q == 0) return x;
    const int big = (p.sk_q + 1) * p.sk_r;
    if (x < big) return x / (p.sk_q + 1);
    return p.sk_r + (x - big) / p.sk_q;
}
__device__ __forceinline__ int sk_start(const GemmParams& p, int v) {
    return v * p.sk_q + min(v, p.sk_r);
}
__device__ __forceinline__ float* sk_slot(const GemmParams& p, int v, int local, int tile_elems) {
    return p.ws + ((size_t)v * p.slots_per_wg + local) * (size_t)tile_elems;
}

// One unit of work of a workgroup: K-iterations [kb, ke) of tile (tm, tn).  `split` >= 0 marks
// a Stream-K piece of split tile `split` that shares the tile with other workgroups and goes
// to partial slot `local` of this workgroup.
struct Unit {
    int tm, tn, kb, ke;
    int split, local;
    bool valid;
};

// Walks the units of virtual workgroup v: whole tiles v, v+G, ... below dp_tiles, then (for
// Stream-K) its contiguous range of split iterations cut at tile boundaries.
template <bool SK>
struct UnitWalker {
    int G, v, dp_next, it, it_begin, it_end;
    __device__ __forceinline__ UnitWalker(const GemmParams& p, int v_, int G_) : G(G_), v(v_) {
        dp_next = v;
        it_begin = it_end = it = 0;
        if constexpr (SK) {
            it_begin = it = sk_start(p, v);
            it_end = sk_start(p, v + 1);
        }
    }
    __device__ __forceinline__ Unit next(const GemmParams& p) {
        Unit u;
        u.valid = false;
        u.split = -1;
        u.local = 0;
        if (dp_next < p.dp_tiles) {
            tile_coords(p, dp_next, u.tm, u.tn);
            u.kb = 0, u.ke = p.k_iters, u.valid = true;
            dp_next += G;
            return u;
        }
        if constexpr (SK) {
            if (it < it_end) {
                const int kI = p.k_iters;
                const int s = it / kI;
                u.kb = it - s * kI;
                u.ke = min(kI, u.kb + (it_end - it));
                tile_coords(p, p.dp_tiles + s, u.tm, u.tn);
                const bool shared = sk_owner(p, s * kI) != sk_owner(p, s * kI + kI - 1);
                u.split = shared ? s : -1;
                u.local = s - it_begin / kI;
                u.valid = true;
                it += u.ke - u.kb;
            }
        }
        return u;
    }
};

// ---------------------------------------------------------------------------
// the GEMM engine
// ---------------------------------------------------------------------------

// ISSUE: this wave issues its share of the refill DMA (false for the waves at or past C::DW).
// MMA: this wave holds a wave tile (false for the refill waves of a tile with C::PROD > 0).
// Both are the calling wave's roles and have no default: an engine is built only inside
// with_wave_roles (below), which gives every wave the roles of its number.  (The refill blocks
// of wave w are w * A_PW + D: a wave at or past C::DW given ISSUE would address rows past the
// tile, which on the SALU-addressed refill are reads past the operand.)
template <int DT, class C, bool GA, bool ISSUE, bool MMA>
struct Engine {
    static constexpr int FM = C::FM, FN = C::FN, NT = C::NT, S = C::STAGES, KS = C::KSTEPS;
    static constexpr int MF = C::MF;
    static_assert(MF == 16 || KS % 2 == 0, "fragment double-buffer assumes an even number of k-steps per wave");
    using Acc = typename AccOf<MF>::type;
    static constexpr int NQ = MF == 32 ? 4 : 1;  // groups of four accumulators per block
    static constexpr int CPK = C::KSTEP_K / 8;   // 16-byte K chunks of one k-step (2 or 4)
    static constexpr int LSH = MF == 32 ? 5 : 4; // lane >> LSH: this lane's chunk of the k-step

    lds_char* smem;
    int tid, lane, wave, wm, wn, wk;
    int twave;  // index among the tile waves (0 for a refill-only wave)
    int a_row_off, b_row_off;  // per-lane LDS byte offsets of the fragment rows
    int swz;                   // chunk XOR of this lane's fragment rows
    static __device__ __forceinline__ int swz_of(int row) { return (row / C::R256) % C::CH; }

    __device__ __forceinline__ Engine(lds_char* s, const GemmParams& p) : smem(s) {
        tid = threadIdx.x;
        lane = tid & 63;
        wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int tw = MMA ? wave - C::PROD : 0;
        twave = tw;
        wm = tw % C::WGM;
        wn = C::WGK == 1 ? tw / C::WGM : (tw / C::WGM) % C::WGN;
        wk = C::WGK == 1 ? 0 : tw / (C::WGM * C::WGN);
        const int r = lane & (MF - 1);
        a_row_off = (wm * C::WTM + r) * C::ROWB;
        b_row_off = C::A_BYTES + (wn * C::WTN + r) * C::ROWB;
        swz = swz_of(r);
        khalf = CPK * KS * wk + (lane >> LSH);
    }

    __device__ __forceinline__ void rsrc(const GemmParams& p, const Unit& u,
                                         __amdgpu_buffer_rsrc_t& ra, __amdgpu_buffer_rsrc_t& rb) const {
        const int row0 = u.tm * C::BM, col0 = u.tn * C::BN;
        const int lda2 = p.lda * 2, ldb2 = p.ldb * 2;
        const char* abase = (const char*)p.a + (size_t)row0 * (size_t)lda2;
        const char* bbase = (const char*)p.b + (size_t)col0 * (size_t)ldb2;
        // zero-padding rows of A are not fetched: past m_valid the range check returns zeros
        // (gathered rows: the whole operand, rows past m_valid get the zero-fill offset)
        if constexpr (GA) ra = make_rsrc(p.a, p.a_bytes);
        else ra = make_rsrc(abase, (uint32_t)max(0, min(C::BM, p.m_valid - row0)) * (uint32_t)lda2);
        rb = make_rsrc(bbase, (uint32_t)max(0, min(C::BN, p.n_valid - col0)) * (uint32_t)ldb2);
    }

    // Per-lane DMA addressing, computed once per unit.  The lane fills physical chunk pc of
    // row rl of every 1 KiB block, i.e. logical chunk pc ^ swz(row); the swizzle of a block's
    // rows depends only on the block's parity.  a/b: byte offset of that chunk inside a block
    // at K offset 0; kk: its first K element.
    struct DmaLane {
        uint32_t a[C::NPAR], b[C::NPAR];
        int kk[C::NPAR];
        uint32_t ga[GA ? C::A_PW : 1];  // gathered rows: byte offset of each A instruction's chunk
    };
    __device__ __forceinline__ DmaLane dma_lane(const GemmParams& p, const Unit& u) const {
        // from an opaque lane id: the values depend only on the thread and would otherwise be
        // hoisted out of the persistent loop and held (spilled) across the epilogue
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const int rl = ln / C::CH, pc = ln % C::CH;
        DmaLane d;
#pragma unroll
        for (int par = 0; par < C::NPAR; ++par) {
            const int kk = (pc ^ swz_of((par % C::SWZ_PERIOD) * C::RPB + rl)) * 8;
            d.kk[par] = kk;
            d.a[par] = (uint32_t)(rl * p.lda * 2 + kk * 2);
            d.b[par] = (uint32_t)(rl * p.ldb * 2 + kk * 2);
        }
        if constexpr (GA) {
            // the row of each A instruction, decomposed over the gathered grid once per unit
#pragma unroll
            for (int D = 0; D < C::A_PW; ++D) {
                const int r = u.tm * C::BM + ((ISSUE ? wave : 0) * C::A_PW + D) * C::RPB + rl;
                const unsigned i2 = (unsigned)r % (unsigned)p.a_d2, t = (unsigned)r / (unsigned)p.a_d2;
                const unsigned i1 = t % (unsigned)p.a_d1, i0 = t / (unsigned)p.a_d1;
                const unsigned e = i0 * (unsigned)p.a_s0 + i1 * (unsigned)p.a_s1 + i2 * (unsigned)p.a_s2;
                d.ga[D] = r < p.m_valid ? e * 2u + (unsigned)d.kk[D % C::NPAR] * 2u : 0x80000000u;
            }
        }
        return d;
    }
    // Per-iteration scalars: the K byte offset of K-iteration kit, and the number of K elements
    // left from there (0 for an iteration past the unit, whose DMA then reads only zeros).
    struct DmaIt {
        uint32_t k0x2;
        int lim;
        uint32_t e_k0x2;  // the same for the iteration whose early refill (C::EARLY) this one issues
        int e_lim;
    };
    __device__ __forceinline__ DmaIt dma_it(const GemmParams& p, int kit, bool real) const {
        DmaIt t{};
        t.k0x2 = (uint32_t)(kit * C::BK * 2);
        t.lim = real ? p.K - kit * C::BK : 0;
        return t;
    }

    // DMA instruction D (of the LOADS this wave issues per stage) into LDS stage `stage`.  A
    // chunk at or past K (and every chunk of an empty iteration) gets an offset >= 2^31, beyond
    // any range, and reads as zero without a memory access; rows past the operand are out of
    // range of the tile's descriptor.  The whole offset travels in the VGPR operand: the buffer
    // range check covers voffset but not soffset.
    template <int D>
    __device__ __forceinline__ void issue_one(const GemmParams& p, const __amdgpu_buffer_rsrc_t& ra,
                                              const __amdgpu_buffer_rsrc_t& rb, int stage,
                                              const DmaLane& L, const DmaIt& t) const {
        lds_char* st = smem + stage * C::STAGE_BYTES;
        if constexpr (D < C::A_PW) {
            const int blk = wave * C::A_PW + D;
            constexpr int par = D % C::NPAR;
            // (a gathered row past m_valid already holds the zero-fill offset; adding the K
            // offset keeps it at or past 2^31)
            const uint32_t off = L.kk[par] < t.lim
                                     ? (GA ? L.ga[GA ? D : 0] + t.k0x2
                                           : L.a[par] + (uint32_t)blk * (uint32_t)(C::RPB * p.lda * 2) + t.k0x2)
                                     : 0x80000000u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (__attribute__((address_space(3))) void*)(st + blk * 1024), 16, (int)off, 0, 0, 0);
        } else {
            const int blk = wave * C::B_PW + (D - C::A_PW);
            constexpr int par = (D - C::A_PW) % C::NPAR;
            const uint32_t off = L.kk[par] < t.lim
                                     ? L.b[par] + (uint32_t)blk * (uint32_t)(C::RPB * p.ldb * 2) + t.k0x2
                                     : 0x80000000u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rb, (__attribute__((address_space(3))) void*)(st + C::A_BYTES + blk * 1024), 16, (int)off, 0, 0, 0);
        }
    }

    // The same DMA instruction for a full iteration of an interior tile: every row of the tile
    // lies inside its operand and every chunk inside K, so no lane needs the zero-fill offset.
    // The lane's VGPR offset is then a constant of the kernel and the row-block and K offsets
    // travel in soffset (SALU arithmetic only): no vector instruction per DMA, which keeps the
    // VALU out of the MFMA's way.  Every address is in bounds by construction, so this does
    // not rely on the descriptor's range check.
    template <int D>
    __device__ __forceinline__ void issue_one_fast(const GemmParams& p, const __amdgpu_buffer_rsrc_t& ra,
                                                   const __amdgpu_buffer_rsrc_t& rb, int stage,
                                                   const DmaLane& L, const DmaIt& t) const {
        lds_char* st = smem + stage * C::STAGE_BYTES;
        if constexpr (D < C::A_PW) {
            const int blk = wave * C::A_PW + D;
            constexpr int par = D % C::NPAR;
            const uint32_t soff = (uint32_t)blk * (uint32_t)(C::RPB * p.lda * 2) + t.k0x2;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (__attribute__((address_space(3))) void*)(st + blk * 1024), 16, (int)L.a[par], (int)soff, 0, 0);
        } else {
            const int blk = wave * C::B_PW + (D - C::A_PW);
            constexpr int par = (D - C::A_PW) % C::NPAR;
            const uint32_t soff = (uint32_t)blk * (uint32_t)(C::RPB * p.ldb * 2) + t.k0x2;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rb, (__attribute__((address_space(3))) void*)(st + C::A_BYTES + blk * 1024), 16, (int)L.b[par],
                (int)soff, 0, 0);
        }
    }

    template <bool FAST, int D0, int D1>
    __device__ __forceinline__ void issue_range_impl(const GemmParams& p, const __amdgpu_buffer_rsrc_t& ra,
                                                const __amdgpu_buffer_rsrc_t& rb, int stage,
                                                const DmaLane& L, const DmaIt& t) const {
        if constexpr (D0 < D1) {
            if constexpr (FAST) issue_one_fast<D0>(p, ra, rb, stage, L, t);
            else issue_one<D0>(p, ra, rb, stage, L, t);
            issue_range_impl<FAST, D0 + 1, D1>(p, ra, rb, stage, L, t);
        }
    }

    // (gathered rows always take the checked path: the host launches them without FASTK)
    template <bool FAST, int D0, int D1>
    __device__ __forceinline__ void issue_range(const GemmParams& p, const __amdgpu_buffer_rsrc_t& ra,
                                                const __amdgpu_buffer_rsrc_t& rb, int stage,
                                                const DmaLane& L, const DmaIt& t) const {
        if constexpr (ISSUE) issue_range_impl<FAST && !GA, D0, D1>(p, ra, rb, stage, L, t);
    }

    // K-iterations 0..S-2 of a unit go to stages 0..S-2; iteration S-1+it is fetched during
    // iteration it.  A unit shorter than S-1 iterations still issues all S-1 stages (zeros past
    // its end): the epilogue then knows that exactly the last LOADS*(S-1) loads of an issuing
    // wave belong to the next unit, and that every load before them -- the zero fills of the
    // current unit's last iterations included -- has to land before the staging area is
    // written.
    __device__ __forceinline__ void prologue(const GemmParams& p, const Unit& u) const {
        __amdgpu_buffer_rsrc_t ra, rb;
        rsrc(p, u, ra, rb);
        const DmaLane L = dma_lane(p, u);
#pragma unroll
        for (int s = 0; s < S - 1; ++s)
            issue_range<false, 0, C::LOADS>(p, ra, rb, s, L, dma_it(p, u.kb + s, u.kb + s < u.ke));
        // the early part of iteration S-1, whose stage is free too
        if constexpr (C::EARLY > 0)
            issue_range<false, 0, C::EARLY>(p, ra, rb, S - 1, L, dma_it(p, u.kb + S - 1, u.kb + S - 1 < u.ke));
    }
    // loads of an issuing wave's DMA prologue (what the next unit has in flight at its start)
    static constexpr int PRO_LOADS = C::LOADS * (S - 1) + C::EARLY;

    // Fragment registers: A (activation rows) double-buffered across k-steps, B (weight rows)
    // reloaded in place right after its last use, which the j-major MFMA order makes early.
    // SPLIT (16x16x32 blocks): the MFMAs of a k-step go in two halves, each over half of the A
    // fragments (j-major inside a half), so every A and B fragment has its last use well before
    // the end of the k-step and is read again into the same registers right after it.  One
    // buffer of each instead of two for A: the 16-row fragments of a 64x128 wave tile would
    // otherwise hold 64 VGPRs beside the 128 accumulators.
    static constexpr bool SPLIT = MF == 16;
    static_assert(!SPLIT || FM % 2 == 0, "the split order halves the A fragments");
    u32x4 fa[SPLIT ? 1 : 2][FM], fb[FN];

    // byte offset in its row of this lane's 16-byte K chunk for k-step ks of the wave's slice
    int khalf;  // CPK * (first k-step of the wave's slice) + (lane >> LSH)
    __device__ __forceinline__ int frag_chunk(int ks) const {
        return ((CPK * ks + khalf) ^ swz) * 16;
    }
    template <int BUF, int I>
    __device__ __forceinline__ void read_a(int stage, int ks) {
        if constexpr (MMA) {
            const lds_char* st = smem + stage * C::STAGE_BYTES;
            fa[BUF][I] = *(const __attribute__((address_space(3))) u32x4*)(st + a_row_off + I * MF * C::ROWB + frag_chunk(ks));
        }
    }
    template <int J>
    __device__ __forceinline__ void read_b(int stage, int ks) {
        if constexpr (MMA) {
            const lds_char* st = smem + stage * C::STAGE_BYTES;
            fb[J] = *(const __attribute__((address_space(3))) u32x4*)(st + b_row_off + J * MF * C::ROWB + frag_chunk(ks));
        }
    }
    template <int BUF, int I0, int I1>
    __device__ __forceinline__ void read_a_range(int stage, int ks) {
        if constexpr (I0 < I1) {
            read_a<BUF, I0>(stage, ks);
            read_a_range<BUF, I0 + 1, I1>(stage, ks);
        }
    }
    template <int J0, int J1>
    __device__ __forceinline__ void read_b_range(int stage, int ks) {
        if constexpr (J0 < J1) {
            read_b<J0>(stage, ks);
            read_b_range<J0 + 1, J1>(stage, ks);
        }
    }

    __device__ __forceinline__ void barrier() const {
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS reads are done
        __builtin_amdgcn_s_barrier();
    }

    // ---- one k-step, scheduled by hand ------------------------------------------------------
    // The FN*FM MFMAs of A-buffer CB are issued one per slot in j-major order; between them go
    // the fragment reads of the next k-step (MODE 0: same stage; MODE 1: after the stage wait +
    // barrier, k-step 0 of the next stage; MODE 2: after a barrier, the DMA prologue of the
    // next unit) and this slot's share of the refill DMA.  sched_barrier fences keep the
    // compiler from regrouping them: a burst of DMA instructions fills the texture-address FIFO
    // and stalls the in-order issue of the MFMAs behind it.
    static constexpr int NM = FN * FM;
    // slot of the last k-step after whose MFMA the stage wait + barrier is placed: the end of
    // the j = 0 block, from where every B fragment can be reloaded after its last use
    static constexpr int SYNC_Q = C::SYNCQ >= 0 ? C::SYNCQ : SPLIT ? NM / 2 - 1 : FM - 1;
    static_assert(SYNC_Q >= FM - 1 && SYNC_Q < NM, "the barrier may not precede the in-place B reloads");
    // slot of a unit's last k-step after which the barrier and the next unit's DMA prologue go.
    // The split order reads no fragment in that k-step, so they wait for its last MFMA, when no
    // fragment register is live beside the accumulators and the prologue's addressing.
    static constexpr int PRO_Q = SPLIT ? NM - 1 : SYNC_Q;
    // Split order: slot Q of a k-step takes block (slot_j(Q), slot_i(Q)); last_a(i) / last_b(j)
    // is the last slot using A fragment i / B fragment j.
    static constexpr int HS = NM / 2, FMH = FM / 2;
    static constexpr int slot_i(int Q) { return (Q / HS) * FMH + (Q % HS) % FMH; }
    static constexpr int slot_j(int Q) { return (Q % HS) / FMH; }
    static constexpr int last_a(int i) { return (i / FMH) * HS + (FN - 1) * FMH + i % FMH; }
    static constexpr int last_b(int j) { return HS + j * FMH + FMH - 1; }
    // Split order: the fragment reads of slot Q -- fragment X (A for X < FM, B after) is read at
    // max(its last use, FLOOR) -- from `stage`, k-step ks.
    template <int Q, int FLOOR, int X>
    __device__ __forceinline__ void reread_at(int stage, int ks) {
        if constexpr (X < FM + FN) {
            if constexpr (X < FM) {
                if constexpr ((last_a(X) > FLOOR ? last_a(X) : FLOOR) == Q) read_a<0, X>(stage, ks);
            } else {
                if constexpr ((last_b(X - FM) > FLOOR ? last_b(X - FM) : FLOOR) == Q) read_b<X - FM>(stage, ks);
            }
            reread_at<Q, FLOOR, X + 1>(stage, ks);
        }
    }
    // Slots carrying the refill DMA.  DMAKS counts 16-deep steps of K: k-steps of 32x32x16 blocks,
    // halves of 16x16x32 ones.  With two stages the data is waited for at the end of the same
    // iteration, so it goes out in the slots of the first DMAKS * 16 K elements of the iteration
    // (default: the first half).  With more, it is spread over every slot before the stage
    // wait, or (DMAKS covering the whole stage) over every slot of the iteration: the stage
    // wait then also allows the part of this iteration's group issued after it.
    static constexpr bool DMA_ALL = S > 2 && C::DMAKS * 16 == KS * C::KSTEP_K;
    static_assert(S != 2 || C::DMAKS <= 0 || (C::DMAKS * NM * 16) % C::KSTEP_K == 0,
                  "the refill window covers whole slots");
    static constexpr int DMA_SLOTS = (S == 2)  ? (C::DMAKS > 0 ? C::DMAKS * NM * 16 / C::KSTEP_K : KS / 2 * NM)
                                     : DMA_ALL ? KS * NM
                                               : (KS - 1) * NM + SYNC_Q;
    static_assert(DMA_SLOTS >= 1, "at least one slot carries the refill");
    // With two stages the stage wait (before the DMA of slot SYNC_Q of the last k-step) drains
    // every load: a refill issued after it would land unwaited in the stage the next iteration
    // reads.
    static_assert(S != 2 || DMA_SLOTS <= (KS - 1) * NM + SYNC_Q,
                  "two stages: the whole refill must be issued before the stage wait");
    // loads of the current iteration's group issued before the stage wait (after the MFMA and
    // before the DMA of slot SYNC_Q of the last k-step)
    static constexpr int DMA_BEFORE_WAIT =
        DMA_ALL ? ((KS - 1) * NM + SYNC_Q) * C::LOADS / DMA_SLOTS : C::LOADS;
    // outstanding loads allowed at the stage wait: the groups of the S-3 iterations after the
    // one that fetched the next stage, plus this iteration's share so far
    static constexpr int STAGE_WAIT = C::LOADS * (S - 3) + DMA_BEFORE_WAIT;

    template <int Q, int JJ>
    __device__ __forceinline__ void reload_b_at(int stage) {
        if constexpr (JJ < FN) {
            constexpr int last_use = JJ * FM + FM - 1;
            if constexpr ((last_use > SYNC_Q ? last_use : SYNC_Q) == Q) read_b<JJ>(stage, 0);
            reload_b_at<Q, JJ + 1>(stage);
        }
    }

    template <bool FAST, int CB, int MODE, bool DMA, int KSI, int Q>
    __device__ __forceinline__ void slot(const GemmParams& p, Acc (&acc)[FN][FM], int cur, int nxt,
                                         const __amdgpu_buffer_rsrc_t& ra, const __amdgpu_buffer_rsrc_t& rb,
                                         int dma_stage, const DmaLane& L, const DmaIt& o, const Unit& nx) {
        constexpr int j = SPLIT ? slot_j(Q) : Q / FM, i = SPLIT ? slot_i(Q) : Q % FM;
        if constexpr (MMA) {
            if constexpr (MF == 32) acc[j][i] = mfma32<DT>(fb[j], fa[CB][i], acc[j][i]);
            else acc[j][i] = mfma16<DT>(fb[j], fa[0][i], acc[j][i]);
        }
        constexpr int NB = 1 - CB;
        if constexpr (MODE == 0 && SPLIT) {
            // the fragments whose last use in this k-step was this slot, for the next k-step
            reread_at<Q, -1, 0>(cur, KSI + 1);
        } else if constexpr (MODE == 0) {
            // A fragments of the next k-step over the first half of the slots; B fragment j
            // right after its last use (the end of block j)
            constexpr int half = NM / 2 > 0 ? NM / 2 : 1;
            constexpr int a0 = Q * FM / half, a1 = (Q + 1) * FM / half;
            if constexpr (Q < half) read_a_range<NB, a0, (a1 < FM ? a1 : FM)>(cur, KSI + 1);
            if constexpr (i == FM - 1) read_b<j>(cur, KSI + 1);
        } else {
            if constexpr (MODE == 1 && Q == SYNC_Q) {
                // every wave's DMA of the next stage has landed; every wave is done with the
                // stage the next refill overwrites
                wait_vmcnt<(S == 2 ? 0 : STAGE_WAIT)>();
                barrier();
            } else if constexpr (MODE == 2 && Q == PRO_Q) {
                if (nx.valid) {
                    barrier();
                    prologue(p, nx);
                }
            }
            if constexpr (MODE == 1 && Q >= SYNC_Q) {
                constexpr int span = NM - SYNC_Q, qq = Q - SYNC_Q;
                if constexpr (SPLIT) {
                    // each fragment once both its last use and the barrier are behind
                    reread_at<Q, SYNC_Q, 0>(nxt, 0);
                } else {
                    constexpr int a0 = qq * FM / span, a1 = (qq + 1) * FM / span;
                    read_a_range<NB, a0, a1>(nxt, 0);
                    // B fragment jj is reloaded once both its last use (the end of block jj)
                    // and the barrier are behind
                    reload_b_at<Q, 0>(nxt);
                }
                // the stage this iteration read is free: the early part of the iteration after
                // next goes into it (range-checked: that iteration may be a K tail or past the
                // unit, which reads zeros)
                if constexpr (C::EARLY > 0 && DMA) {
                    constexpr int e0 = qq * C::EARLY / span, e1 = (qq + 1) * C::EARLY / span;
                    issue_range<false, e0, e1>(p, ra, rb, cur, L, DmaIt{o.e_k0x2, o.e_lim, 0u, 0});
                }
            }
        }
        constexpr int g = KSI * NM + Q;  // this slot's share of the refill DMA (the loads past the early part)
        if constexpr (DMA && g < DMA_SLOTS && (DMA_ALL || KSI + 1 < KS || Q < SYNC_Q)) {
            constexpr int t0 = C::EARLY + g * (C::LOADS - C::EARLY) / DMA_SLOTS;
            constexpr int t1 = C::EARLY + (g + 1) * (C::LOADS - C::EARLY) / DMA_SLOTS;
            issue_range<FAST, t0, t1>(p, ra, rb, dma_stage, L, o);
        }
        __builtin_amdgcn_sched_barrier(0);
    }

    template <bool FAST, int CB, int MODE, bool DMA, int KSI, int Q>
    __device__ __forceinline__ void slots(const GemmParams& p, Acc (&acc)[FN][FM], int cur, int nxt,
                                          const __amdgpu_buffer_rsrc_t& ra, const __amdgpu_buffer_rsrc_t& rb,
                                          int dma_stage, const DmaLane& L, const DmaIt& o, const Unit& nx) {
        if constexpr (Q < NM) {
            slot<FAST, CB, MODE, DMA, KSI, Q>(p, acc, cur, nxt, ra, rb, dma_stage, L, o, nx);
            slots<FAST, CB, MODE, DMA, KSI, Q + 1>(p, acc, cur, nxt, ra, rb, dma_stage, L, o, nx);
        }
    }

    template <bool FAST, bool LAST, int KSI>
    __device__ __forceinline__ void ksteps(const GemmParams& p, const Unit& nx,
                                           const __amdgpu_buffer_rsrc_t& ra,
                                           const __amdgpu_buffer_rsrc_t& rb, int cur, int dstage,
                                           const DmaLane& L, const DmaIt& o, Acc (&acc)[FN][FM]) {
        if constexpr (KSI < KS) {
            constexpr int MODE = (KSI + 1 < KS) ? 0 : (LAST ? 2 : 1);
            const int nxt = (cur + 1 == S) ? 0 : cur + 1;
            // the last iteration of a unit refills nothing (its DMA prologue for the next unit
            // is issued after the barrier of its last k-step)
            slots<FAST, KSI & 1, MODE, !LAST, KSI, 0>(p, acc, cur, nxt, ra, rb, dstage, L, o, nx);
            ksteps<FAST, LAST, KSI + 1>(p, nx, ra, rb, cur, dstage, L, o, acc);
        }
    }

    // One iteration `it` of a unit that refills stage cur-1 with iteration it+S-1 (zeros past
    // the unit), then advances cur.
    template <bool FAST>
    __device__ __forceinline__ void step(const GemmParams& p, const Unit& u, const Unit& nx,
                                         const __amdgpu_buffer_rsrc_t& ra, const __amdgpu_buffer_rsrc_t& rb,
                                         const DmaLane& L, Acc (&acc)[FN][FM], int& cur, int it, int n) {
        const int dkit = it + S - 1;
        DmaIt o = dma_it(p, u.kb + dkit, FAST || dkit < n);
        if constexpr (C::EARLY > 0) {
            const DmaIt e = dma_it(p, u.kb + dkit + 1, dkit + 1 < n);
            o.e_k0x2 = e.k0x2, o.e_lim = e.lim;
        }
        const int dstage = (cur == 0) ? S - 1 : cur - 1;
        ksteps<FAST, false, 0>(p, nx, ra, rb, cur, dstage, L, o, acc);
        cur = (cur + 1 == S) ? 0 : cur + 1;
    }

    // acc = sum over K-iterations [u.kb, u.ke) of tile (u.tm, u.tn).  On entry the DMA prologue
    // of the unit is in flight (behind the previous unit's stores but for the first unit), and
    // the first wait takes stage 0 (first unit) or drains everything.  Iteration it fetches iteration it+S-1 into the stage freed at the end
    // of it-1; past the end of the unit it issues the same DMA with out-of-range offsets
    // (zeros into the free stage), which keeps every stage wait a compile-time count.  The
    // last iteration starts the DMA prologue of `nx`, which then overlaps this unit's epilogue.
    // `first`: the workgroup's first unit, whose DMA prologue has no stores behind it; its first
    // iteration then waits for stage 0 alone instead of the whole prologue.  (Behind a later
    // unit's prologue lie the previous unit's output stores, which the load count cannot
    // order against, so that unit waits for everything.)
    template <bool FASTK>
    __device__ __forceinline__ void mainloop(const GemmParams& p, const Unit& u, const Unit& nx,
                                             Acc (&acc)[FN][FM], bool first = false) {
        if constexpr (MMA) {
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int i = 0; i < FM; ++i) acc[j][i] = Acc{};
        }
        __amdgpu_buffer_rsrc_t ra, rb;
        rsrc(p, u, ra, rb);
        const DmaLane L = dma_lane(p, u);
        const int n = u.ke - u.kb;
        if (first) wait_vmcnt<C::LOADS * (S - 2) + C::EARLY>();
        else wait_vmcnt<0>();
        barrier();
        read_a_range<0, 0, FM>(0, 0);
        read_b_range<0, FN>(0, 0);
        // In a FASTK kernel, iterations whose refill targets a full K-iteration of an interior
        // tile take the fast DMA path; the K tail, the zero-fill past the unit and edge tiles
        // take the checked one.  (A kernel without FASTK carries the checked loop alone: the
        // second loop body would raise its scalar register pressure.)
        int cur = 0, it = 0;
        if constexpr (FASTK) {
            const bool interior = (u.tm + 1) * C::BM <= p.m_valid && (u.tn + 1) * C::BN <= p.n_valid;
            const int fast_end = interior ? max(0, min(n, p.K / C::BK - u.kb) - (S - 1)) : 0;
            for (; it < fast_end && it < n - 1; ++it) step<true>(p, u, nx, ra, rb, L, acc, cur, it, n);
        }
        for (; it < n - 1; ++it) step<false>(p, u, nx, ra, rb, L, acc, cur, it, n);
        ksteps<false, true, 0>(p, nx, ra, rb, cur, 0, L, DmaIt{0u, 0, 0u, 0}, acc);
    }

    // ---- epilogue through LDS --------------------------------------------------------------
    // The accumulators of a lane cover 4 consecutive columns of 16 different rows, so storing
    // them directly writes every 128-byte output line in eight 16-byte pieces spread over time,
    // which the memory side pays for dearly.  Instead the tile is activated and cast in
    // registers, written into the staging area ER rows at a time, and copied out with full-row
    // 16-byte-per-lane stores.  Staged rows are unpadded; the 16-byte chunk c of staged row s
    // sits at c ^ ((s / RPW) mod OSWZ), RPW = rows per 256-byte bank line, which spreads the
    // 32 rows of one ds_write_b64 and the chunks of one ds_read_b128 over all 64 banks.
    static constexpr int ER = C::ER;
    static constexpr int ERW = ER / C::WGM;              // rows of each wave row per chunk
    static constexpr int BPC = ERW / 32;                 // 32-row blocks of a wave per chunk
    static constexpr int NCH = C::BM / ER;               // chunks per tile
    static constexpr int TPR = C::BN / 8;                // 16-byte pieces per output row
    static constexpr int RPW = C::OUT_ROWB >= 256 ? 1 : 256 / C::OUT_ROWB;
    static constexpr int OSWZ = TPR < 16 ? TPR : 16;
    static constexpr int PIECES = ER * TPR / NT;         // pieces per thread per chunk
    static constexpr int PB = PIECES < 8 ? PIECES : 8;   // pieces in flight per thread
    static_assert(BPC >= 1 && FM % BPC == 0, "whole blocks per chunk");

    static __device__ __forceinline__ int out_off(int s, int ch) {
        return s * C::OUT_ROWB + ((ch ^ ((s / RPW) % OSWZ)) << 4);
    }

    // Activate and cast the blocks of chunk c in registers: group (j, i, q) packs into words
    // 2q, 2q+1 of acc[j][i], whose sources are already consumed.
    template <int EPI, bool BIAS>
    __device__ __forceinline__ void activate_chunk(const GemmParams& p, const Unit& u, int c,
                                                   Acc (&acc)[FN][FM]) const {
        const int bcol = u.tn * C::BN + wn * C::WTN + 4 * (lane >> 5);
#pragma unroll
        for (int ib = 0; ib < BPC; ++ib) {
            const int i = c * BPC + ib;
#pragma unroll
            for (int j = 0; j < FN; ++j) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const u32x2 v = out4<EPI, BIAS>(p, acc[j][i], q, bcol + 32 * j + 8 * q);
                    acc[j][i][2 * q] = u2f(v.x);
                    acc[j][i][2 * q + 1] = u2f(v.y);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }

    template <int EPI>
    __device__ __forceinline__ void store_tile_lds(const GemmParams& p, const Unit& u, bool next,
                                                   Acc (&acc)[FN][FM]) {
        if (p.bias) store_tile_lds_as<EPI, true>(p, u, next, acc);
        else store_tile_lds_as<EPI, false>(p, u, next, acc);
    }
    template <int EPI, bool BIAS>
    __device__ __forceinline__ void store_tile_lds_as(const GemmParams& p, const Unit& u, bool next,
                                                      Acc (&acc)[FN][FM]) {
        static_assert(C::OUT_POW2, "the staging swizzle needs a power-of-two number of pieces per row");
        static_assert((ER * TPR) % NT == 0, "chunk pieces split evenly over the threads");
        static_assert(C::EARLY == 0, "the next unit's early refill fills part of the staging stage");
        static_assert(C::MF == 32, "the staged epilogue moves 32x32 blocks");
        lds_char* eb = smem + C::EPI_OFF;
        // DMA still in flight may target any stage but the next unit's prologue (issued last):
        // drain it; the barrier before the first staging write makes sure every wave has
        if (next) wait_vmcnt<PRO_LOADS>();
        else wait_vmcnt<0>();
        const int row0 = u.tm * C::BM, col0 = u.tn * C::BN;
        // opaque copies: the addressing below depends only on the thread id, and would
        // otherwise be hoisted out of the persistent loop and held (spilled) across it
        int ln = lane, td = tid;
        asm volatile("" : "+v"(ln));
        asm volatile("" : "+v"(td));
        activate_chunk<EPI, BIAS>(p, u, 0, acc);
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            barrier();
            // staged row of this lane's rows in block (c*BPC + ib): wave row wm, local row
            const int sr = wm * ERW + (ln & 31);
#pragma unroll
            for (int ib = 0; ib < BPC; ++ib) {
                const int i = c * BPC + ib;
                const int s = sr + ib * 32;
#pragma unroll
                for (int j = 0; j < FN; ++j) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int nt = wn * C::WTN + 32 * j + 8 * q + 4 * (ln >> 5);
                        u32x2 v;
                        v.x = f2u(acc[j][i][2 * q]);
                        v.y = f2u(acc[j][i][2 * q + 1]);
                        *(__attribute__((address_space(3))) unsigned long long*)(eb + out_off(s, nt >> 3) + (nt & 7) * 2) =
                            __builtin_bit_cast(unsigned long long, v);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            barrier();
            // copy-out of chunk c in batches of PB pieces: the LDS reads of a batch go first
            // (with the next chunk's activation behind the first batch), then its stores
#pragma unroll
            for (int k0 = 0; k0 < PIECES; k0 += PB) {
                u32x4 v[PB];
#pragma unroll
                for (int k = 0; k < PB; ++k) {
                    const int idx = (k0 + k) * NT + td;
                    const int s = idx / TPR, ch = idx - s * TPR;
                    v[k] = *(const __attribute__((address_space(3))) u32x4*)(eb + out_off(s, ch));
                }
                __builtin_amdgcn_sched_barrier(0);
                if (k0 == 0 && c + 1 < NCH) activate_chunk<EPI, BIAS>(p, u, c + 1, acc);
#pragma unroll
                for (int k = 0; k < PB; ++k) {
                    const int idx = (k0 + k) * NT + td;
                    const int s = idx / TPR, ch = idx - s * TPR;
                    const int gm = row0 + (s / ERW) * C::WTM + c * ERW + (s % ERW), gn = col0 + ch * 8;
                    if (gm < p.M && gn < p.c_cols)
                        *(u32x4*)((char*)p.c + ((size_t)gm * (size_t)p.ldc + (size_t)gn) * 2) = v[k];
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }

    // ---- epilogue straight from registers --------------------------------------------------
    // Group q of a lane holds columns 8q + 4h + 0..3 of row (lane & 31), h = lane >> 5.  One
    // v_permlane32_swap per word exchanges the high-lane words of group 2p with the low-lane
    // words of group 2p+1, after which lane l < 32 holds columns 16p + 0..7 and lane l + 32
    // columns 16p + 8..15 of the same row: every 32x32 block leaves in two 16-byte stores per
    // lane (32 rows x 32 contiguous bytes per instruction), with no LDS round trip and no
    // barrier, so the next unit's main loop starts as soon as the stores are issued.  Row
    // blocks [I0, I1) of the wave tile are stored.
    // Bias (if any) added to acc's columns: group q of block j holds columns
    // col0 + 32j + 8q + 4h + 0..3 of the tile, h = lane >> 5.
    template <int EPI, bool BIAS>
    __device__ __forceinline__ u32x2 out4(const GemmParams& p, const Acc& a, int q, int col) const {
        if constexpr (BIAS) {
            const f32x4 b = bias4<DT>(p, col);
            return pack4<DT>(activate<EPI>(a[4 * q] + b.x), activate<EPI>(a[4 * q + 1] + b.y),
                             activate<EPI>(a[4 * q + 2] + b.z), activate<EPI>(a[4 * q + 3] + b.w));
        } else {
            return pack4<DT>(activate<EPI>(a[4 * q]), activate<EPI>(a[4 * q + 1]), activate<EPI>(a[4 * q + 2]),
                             activate<EPI>(a[4 * q + 3]));
        }
    }
    // SwiGLU: SiLU(gate + its bias) * (up + its bias) of the matching groups of a block pair.
    template <bool BIAS>
    __device__ __forceinline__ u32x2 swiglu4(const GemmParams& p, const Acc& g, const Acc& up, int q,
                                             int gcol, int ucol) const {
        f32x4 bg = {0.0f, 0.0f, 0.0f, 0.0f}, bu = bg;
        if constexpr (BIAS) bg = bias4<DT>(p, gcol), bu = bias4<DT>(p, ucol);
        return pack4<DT>(silu(g[4 * q] + bg.x) * (up[4 * q] + bu.x), silu(g[4 * q + 1] + bg.y) * (up[4 * q + 1] + bu.y),
                         silu(g[4 * q + 2] + bg.z) * (up[4 * q + 2] + bu.z),
                         silu(g[4 * q + 3] + bg.w) * (up[4 * q + 3] + bu.w));
    }
    // Lanes l and l + 32 hold the two 16-byte halves of 16 consecutive output columns after one
    // v_permlane32_swap per word; n0 is the first output column of the lane's 32-column block.
    __device__ __forceinline__ void store_block(const GemmParams& p, char* row, int m, int n0, const u32x2 (&g)[4]) const {
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
            const auto s0 = __builtin_amdgcn_permlane32_swap(g[2 * pp].x, g[2 * pp + 1].x, false, false);
            const auto s1 = __builtin_amdgcn_permlane32_swap(g[2 * pp].y, g[2 * pp + 1].y, false, false);
            const u32x4 v = {(uint32_t)s0[0], (uint32_t)s1[0], (uint32_t)s0[1], (uint32_t)s1[1]};
            const int n = n0 + 16 * pp;
            if (m < p.M && n < p.c_cols) *(u32x4*)(row + (size_t)n * 2) = v;
        }
    }
    template <int EPI, int I0 = 0, int I1 = FM>
    __device__ __forceinline__ void store_tile_regs(const GemmParams& p, const Unit& u,
                                                    Acc (&acc)[FN][FM]) const {
        static_assert(0 <= I0 && I0 <= I1 && I1 <= FM, "accumulator block rows");
        if constexpr (MF == 16) {
            if (p.bias) store_tile_regs16_as<EPI, I0, I1, true>(p, u, acc);
            else store_tile_regs16_as<EPI, I0, I1, false>(p, u, acc);
        } else {
            if (p.bias) store_tile_regs_as<EPI, I0, I1, true>(p, u, acc);
            else store_tile_regs_as<EPI, I0, I1, false>(p, u, acc);
        }
    }
    // 16x16 blocks: lane l holds columns 4g..4g+3 (g = l >> 4) of row l & 15 of every block.
    // For two blocks X and Y of a row, one v_permlane16_swap per word (lanes of 16-lane row 2r+1
    // of X trade with those of row 2r of Y) leaves each lane 8 consecutive columns of one block:
    // lanes of rows 0 and 2 columns 0-7 and 8-15 of X, rows 1 and 3 the same of Y.  n is the
    // lane's first output column after the swap.
    __device__ __forceinline__ void store_pair16(const GemmParams& p, char* row, int m, int n, u32x2 x, u32x2 y) const {
        const auto s0 = __builtin_amdgcn_permlane16_swap(x.x, y.x, false, false);
        const auto s1 = __builtin_amdgcn_permlane16_swap(x.y, y.y, false, false);
        const u32x4 v = {(uint32_t)s0[0], (uint32_t)s1[0], (uint32_t)s0[1], (uint32_t)s1[1]};
        if (m < p.M && n < p.c_cols) *(u32x4*)(row + (size_t)n * 2) = v;
    }
    // Block rows [I0, I1) of the wave tile, 16x16 blocks.
    template <int EPI, int I0, int I1, bool BIAS>
    __device__ __forceinline__ void store_tile_regs16_as(const GemmParams& p, const Unit& u,
                                                         Acc (&acc)[FN][FM]) const {
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const int g = ln >> 4;
        const int m0 = u.tm * C::BM + wm * C::WTM + (ln & 15);
        const int col0 = u.tn * C::BN + wn * C::WTN;   // first column of the wave tile
        const int bcol = col0 + 4 * g;                  // the lane's bias columns in block 0
        const int scol = 16 * (g & 1) + 8 * (g >> 1);   // its 8 columns of a block pair after the swap
#pragma unroll
        for (int i = I0; i < I1; ++i) {
            const int m = m0 + 16 * i;
            char* row = (char*)p.c + (size_t)m * (size_t)p.ldc * 2;
            if constexpr (EPI == EPI_SWIGLU) {
                // gate columns 64k + 0..31 are blocks 4k, 4k+1, their up columns blocks 4k+2, 4k+3
                static_assert(FN % 4 == 0, "SwiGLU pairs the 32-column groups of a wave tile");
#pragma unroll
                for (int k = 0; k < FN / 4; ++k) {
                    const u32x2 x = swiglu4<BIAS>(p, acc[4 * k][i], acc[4 * k + 2][i], 0, bcol + 64 * k,
                                                  bcol + 64 * k + 32);
                    const u32x2 y = swiglu4<BIAS>(p, acc[4 * k + 1][i], acc[4 * k + 3][i], 0, bcol + 64 * k + 16,
                                                  bcol + 64 * k + 48);
                    store_pair16(p, row, m, col0 / 2 + 32 * k + scol, x, y);
                    __builtin_amdgcn_sched_barrier(0);
                }
            } else {
#pragma unroll
                for (int k = 0; k < FN / 2; ++k) {
                    const u32x2 x = out4<EPI, BIAS>(p, acc[2 * k][i], 0, bcol + 32 * k);
                    const u32x2 y = out4<EPI, BIAS>(p, acc[2 * k + 1][i], 0, bcol + 32 * k + 16);
                    store_pair16(p, row, m, col0 + 32 * k + scol, x, y);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
    }
    template <int EPI, int I0, int I1, bool BIAS>
    __device__ __forceinline__ void store_tile_regs_as(const GemmParams& p, const Unit& u,
                                                       Acc (&acc)[FN][FM]) const {
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const int m0 = u.tm * C::BM + wm * C::WTM + (ln & 31);
        const int col0 = u.tn * C::BN + wn * C::WTN;  // first column of the wave tile
        const int bcol = col0 + 4 * (ln >> 5);         // bias column of group q = 0, block 0
#pragma unroll
        for (int i = I0; i < I1; ++i) {
            const int m = m0 + 32 * i;
            char* row = (char*)p.c + (size_t)m * (size_t)p.ldc * 2;
            if constexpr (EPI == EPI_SWIGLU) {
                static_assert(FN % 2 == 0, "SwiGLU pairs the 32-column blocks of a wave tile");
#pragma unroll
                for (int k = 0; k < FN / 2; ++k) {
                    u32x2 g[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        g[q] = swiglu4<BIAS>(p, acc[2 * k][i], acc[2 * k + 1][i], q, bcol + 64 * k + 8 * q,
                                             bcol + 64 * k + 32 + 8 * q);
                    store_block(p, row, m, col0 / 2 + 32 * k + 8 * (ln >> 5), g);
                    __builtin_amdgcn_sched_barrier(0);
                }
            } else {
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    u32x2 g[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) g[q] = out4<EPI, BIAS>(p, acc[j][i], q, bcol + 32 * j + 8 * q);
                    store_block(p, row, m, col0 + 32 * j + 8 * (ln >> 5), g);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
    }

    // ---- epilogue of a K-sliced tile (two waves along K) ------------------------------------
    // The two slices of a wave tile hold FP32 partial sums over the two halves of every stage.
    // Slice WK owns row blocks [WK*IH, (WK+1)*IH) (all j).  Each slice writes the blocks its
    // partner owns into the free stage(s) in register order -- 16-byte group q of block b at
    // ((b*NQ + q)*64 + lane)*16 of the wave's area, so every ds_write_b128 / ds_read_b128 is one
    // contiguous 1 KiB -- the partner adds them to its own, and each slice then activates,
    // casts and stores its blocks from registers.  A sum of two FP32 terms does not depend on
    // which slice adds, so the result is bit-reproducible.  The exchange goes in phases of XB
    // blocks per wave when the area is smaller than the blocks to send.  With an odd number of
    // row blocks (a single one: 32-row wave tiles) slice 0 owns them all, slice 1 only sends.
    static constexpr int OWN0 = FM % 2 == 0 ? FM / 2 : FM;  // row blocks [0, OWN0) of slice 0
    static constexpr int own_rows(int wk) { return wk == 0 ? OWN0 : FM - OWN0; }
    static constexpr int own_base(int wk) { return wk == 0 ? 0 : OWN0; }
    static constexpr int XMAX = FN * (OWN0 > FM - OWN0 ? OWN0 : FM - OWN0);  // most blocks a wave sends
    static constexpr int XPW = C::EPI_AVAIL / C::NW;      // exchange bytes per wave
    static constexpr int XBLK = NQ * 1024;                // exchange bytes of one block
    static constexpr int XB = XPW / XBLK < XMAX ? XPW / XBLK : XMAX;  // blocks per phase
    static_assert(C::WGK == 1 || (C::WGK == 2 && XB >= 1),
                  "K slicing: two slices, room for one block per wave");

    // Block b (0-based) of the ROWS x FN blocks owned by a slice whose rows start at BASE: row
    // block BASE + b % ROWS, column block b / ROWS.
    template <int ROWS, int BASE, int B0, int B1>
    __device__ __forceinline__ void xsend(lds_char* area, Acc (&acc)[FN][FM]) const {
        if constexpr (B0 < B1) {
            constexpr int j = B0 / ROWS, i = BASE + B0 % ROWS, sl = B0 % XB;
#pragma unroll
            for (int q = 0; q < NQ; ++q)
                *(__attribute__((address_space(3))) f32x4*)(area + ((sl * NQ + q) * 64 + lane) * 16) =
                    f32x4{acc[j][i][4 * q], acc[j][i][4 * q + 1], acc[j][i][4 * q + 2], acc[j][i][4 * q + 3]};
            xsend<ROWS, BASE, B0 + 1, B1>(area, acc);
        }
    }
    template <int ROWS, int BASE, int B0, int B1>
    __device__ __forceinline__ void xrecv(const lds_char* area, Acc (&acc)[FN][FM]) const {
        if constexpr (B0 < B1) {
            constexpr int j = B0 / ROWS, i = BASE + B0 % ROWS, sl = B0 % XB;
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                const f32x4 v = *(const __attribute__((address_space(3))) f32x4*)(area + ((sl * NQ + q) * 64 + lane) * 16);
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[j][i][4 * q + c] += v[c];
            }
            xrecv<ROWS, BASE, B0 + 1, B1>(area, acc);
        }
    }
    static constexpr int clampb(int v, int hi) { return v < hi ? v : hi; }
    template <int WK, int PH>
    __device__ __forceinline__ void xphases(Acc (&acc)[FN][FM]) const {
        if constexpr (PH * XB < XMAX) {
            // this slice sends the partner's blocks and receives its own; both lists run in
            // phases of XB blocks (every wave passes the same barriers, also with nothing to send)
            constexpr int PK = 1 - WK;
            constexpr int nsend = FN * own_rows(PK), nrecv = FN * own_rows(WK);
            constexpr int b0 = PH * XB, b1 = (PH + 1) * XB;
            const int partner = twave + (WK == 0 ? 1 : -1) * C::WGM * C::WGN;
            if constexpr (PH > 0) barrier();  // the partner has read the previous phase
            xsend<(own_rows(PK) > 0 ? own_rows(PK) : 1), own_base(PK), clampb(b0, nsend), clampb(b1, nsend)>(
                smem + C::EPI_OFF + twave * XPW, acc);
            barrier();
            xrecv<(own_rows(WK) > 0 ? own_rows(WK) : 1), own_base(WK), clampb(b0, nrecv), clampb(b1, nrecv)>(
                smem + C::EPI_OFF + partner * XPW, acc);
            xphases<WK, PH + 1>(acc);
        }
    }
    template <int EPI, int WK>
    __device__ __forceinline__ void store_sliced_as(const GemmParams& p, const Unit& u, bool next,
                                                    Acc (&acc)[FN][FM]) {
        // DMA still in flight may target any stage but the next unit's prologue (issued last):
        // drain it; the barrier makes sure every wave has before the area is written
        if (next) wait_vmcnt<PRO_LOADS>();
        else wait_vmcnt<0>();
        barrier();
        xphases<WK, 0>(acc);
        store_tile_regs<EPI, own_base(WK), own_base(WK) + own_rows(WK)>(p, u, acc);
    }
    // A refill-only wave's share of store_sliced: the same drain and the same barriers (one
    // before the exchange, then those of xphases: two per phase but the first), no data.
    template <int PH>
    __device__ __forceinline__ void xphase_barriers() const {
        if constexpr (PH * XB < XMAX) {
            if constexpr (PH > 0) barrier();
            barrier();
            xphase_barriers<PH + 1>();
        }
    }
    __device__ __forceinline__ void store_sliced_sync(bool next) const {
        if (next) wait_vmcnt<PRO_LOADS>();
        else wait_vmcnt<0>();
        barrier();
        xphase_barriers<0>();
    }
    template <int EPI>
    __device__ __forceinline__ void store_sliced(const GemmParams& p, const Unit& u, bool next,
                                                 Acc (&acc)[FN][FM]) {
        // one static body per slice (acc is dead after either)
        if (wk == 0) store_sliced_as<EPI, 0>(p, u, next, acc);
        else store_sliced_as<EPI, 1>(p, u, next, acc);
    }

    // FP32 partial tile in the accumulator's own register order: group (j, i, q) of logical
    // thread t lives at ((j*FM + i)*NQ + q)*NTL + t (16-byte units), so every store is coalesced.
    // t is the thread's index among the WGM x WGN tile waves of one K slice, NTL their thread
    // count: a K-sliced tile first sums its slices (the exchange above) and each slice then
    // writes the row blocks [I0, I1) it owns.  (Refill-only waves, numbered first, hold none.)
    static constexpr int NTL = C::NW * 64 / C::WGK;
    __device__ __forceinline__ int slice_thread() const { return tid - C::PROD * 64 - wk * NTL; }
    static __device__ __forceinline__ uint32_t part_off(int idx, int t) { return (uint32_t)(idx * NTL + t) * 16u; }
    template <int I0 = 0, int I1 = FM>
    __device__ __forceinline__ void store_partial(const __amdgpu_buffer_rsrc_t& r, uint32_t slot_off,
                                                  Acc (&acc)[FN][FM]) const {
        static_assert(0 <= I0 && I0 <= I1 && I1 <= FM, "accumulator block rows");
        const int t = slice_thread();
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int i = I0; i < I1; ++i)
#pragma unroll
                for (int q = 0; q < NQ; ++q) {
                    const int idx = (j * FM + i) * NQ + q;
                    const f32x4 v = {acc[j][i][4 * q], acc[j][i][4 * q + 1], acc[j][i][4 * q + 2],
                                     acc[j][i][4 * q + 3]};
                    store_coherent(r, slot_off + part_off(idx, t), v);
                    if (q == NQ - 1) __builtin_amdgcn_sched_barrier(0);
                }
    }

    // Adds the partials of `c` pieces (slot byte offsets so[0..c), c <= PC, in K order) to the
    // wave's positions, the first replacing them when `set`.  The loads of all c pieces (and,
    // the blocks being unrolled, of several blocks) are in flight together; the sums are taken
    // one piece after another.
    template <int PC, int I0, int I1>
    __device__ __forceinline__ void add_pieces(const __amdgpu_buffer_rsrc_t& r, const uint32_t (&so)[PC], int c,
                                               bool set, int t, Acc (&acc)[FN][FM]) const {
        static_assert(0 <= I0 && I0 <= I1 && I1 <= FM, "accumulator block rows");
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int i = I0; i < I1; ++i) {
                f32x4 g[PC][NQ];
#pragma unroll
                for (int k = 0; k < PC; ++k)
                    if (k < c)
#pragma unroll
                        for (int q = 0; q < NQ; ++q) g[k][q] = load_coherent(r, so[k] + part_off((j * FM + i) * NQ + q, t));
#pragma unroll
                for (int k = 0; k < PC; ++k)
                    if (k < c)
#pragma unroll
                        for (int q = 0; q < NQ; ++q)
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                acc[j][i][4 * q + e] = (set && k == 0) ? g[k][q][e] : acc[j][i][4 * q + e] + g[k][q][e];
            }
    }

    // A Stream-K piece of split tile s, after its partial is stored: the wave counts itself in
    // on the tile's counter for this wave (one counter per wave, since every wave stores and
    // later reduces only the positions it holds), and the wave that arrives last -- its partial
    // stores, like every other piece's, complete at device scope before its increment -- sums
    // the pieces of its positions in ascending K order, resets the counter for the next launch,
    // and stores its part of the tile through the register epilogue (bias, activation).  Nothing
    // waits on another workgroup, so the grid needs no co-residency.  The sum is
    // (...(p_first + p_first+1) + ...) + p_last, whichever piece arrives last: its own piece is
    // used from registers when it is the first or one of two (a + b = b + a exactly), otherwise
    // every piece is read back.
    template <int EPI, int I0, int I1>
    __device__ __forceinline__ void finish_piece(const GemmParams& p, const Unit& u, int v,
                                                 const __amdgpu_buffer_rsrc_t& r, Acc (&acc)[FN][FM]) {
        static_assert(0 <= I0 && I0 <= I1 && I1 <= FM, "accumulator block rows");
        const int kI = p.k_iters, sp = u.split;
        const int first = sk_owner(p, sp * kI), last = sk_owner(p, sp * kI + kI - 1);
        wait_vmcnt<0>();
        // (sk_stride: 32 words, one 128-byte line per split tile, or NW when packed)
        static_assert(C::NW <= 32, "a split tile's counters fit one 128-byte line");
        unsigned* flag = p.sk_flags + (size_t)sp * (size_t)p.sk_stride + twave;
        unsigned old = 0;
        if (lane == 0) old = __hip_atomic_fetch_add(flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        old = (unsigned)__builtin_amdgcn_readfirstlane((int)old);
        if (old != (unsigned)(last - first)) return;
        if (lane == 0) __hip_atomic_store(flag, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int t = slice_thread();
        auto slot_of = [&](int w) {
            return (uint32_t)((sk_slot(p, w, sp - sk_start(p, w) / kI, C::BM * C::BN) - p.ws) * 4);
        };
        // own piece first or one of two: the others are added to it in K order; otherwise the
        // sum starts over from the first piece and the own one is read back too.  Pieces are
        // read PC at a time (several for a wave holding few blocks, whose registers allow it).
        const bool keep = v == first || last - first == 1;
        constexpr int PC = FN * (I1 - I0) <= 2 ? 4 : 1;
        // k-th piece to add from w0 on (the own piece skipped when kept)
        auto nth = [&](int w0, int k) { return w0 + k + ((keep && w0 <= v && w0 + k >= v) ? 1 : 0); };
        bool set = !keep;
        for (int w = first; nth(w, 0) <= last;) {
            uint32_t so[PC];
            int c = 0;
#pragma unroll
            for (int k = 0; k < PC; ++k) {
                const int wk_ = nth(w, k);
                so[k] = wk_ <= last ? slot_of(wk_) : 0u;
                c += wk_ <= last ? 1 : 0;
            }
            add_pieces<PC, I0, I1>(r, so, c, set, t, acc);
            set = false;
            w = nth(w, PC - 1) + 1;
        }
        store_tile_regs<EPI, I0, I1>(p, u, acc);
    }
    template <int EPI, int WK>
    __device__ __forceinline__ void finish_piece_sliced_as(const GemmParams& p, const Unit& u, int v,
                                                           uint32_t slot_off, bool next, Acc (&acc)[FN][FM]) {
        if (next) wait_vmcnt<PRO_LOADS>();
        else wait_vmcnt<0>();
        barrier();
        xphases<WK, 0>(acc);
        if constexpr (own_rows(WK) > 0) {
            const __amdgpu_buffer_rsrc_t r = make_rsrc(p.ws, p.ws_bytes);
            store_partial<own_base(WK), own_base(WK) + own_rows(WK)>(r, slot_off, acc);
            finish_piece<EPI, own_base(WK), own_base(WK) + own_rows(WK)>(p, u, v, r, acc);
        }
    }
    // A Stream-K piece: store its FP32 partial, then the last arrival finishes the tile.  A
    // K-sliced tile sums its slices first (as for a whole tile) and each slice goes on with the
    // blocks it owns.
    template <int EPI>
    __device__ __forceinline__ void finish_split(const GemmParams& p, const Unit& u, int v, bool next,
                                                 Acc (&acc)[FN][FM]) {
        const uint32_t slot_off = (uint32_t)((sk_slot(p, v, u.local, C::BM * C::BN) - p.ws) * 4);
        if constexpr (C::WGK > 1) {
            if (wk == 0) finish_piece_sliced_as<EPI, 0>(p, u, v, slot_off, next, acc);
            else finish_piece_sliced_as<EPI, 1>(p, u, v, slot_off, next, acc);
        } else {
            const __amdgpu_buffer_rsrc_t r = make_rsrc(p.ws, p.ws_bytes);
            store_partial(r, slot_off, acc);
            finish_piece<EPI, 0, FM>(p, u, v, r, acc);
        }
    }
};

// The activation epilogue stores from registers, where its VALU work overlaps the stores;
// the plain cast stages through LDS, whose full-row stores drain faster when every
// workgroup stores at once.  The Stream-K kernel, whose split pieces leave through
// store_partial, stores its whole tiles from registers too: the staging registers would
// push it past 256 VGPRs.
// A K-sliced tile exchanges its partial sums through the free stage(s) and stores from
// registers; its Stream-K pieces exchange first and then store their FP32 partials.  A tile
// whose output rows are not a power-of-two number of 16-byte pieces stores from registers, and
// so does a tile with refill-only waves: they skip the epilogue, which may then hold no barrier.
// A tile with an early refill stores from registers too: the next unit's DMA prologue then fills
// part of stage S-1, the staging area.
template <class C, int EPI, bool SK>
constexpr bool epi_in_regs() {
    return EPI != EPI_STORE || SK || !C::OUT_POW2 || C::PROD > 0 || C::EARLY > 0 || C::MF != 32;
}

// The wave roles of a tile: with refill-only waves (C::PROD > 0) waves [0, PROD) issue the whole
// refill and hold no wave tile, and the others hold wave tiles and issue no DMA; otherwise every
// wave holds a wave tile and waves [0, C::DW) issue the refill.  Calls
// body.template run<ISSUE, MMA>() with the calling wave's roles, a wave-uniform choice made once.
// Every kernel builds its engines inside a body run here.
template <class C, class Body>
__device__ __forceinline__ void with_wave_roles(Body& body) {
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    if constexpr (C::PROD > 0) {
        if (wave < C::PROD) body.template run<true, false>();
        else body.template run<false, true>();
    } else if constexpr (C::DW == C::NW) {
        body.template run<true, true>();
    } else {
        if (wave < C::DW) body.template run<true, true>();
        else body.template run<false, true>();
    }
}

// One wave's walk over its workgroup's units, in the refill role ISSUE and tile role MMA.
// Every wave of the workgroup passes the same barriers whatever its roles.
template <int DT, class C, int EPI, bool SK, bool FASTK, bool GATHER, bool ISSUE, bool MMA>
__device__ __forceinline__ void walk_units(const GemmParams& p, lds_char* smem, int v, int G) {
    constexpr bool EPI_IN_REGS = epi_in_regs<C, EPI, SK>();
    // the refill waves skip the epilogue's data: a register epilogue or a split piece's partial
    // and finish (no barrier), or a K-sliced tile's exchange, whose barriers they pass too
    static_assert(C::PROD == 0 || EPI_IN_REGS || C::WGK > 1, "refill waves: no staged epilogue");
    Engine<DT, C, GATHER, ISSUE, MMA> eng(smem, p);
    typename AccOf<C::MF>::type acc[C::FN][C::FM];
    UnitWalker<SK> walk(p, v, G);
    Unit u = walk.next(p);
    if (!u.valid) return;
    eng.prologue(p, u);
    bool first = true;
    while (true) {
        const Unit nx = walk.next(p);
        eng.template mainloop<FASTK>(p, u, nx, acc, first);
        first = false;
        if constexpr (MMA) {
            if (SK && u.split >= 0)
                eng.template finish_split<EPI>(p, u, v, nx.valid, acc);
            else if constexpr (C::WGK > 1)
                eng.template store_sliced<EPI>(p, u, nx.valid, acc);
            else if constexpr (EPI_IN_REGS)
                eng.template store_tile_regs<EPI>(p, u, acc);
            else
                eng.template store_tile_lds<EPI>(p, u, nx.valid, acc);
        } else if constexpr (C::WGK > 1) {
            eng.store_sliced_sync(nx.valid);
        }
        if (!nx.valid) break;
        u = nx;
    }
}

template <int DT, class C, int EPI, bool SK, bool FASTK, bool GATHER>
struct WalkBody {
    const GemmParams& p;
    lds_char* smem;
    int v, G;
    template <bool ISSUE, bool MMA>
    __device__ __forceinline__ void run() { walk_units<DT, C, EPI, SK, FASTK, GATHER, ISSUE, MMA>(p, smem, v, G); }
};

// Persistent GEMM: every workgroup walks its units (whole tiles, then for Stream-K its split
// iterations) with the DMA of the next unit overlapping the epilogue of the current one.
// Split pieces that share a tile publish FP32 partials; the last to arrive finishes the tile.
template <int DT, class C, int EPI, bool SK, bool FASTK, bool GATHER = false>
__global__ void __launch_bounds__(C::NT) ffn_gemm_kernel(GemmParams p) {
    constexpr int SMEM = C::WGK > 1 ? C::LDS_USE : epi_in_regs<C, EPI, SK>() ? C::LDS_BYTES : C::LDS_ALLOC;
    __shared__ __attribute__((aligned(1024))) char smem_raw[SMEM];
    static_assert(!(GATHER && FASTK), "gathered rows take the checked refill path");

    const int G = gridDim.x;
    const int g = blockIdx.x;
    // Workgroups are dispatched round-robin over the 8 XCDs; renumber them so that
    // consecutive virtual ids (which take neighbouring tiles) share one XCD's L2.
    const int v = ((G & 7) == 0) ? (g & 7) * (G >> 3) + (g >> 3) : g;

    // Output rows past the last tile row that holds data (zero padding of a small-M problem) are
    // not computed: every workgroup writes its share of them as zeros, ahead of its first unit.
    if (p.zero_row0 < p.M) {
        const int cpr = p.c_cols / 8;  // 16-byte chunks per row
        const long long total = (long long)(p.M - p.zero_row0) * cpr;
        for (long long i = (long long)g * C::NT + threadIdx.x; i < total; i += (long long)G * C::NT) {
            const long long r = p.zero_row0 + i / cpr, c = i % cpr;
            *(u32x4*)((char*)p.c + ((size_t)r * (size_t)p.ldc + (size_t)c * 8) * 2) = u32x4{0u, 0u, 0u, 0u};
        }
    }
    for (int i = g * C::NT + (int)threadIdx.x; i < p.clear_count; i += G * C::NT)
        __hip_atomic_store(p.clear_words + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    WalkBody<DT, C, EPI, SK, FASTK, GATHER> body{p, (lds_char*)smem_raw, v, G};
    with_wave_roles<C>(body);
}

}  // namespace ffn
