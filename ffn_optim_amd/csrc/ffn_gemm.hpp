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
//   LDS --ds_read_b128--> A/B fragments --v_mfma_f32_32x32x16_{bf16,f16}--> FP32 acc
// LDS rows are BK*2 bytes; the 16-byte chunk c of row r lives at c ^ swz(r) so
// that the 8 lanes served per LDS cycle hit 8 distinct bank groups.  Out-of-range
// rows and the K tail read as zero through the buffer descriptor's range check,
// so tiles may overhang the matrices and no load can leave its buffer.
//
// The MFMA is issued with the weight fragment as operand A and the activation
// fragment as operand B, so an accumulator holds D[n][m]; each lane then owns
// four consecutive n of one row m and the epilogue writes 8-byte packed stores.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ffn {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((__vector_size__(16)));
typedef _Float16 f16x8 __attribute__((__vector_size__(16)));
typedef __attribute__((address_space(3))) char lds_char;

enum { DT_F16 = 0, DT_BF16 = 1 };
enum { EPI_GELU_ERF = 0, EPI_GELU_RATIONAL = 1, EPI_STORE = 2 };

// Launch-time description of one GEMM.  All extents are in elements.
struct GemmParams {
    const void* a;        // [M][lda]   activations (X or hidden)
    const void* b;        // [N][ldb]   weights (W1 or W2)
    void* c;              // [M][ldc]   hidden or out
    float* ws;            // Stream-K partial-tile slots (FP32)
    unsigned* counters;   // Stream-K arrivals, one per split tile, zero between launches
    int M, N, K;
    int lda, ldb, ldc;
    int tiles_m, tiles_n;
    int k_iters;          // ceil(K / BK)
    int dp_tiles;         // tiles [0, dp_tiles) are reduced whole by one workgroup
    int sk_tiles;         // tiles [dp_tiles, dp_tiles + sk_tiles) are split along K
    int sk_q, sk_r;       // split iterations per workgroup: q, plus one for the first r
    int slots_per_wg;     // partial-tile slots owned by each workgroup
    int group_m;          // tile-order swizzle: tiles walk group_m tile-rows column by column
};

template <int BM_, int BN_, int BK_, int WGM_, int WGN_, int STAGES_>
struct TileCfg {
    static constexpr int BM = BM_, BN = BN_, BK = BK_;
    static constexpr int WGM = WGM_, WGN = WGN_, STAGES = STAGES_;
    static constexpr int NW = WGM * WGN;           // waves per workgroup
    static constexpr int NT = NW * 64;             // threads per workgroup
    static constexpr int WTM = BM / WGM, WTN = BN / WGN;  // wave tile
    static constexpr int FM = WTM / 32, FN = WTN / 32;    // 32x32 MFMA blocks per wave
    static constexpr int ROWB = BK * 2;            // bytes of one LDS row
    static constexpr int CH = ROWB / 16;           // 16-byte chunks per row
    static constexpr int RPB = 1024 / ROWB;        // rows per 1 KiB DMA block (64 lanes x 16 B)
    static constexpr int RPL = (ROWB >= 128) ? 1 : 128 / ROWB;  // rows per 128-byte bank line
    static constexpr int A_BYTES = BM * ROWB, B_BYTES = BN * ROWB;
    static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
    static constexpr int A_BLKS = A_BYTES / 1024, B_BLKS = B_BYTES / 1024;
    static constexpr int A_PW = A_BLKS / NW, B_PW = B_BLKS / NW;  // DMA blocks per wave
    static constexpr int LOADS = A_PW + B_PW;      // DMA instructions per wave per stage
    static constexpr int LDS_BYTES = STAGES * STAGE_BYTES;
    static constexpr int KSTEPS = BK / 16;         // MFMA k-steps per stage
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32");
    static_assert(ROWB % 16 == 0 && CH >= 2, "BK must be a multiple of 16");
    static_assert(A_BLKS % NW == 0 && B_BLKS % NW == 0, "DMA blocks must split evenly over waves");
    static_assert(32 % (CH * RPL) == 0 || (CH * RPL) % 32 == 0, "swizzle period");
    static_assert(LDS_BYTES <= 160 * 1024, "gfx950 has 160 KiB of LDS per CU");
};

// ---------------------------------------------------------------------------
// small device helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    // word3 0x00020000: raw (untyped) 32-bit data format, range-checked against `bytes`
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
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

// Round-to-nearest-even FP32 -> storage type, four values packed into 8 bytes.
template <int DT>
__device__ __forceinline__ uint2 pack4(float a, float b, float c, float d) {
    if constexpr (DT == DT_BF16) {
        __bf16 h0 = (__bf16)a, h1 = (__bf16)b, h2 = (__bf16)c, h3 = (__bf16)d;
        uint2 r;
        r.x = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
        r.y = (uint32_t)__builtin_bit_cast(uint16_t, h2) | ((uint32_t)__builtin_bit_cast(uint16_t, h3) << 16);
        return r;
    } else {
        _Float16 h0 = (_Float16)a, h1 = (_Float16)b, h2 = (_Float16)c, h3 = (_Float16)d;
        uint2 r;
        r.x = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
        r.y = (uint32_t)__builtin_bit_cast(uint16_t, h2) | ((uint32_t)__builtin_bit_cast(uint16_t, h3) << 16);
        return r;
    }
}

// ---------------------------------------------------------------------------
// GELU forms (applied to the FP32 accumulator before the cast)
// ---------------------------------------------------------------------------

// Exact-form GELU, 0.5*z*(1+erf(z/sqrt(2))) -- torch.nn.functional.gelu(approximate='none') --
// evaluated as 0.5*z*erfc(-z/sqrt(2)), which is the same function without the cancellation of
// 1+erf in the negative tail.  erfcf is the ROCm device library's single-precision erfc.
__device__ __forceinline__ float gelu_erf(float z) {
    return 0.5f * z * erfcf(-z * 0.70710678118654752f);
}

// Rational erf GELU: t = clamp(z/sqrt2, +-3.92), erf(t) ~ t*P5(t^2)/Q5(t^2), coefficients and
// operation order of validation/reference.py:5-13 (= ops/kernel/ffn.py:548-572).
__device__ __forceinline__ float gelu_rational(float z) {
    float t = z * 0.70710678118654752f;
    t = fminf(fmaxf(t, -3.92f), 3.92f);
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

template <int EPI>
__device__ __forceinline__ float activate(float z) {
    if constexpr (EPI == EPI_GELU_ERF) return gelu_erf(z);
    else if constexpr (EPI == EPI_GELU_RATIONAL) return gelu_rational(z);
    else return z;
}

// tile index -> (tile row, tile column); tiles walk `group_m` tile-rows column by column so
// that consecutive tiles share weight panels (columns) and activation panels (rows).
__device__ __forceinline__ void tile_coords(const GemmParams& p, int t, int& tm, int& tn) {
    const int per_group = p.group_m * p.tiles_n;
    const int gidx = t / per_group;
    const int first_m = gidx * p.group_m;
    const int rows = min(p.tiles_m - first_m, p.group_m);
    const int r = t - gidx * per_group;
    tm = first_m + r % rows;
    tn = r / rows;
}

// ---------------------------------------------------------------------------
// the GEMM engine
// ---------------------------------------------------------------------------

template <int DT, class C>
struct Engine {
    static constexpr int FM = C::FM, FN = C::FN, NT = C::NT;

    lds_char* smem;
    int tid, lane, wave, wm, wn;
    // per-lane LDS byte offsets of the fragment rows (without stage / k-step parts)
    int a_row_off, b_row_off;
    int swz;  // chunk XOR of this lane's fragment rows

    __device__ __forceinline__ Engine(lds_char* s) : smem(s) {
        tid = threadIdx.x;
        lane = tid & 63;
        wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        wm = wave % C::WGM;
        wn = wave / C::WGM;
        const int r = lane & 31;
        a_row_off = (wm * C::WTM + r) * C::ROWB;
        b_row_off = C::A_BYTES + (wn * C::WTN + r) * C::ROWB;
        swz = (r / C::RPL) % C::CH;
    }

    // Per-lane part of the DMA source offset: this lane fills physical chunk (lane % CH) of
    // row (lane / CH) of every 1 KiB block, i.e. logical chunk c = pc ^ swz(row).  The swizzle
    // of a row depends only on its position inside the block, so one lane offset per operand
    // serves every block; the block's row offset is added to it.  The whole offset stays in
    // the VGPR operand: the buffer range check covers voffset but not soffset.
    __device__ __forceinline__ int dma_chunk() const {
        const int rl = lane / C::CH;
        const int pc = lane % C::CH;
        return pc ^ ((rl / C::RPL) % C::CH);
    }

    // Issue the DMA of K-iteration `kit` into LDS stage `stage`.  Rows past the operand and
    // chunks past K get an offset >= 2^31, beyond any range, and read as zero.
    __device__ __forceinline__ void issue(const __amdgpu_buffer_rsrc_t& ra,
                                          const __amdgpu_buffer_rsrc_t& rb, int lda2, int ldb2,
                                          int K, int stage, int kit) {
        const int k0 = kit * C::BK;
        lds_char* st = smem + stage * C::STAGE_BYTES;
        const int rl = lane / C::CH;
        const int kk = k0 + dma_chunk() * 8;
        const bool ok = (k0 + C::BK <= K) || (kk < K);
        const uint32_t va = ok ? (uint32_t)(rl * lda2 + kk * 2) : 0x80000000u;
        const uint32_t vb = ok ? (uint32_t)(rl * ldb2 + kk * 2) : 0x80000000u;
#pragma unroll
        for (int i = 0; i < C::A_PW; ++i) {
            const int blk = wave * C::A_PW + i;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (__attribute__((address_space(3))) void*)(st + blk * 1024), 16,
                (int)(va + (uint32_t)(blk * C::RPB * lda2)), 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < C::B_PW; ++i) {
            const int blk = wave * C::B_PW + i;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rb, (__attribute__((address_space(3))) void*)(st + C::A_BYTES + blk * 1024), 16,
                (int)(vb + (uint32_t)(blk * C::RPB * ldb2)), 0, 0, 0);
        }
    }

    __device__ __forceinline__ void compute(int stage, f32x16 (&acc)[FN][FM]) {
        const lds_char* st = smem + stage * C::STAGE_BYTES;
#pragma unroll
        for (int s = 0; s < C::KSTEPS; ++s) {
            const int chunk = ((2 * s + (lane >> 5)) ^ swz) * 16;
            u32x4 af[FM], bf[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i)
                af[i] = *(const __attribute__((address_space(3))) u32x4*)(st + a_row_off + i * 32 * C::ROWB + chunk);
#pragma unroll
            for (int j = 0; j < FN; ++j)
                bf[j] = *(const __attribute__((address_space(3))) u32x4*)(st + b_row_off + j * 32 * C::ROWB + chunk);
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int i = 0; i < FM; ++i) acc[j][i] = mfma32<DT>(bf[j], af[i], acc[j][i]);
        }
    }

    // acc = sum over K-iterations [kb, ke) of tile (tm, tn).
    __device__ __forceinline__ void mainloop(const GemmParams& p, int tm, int tn, int kb, int ke,
                                             f32x16 (&acc)[FN][FM]) {
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int i = 0; i < FM; ++i) acc[j][i] = f32x16{};

        const int row0 = tm * C::BM, col0 = tn * C::BN;
        const int lda2 = p.lda * 2, ldb2 = p.ldb * 2;
        const char* abase = (const char*)p.a + (size_t)row0 * (size_t)lda2;
        const char* bbase = (const char*)p.b + (size_t)col0 * (size_t)ldb2;
        const uint32_t abytes = (uint32_t)min(C::BM, p.M - row0) * (uint32_t)lda2;
        const uint32_t bbytes = (uint32_t)min(C::BN, p.N - col0) * (uint32_t)ldb2;
        const __amdgpu_buffer_rsrc_t ra = make_rsrc(abase, abytes);
        const __amdgpu_buffer_rsrc_t rb = make_rsrc(bbase, bbytes);

        // no wave may still be reading LDS from the previous unit
        __syncthreads();
#pragma unroll
        for (int s = 0; s < C::STAGES - 1; ++s)
            if (kb + s < ke) issue(ra, rb, lda2, ldb2, p.K, s, kb + s);

        int stage = 0;
        for (int kit = kb; kit < ke; ++kit) {
            if constexpr (C::STAGES == 2) {
                wait_vmcnt<0>();
            } else {
                static_assert(C::STAGES == 3, "2 or 3 LDS stages");
                if (kit + 1 < ke) wait_vmcnt<C::LOADS>();
                else wait_vmcnt<0>();
            }
            __syncthreads();
            const int nk = kit + C::STAGES - 1;
            if (nk < ke) {
                int ns = stage + C::STAGES - 1;
                if (ns >= C::STAGES) ns -= C::STAGES;
                issue(ra, rb, lda2, ldb2, p.K, ns, nk);
            }
            compute(stage, acc);
            stage = (stage + 1 == C::STAGES) ? 0 : stage + 1;
        }
    }

    // Output position of accumulator group (j, i, q): row m, columns n..n+3.
    __device__ __forceinline__ void group_pos(int tm, int tn, int j, int i, int q, int& m,
                                              int& n) const {
        m = tm * C::BM + wm * C::WTM + 32 * i + (lane & 31);
        n = tn * C::BN + wn * C::WTN + 32 * j + 8 * q + 4 * (lane >> 5);
    }

    template <int EPI>
    __device__ __forceinline__ void store4(const GemmParams& p, int m, int n, float v0, float v1,
                                           float v2, float v3) const {
        if (m < p.M && n < p.N) {
            const uint2 v = pack4<DT>(activate<EPI>(v0), activate<EPI>(v1), activate<EPI>(v2),
                                      activate<EPI>(v3));
            *(uint2*)((char*)p.c + ((size_t)m * (size_t)p.ldc + (size_t)n) * 2) = v;
        }
    }

    // Write acc (activated, cast) to C[tile] with row/column masking.
    template <int EPI>
    __device__ __forceinline__ void store_tile(const GemmParams& p, int tm, int tn,
                                               f32x16 (&acc)[FN][FM]) const {
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    int m, n;
                    group_pos(tm, tn, j, i, q, m, n);
                    store4<EPI>(p, m, n, acc[j][i][4 * q], acc[j][i][4 * q + 1],
                                acc[j][i][4 * q + 2], acc[j][i][4 * q + 3]);
                }
    }

    // FP32 partial tile in the accumulator's own register order: group (j, i, q) of thread
    // tid lives at ((j*FM + i)*4 + q)*NT + tid (16-byte units), so every store is coalesced.
    __device__ __forceinline__ void store_partial(float* slot, f32x16 (&acc)[FN][FM]) const {
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int idx = (j * FM + i) * 4 + q;
                    const f32x4 v = {acc[j][i][4 * q], acc[j][i][4 * q + 1], acc[j][i][4 * q + 2],
                                     acc[j][i][4 * q + 3]};
                    *(f32x4*)(slot + ((size_t)idx * NT + tid) * 4) = v;
                }
    }
};

// Split-region bookkeeping: iteration x (0-based inside the split region) belongs to
// workgroup sk_owner(x); workgroup v starts at sk_start(v).
__device__ __forceinline__ int sk_owner(const GemmParams& p, int x) {
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

template <int DT, class C, int EPI, bool SK>
__global__ void __launch_bounds__(C::NT) ffn_gemm_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(1024))) char smem_raw[C::LDS_BYTES];
    Engine<DT, C> eng((lds_char*)smem_raw);
    f32x16 acc[C::FN][C::FM];

    const int G = gridDim.x;
    const int g = blockIdx.x;
    // Workgroups are dispatched round-robin over the 8 XCDs; renumber them so that
    // consecutive virtual ids (which take neighbouring tiles) share one XCD's L2.
    const int v = ((G & 7) == 0) ? (g & 7) * (G >> 3) + (g >> 3) : g;

    for (int t = v; t < p.dp_tiles; t += G) {
        int tm, tn;
        tile_coords(p, t, tm, tn);
        eng.mainloop(p, tm, tn, 0, p.k_iters, acc);
        eng.template store_tile<EPI>(p, tm, tn, acc);
    }

    if constexpr (SK) {
        // Stream-K region: this workgroup owns split iterations [it_begin, it_end), which may
        // cover the tail of one tile, whole tiles and the head of another.  A tile reduced by
        // one workgroup is stored directly.  Otherwise every contributor publishes an FP32
        // partial and counts its arrival; the last to arrive sums all partials in ascending
        // K order (so the result does not depend on arrival order), rounds once to the
        // storage type and re-arms the counter.  Nobody waits on anybody: no co-residency
        // assumption, every workgroup runs to completion.
        __shared__ int last_flag;
        constexpr int TE = C::BM * C::BN;
        const int kI = p.k_iters;
        const int it_begin = sk_start(p, v), it_end = sk_start(p, v + 1);
        for (int it = it_begin; it < it_end;) {
            const int s = it / kI;
            const int kb = it - s * kI;
            const int ke = min(kI, kb + (it_end - it));
            const int t = p.dp_tiles + s;
            int tm, tn;
            tile_coords(p, t, tm, tn);
            eng.mainloop(p, tm, tn, kb, ke, acc);
            const int first = sk_owner(p, s * kI), last = sk_owner(p, s * kI + kI - 1);
            if (first == last) {
                eng.template store_tile<EPI>(p, tm, tn, acc);
            } else {
                eng.store_partial(sk_slot(p, v, s - it_begin / kI, TE), acc);
                __threadfence();
                __syncthreads();
                if (eng.tid == 0) {
                    const unsigned old = __hip_atomic_fetch_add(
                        p.counters + s, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
                    last_flag = (old == (unsigned)(last - first));
                }
                __syncthreads();
                if (last_flag) {
                    __threadfence();
                    for (int j = 0; j < C::FN; ++j)
                        for (int i = 0; i < C::FM; ++i)
#pragma unroll
                            for (int q = 0; q < 4; ++q) {
                                const size_t off = ((size_t)((j * C::FM + i) * 4 + q) * C::NT + eng.tid) * 4;
                                f32x4 tot = *(const f32x4*)(sk_slot(p, first, s - sk_start(p, first) / kI, TE) + off);
                                for (int w = first + 1; w <= last; ++w)
                                    tot += *(const f32x4*)(sk_slot(p, w, s - sk_start(p, w) / kI, TE) + off);
                                int m, n;
                                eng.group_pos(tm, tn, j, i, q, m, n);
                                eng.template store4<EPI>(p, m, n, tot.x, tot.y, tot.z, tot.w);
                            }
                    if (eng.tid == 0)
                        __hip_atomic_store(p.counters + s, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            it += ke - kb;
        }
    }
}

}  // namespace ffn
