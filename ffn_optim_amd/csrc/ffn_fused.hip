// ffn_fused.hip -- the whole FFN in one launch, for the mid-size and large problems whose up
// GEMM has at least one row block per XCD: up tiles and down tiles share one persistent grid, and
// a down tile starts as soon as the hidden rows it reads are stored, instead of after a kernel
// boundary (the reference's single artifact with its all-core stage barrier, ops/kernel/ffn.py:
// 371-376, 582-585).
//
// Compiled once per (storage type, up variant, down variant) pair with -DFFN_DT=<0|1>
// -DFFN_UPV=<id> -DFFN_DNV=<id>; each object exports ffn_fused_d<DT>_u<UPV>_n<DNV>.
//
// Work is split by XCD.  Up row block r (BM_up rows of hidden) belongs to XCD r mod 8, and so do
// the down tiles of its rows.  A workgroup reads the XCD it runs on (HW_REG_XCC_ID) and takes
// tickets from that XCD's queue: every up tile of the XCD first, then its down tiles.  A down
// tile waits until its row block's counter shows every up tile of the row block stored.  The
// hidden rows a down tile reads were written by the same XCD, into the L2 it reads them from: no
// write-through and no cache maintenance is needed.  Tickets are handed out in order to running
// workgroups and every up ticket of a queue precedes its down tickets, so a waiting down tile
// waits only on up tiles held by running workgroups, which wait on nothing: the launch cannot
// deadlock, whichever workgroups are resident, and a bounded poll guards even that.  The last
// workgroup to leave clears the queues and counters for the next launch.
//
// Every tile is run through with_wave_roles, as in ffn_gemm_kernel: waves past a tile's refill
// waves never issue its DMA.
#include "ffn_gemm.hpp"
#include "ffn_variants.hpp"

#if !defined(FFN_DT) || !defined(FFN_UPV) || !defined(FFN_DNV)
#error "compile with -DFFN_DT=<0|1> -DFFN_UPV=<id> -DFFN_DNV=<id>"
#endif

namespace {
template <int ID>
struct VariantCfg;
#define FFN_DEFINE_CFG(id, bm, bn, bk, wgm, wgn, st, ...)                   \
    template <>                                                             \
    struct VariantCfg<id> {                                                 \
        using type = ffn::TileCfg<bm, bn, bk, wgm, wgn, st, ##__VA_ARGS__>; \
    };
FFN_VARIANTS(FFN_DEFINE_CFG)
#undef FFN_DEFINE_CFG
using CfgU = VariantCfg<FFN_UPV>::type;
using CfgD = VariantCfg<FFN_DNV>::type;
}  // namespace

namespace ffn {

template <class C, int EPI>
constexpr int tile_lds() { return C::WGK > 1 ? C::LDS_USE : epi_in_regs<C, EPI, false>() ? C::LDS_BYTES : C::LDS_ALLOC; }

// One whole tile (its K range in one unit, no next unit), in the calling wave's roles.  On entry
// no load or store of this workgroup is outstanding, so the first stage wait counts the
// prologue's loads only.  On return the tile's stores are issued, not complete.
template <int DT, class C, int EPI, bool FK>
struct TileBody {
    const GemmParams& p;
    lds_char* smem;
    Unit u;
    template <bool ISSUE, bool MMA>
    __device__ __forceinline__ void run() {
        static_assert(C::PROD == 0 || epi_in_regs<C, EPI, false>() || C::WGK > 1, "refill waves: no staged epilogue");
        Engine<DT, C, false, ISSUE, MMA> eng(smem, p);
        typename AccOf<C::MF>::type acc[C::FN][C::FM];
        Unit none = u;
        none.valid = false;
        eng.prologue(p, u);
        eng.template mainloop<FK>(p, u, none, acc, true);
        if constexpr (MMA) {
            if constexpr (C::WGK > 1) eng.template store_sliced<EPI>(p, u, false, acc);
            else if constexpr (epi_in_regs<C, EPI, false>()) eng.template store_tile_regs<EPI>(p, u, acc);
            else eng.template store_tile_lds<EPI>(p, u, false, acc);
        } else if constexpr (C::WGK > 1) {
            eng.store_sliced_sync(false);
        }
    }
};

__device__ __forceinline__ int xcc_id() {
    // s_getreg_b32 hwreg(HW_REG_XCC_ID, 0, 4): the XCD this wave runs on
    return __builtin_amdgcn_s_getreg((20) | (0 << 6) | ((4 - 1) << 11)) & 7;
}

// Up row blocks of XCD x: x, x + 8, ...; down row blocks of up row block r: [r * ratio, ...).
__device__ __forceinline__ int owned_rbs(int tiles_m_up, int x) { return x < tiles_m_up ? (tiles_m_up - x + 7) / 8 : 0; }
__device__ __forceinline__ int down_rows_of(const GemmParams& pd, int ratio, int rb) {
    return max(0, min(ratio, pd.tiles_m - rb * ratio));
}

__device__ __forceinline__ void zero_padding_rows(const GemmParams& p, int g, int G, int nt) {
    if (p.zero_row0 < p.M) {
        const int cpr = p.c_cols / 8;
        const long long total = (long long)(p.M - p.zero_row0) * cpr;
        for (long long i = (long long)g * nt + threadIdx.x; i < total; i += (long long)G * nt) {
            const long long r = p.zero_row0 + i / cpr, c = i % cpr;
            *(u32x4*)((char*)p.c + ((size_t)r * (size_t)p.ldc + (size_t)c * 8) * 2) = u32x4{0u, 0u, 0u, 0u};
        }
    }
}

template <int DT, class CU, class CD, int EPI, bool FKU, bool FKD>
__global__ void __launch_bounds__(CU::NT) ffn_fused_kernel(GemmParams pu, GemmParams pd, FusedParams f) {
    static_assert(CU::NT == CD::NT, "both phases run on the same workgroup shape");
    constexpr int LU = tile_lds<CU, EPI>(), LD = tile_lds<CD, EPI_STORE>();
    __shared__ __attribute__((aligned(1024))) char smem_raw[LU > LD ? LU : LD];
    lds_char* smem = (lds_char*)smem_raw;
    // The ticket is passed on in the first word of stage 0, which no epilogue uses (they stage and
    // exchange from stage 1 on); it is written only once every wave's loads and stores have
    // completed and every wave has passed a barrier, and read before the next refill of stage 0.
    volatile int* ticket = (volatile int*)smem_raw;
    const int G = gridDim.x, g = blockIdx.x;
    zero_padding_rows(pu, g, G, CU::NT);
    zero_padding_rows(pd, g, G, CU::NT);

    const int x = __builtin_amdgcn_readfirstlane(xcc_id());
    const int nrb = owned_rbs(pu.tiles_m, x);
    const int n_up = nrb * pu.tiles_n;
    int n_down = 0;
    for (int i = 0; i < nrb; ++i) n_down += down_rows_of(pd, f.ratio, x + 8 * i) * pd.tiles_n;

    while (true) {
        wait_vmcnt<0>();
        __syncthreads();
        if (threadIdx.x == 0) *ticket = (int)__hip_atomic_fetch_add(f.ctr + x * kFusedStride, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        const int t = __builtin_amdgcn_readfirstlane(*ticket);
        __syncthreads();  // every wave has read the ticket before stage 0 is refilled
        if (t < n_up) {
            const int rb = x + 8 * (t / pu.tiles_n);
            Unit u;
            u.tm = rb, u.tn = t % pu.tiles_n, u.kb = 0, u.ke = pu.k_iters, u.split = -1, u.local = 0, u.valid = true;
            TileBody<DT, CU, EPI, FKU> body{pu, smem, u};
            with_wave_roles<CU>(body);
            // the tile's hidden stores have reached the XCD's L2 before its row block counts it
            wait_vmcnt<0>();
            __syncthreads();
            if (threadIdx.x == 0)
                __hip_atomic_fetch_add(f.ctr + kFusedReady + rb * kFusedStride, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else if (t < n_up + n_down) {
            int j = t - n_up, rb = x;
            for (int i = 0; i < nrb; ++i) {
                rb = x + 8 * i;
                const int cnt = down_rows_of(pd, f.ratio, rb) * pd.tiles_n;
                if (j < cnt) break;
                j -= cnt;
            }
            if (threadIdx.x == 0) {
                const unsigned need = (unsigned)pu.tiles_n;
                int polls = 0;
                while (__hip_atomic_load(f.ctr + kFusedReady + rb * kFusedStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < need) {
                    if (++polls > f.spin_limit) {
                        __hip_atomic_store(f.ctr + kFusedError, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(4);
                }
            }
            __syncthreads();
            Unit u;
            u.tm = rb * f.ratio + j / pd.tiles_n, u.tn = j % pd.tiles_n, u.kb = 0, u.ke = pd.k_iters;
            u.split = -1, u.local = 0, u.valid = true;
            TileBody<DT, CD, EPI_STORE, FKD> body{pd, smem, u};
            with_wave_roles<CD>(body);
        } else {
            break;
        }
    }
    // the last workgroup to leave: every ticket has been taken and every wait has ended
    if (threadIdx.x == 0) {
        const unsigned left = __hip_atomic_fetch_add(f.ctr + kFusedLeft, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (left == (unsigned)G - 1) {
            for (int i = 0; i < 8; ++i) __hip_atomic_store(f.ctr + i * kFusedStride, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            for (int i = 0; i < pu.tiles_m; ++i)
                __hip_atomic_store(f.ctr + kFusedReady + i * kFusedStride, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(f.ctr + kFusedLeft, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

}  // namespace ffn

#define FFN_CAT_(a, b, c, d, e, f) a##b##c##d##e##f
#define FFN_CAT(a, b, c, d, e, f) FFN_CAT_(a, b, c, d, e, f)
#define FFN_FUSED_LAUNCHER FFN_CAT(ffn_fused_d, FFN_DT, _u, FFN_UPV, _n, FFN_DNV)

namespace {
template <int EPI, bool FKU>
hipError_t launch_fused(const ffn::GemmParams* pu, const ffn::GemmParams* pd, const ffn::FusedParams* f,
                        dim3 g, dim3 b, hipStream_t stream) {
    if (pd->fast_dma)
        hipLaunchKernelGGL((ffn::ffn_fused_kernel<FFN_DT, CfgU, CfgD, EPI, FKU, true>), g, b, 0, stream, *pu, *pd, *f);
    else
        hipLaunchKernelGGL((ffn::ffn_fused_kernel<FFN_DT, CfgU, CfgD, EPI, FKU, false>), g, b, 0, stream, *pu, *pd, *f);
    return hipGetLastError();
}
}  // namespace

// role: the up epilogue (FFN_ROLE_UP_ERF or FFN_ROLE_UP_RATIONAL).  The up GEMM takes the
// SALU-addressed refill for interior tiles (its K is at most 8192), the down GEMM either refill.
extern "C" hipError_t FFN_FUSED_LAUNCHER(int role, const ffn::GemmParams* pu, const ffn::GemmParams* pd,
                                         const ffn::FusedParams* f, int grid, hipStream_t stream) {
    using namespace ffn;
    const dim3 g(grid), b(CfgU::NT);
    if (pu->a_gather || !pu->fast_dma) return hipErrorInvalidValue;
    switch (role) {
        case FFN_ROLE_UP_ERF:
            return launch_fused<EPI_GELU_ERF, true>(pu, pd, f, g, b, stream);
        case FFN_ROLE_UP_RATIONAL:
            return launch_fused<EPI_GELU_RATIONAL, true>(pu, pd, f, g, b, stream);
        default:
            return hipErrorInvalidValue;
    }
}
