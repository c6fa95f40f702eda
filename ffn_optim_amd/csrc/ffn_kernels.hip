// ffn_kernels.hip -- instantiates the GEMM engine for one (storage type, tile variant).
//
// Compiled once per pair with -DFFN_DT=<0 fp16|1 bf16> -DFFN_VARIANT=<id>; each object
// exports one extern "C" launcher ffn_launch_d<DT>_v<VARIANT> used by ffn_mi355x.hip.
#include "ffn_gemm.hpp"
#include "ffn_variants.hpp"

#if !defined(FFN_DT) || !defined(FFN_VARIANT)
#error "compile with -DFFN_DT=<0|1> -DFFN_VARIANT=<id>"
#endif

namespace {
template <int ID>
struct VariantCfg;
#define FFN_DEFINE_CFG(id, bm, bn, bk, wgm, wgn, st, ...)           \
    template <>                                                     \
    struct VariantCfg<id> {                                         \
        using type = ffn::TileCfg<bm, bn, bk, wgm, wgn, st, ##__VA_ARGS__>; \
    };
FFN_VARIANTS(FFN_DEFINE_CFG)
#undef FFN_DEFINE_CFG
using Cfg = VariantCfg<FFN_VARIANT>::type;
}  // namespace

#define FFN_CAT_(a, b, c, d) a##b##c##d
#define FFN_CAT(a, b, c, d) FFN_CAT_(a, b, c, d)
#define FFN_LAUNCHER FFN_CAT(ffn_launch_d, FFN_DT, _v, FFN_VARIANT)

namespace {
// one launch of ffn_gemm_kernel with the DMA addressing the plan chose
template <class CFG, int EPI, bool SK>
void launch_gemm(const ffn::GemmParams* p, dim3 g, dim3 b, hipStream_t stream) {
    if constexpr (EPI != ffn::EPI_STORE) {
        // up roles may read gathered activation rows
        if (p->a_gather) {
            hipLaunchKernelGGL((ffn::ffn_gemm_kernel<FFN_DT, CFG, EPI, SK, false, true>), g, b, 0, stream, *p);
            return;
        }
    }
    if (p->fast_dma)
        hipLaunchKernelGGL((ffn::ffn_gemm_kernel<FFN_DT, CFG, EPI, SK, true>), g, b, 0, stream, *p);
    else
        hipLaunchKernelGGL((ffn::ffn_gemm_kernel<FFN_DT, CFG, EPI, SK, false>), g, b, 0, stream, *p);
}

template <class CFG>
hipError_t launch_role(int role, const ffn::GemmParams* p, int grid, hipStream_t stream) {
    using namespace ffn;
    const dim3 g(grid), b(CFG::NT);
    switch (role) {
        case FFN_ROLE_UP_ERF:
            launch_gemm<CFG, EPI_GELU_ERF, false>(p, g, b, stream);
            break;
        case FFN_ROLE_UP_RATIONAL:
            launch_gemm<CFG, EPI_GELU_RATIONAL, false>(p, g, b, stream);
            break;
        case FFN_ROLE_DOWN_BASIC:
            launch_gemm<CFG, EPI_STORE, false>(p, g, b, stream);
            break;
        case FFN_ROLE_DOWN_STREAMK:
            launch_gemm<CFG, EPI_STORE, true>(p, g, b, stream);
            break;
        case FFN_ROLE_UP_SPLIT_ERF:
            launch_gemm<CFG, EPI_GELU_ERF, true>(p, g, b, stream);
            break;
        case FFN_ROLE_UP_SPLIT_RATIONAL:
            launch_gemm<CFG, EPI_GELU_RATIONAL, true>(p, g, b, stream);
            break;
        case FFN_ROLE_UP_SILU:
            launch_gemm<CFG, EPI_SILU, false>(p, g, b, stream);
            break;
        case FFN_ROLE_UP_SWIGLU:
            if constexpr (CFG::WTN % 64 == 0) launch_gemm<CFG, EPI_SWIGLU, false>(p, g, b, stream);
            else return hipErrorInvalidValue;
            break;
        case FFN_ROLE_UP_SPLIT_SILU:
            launch_gemm<CFG, EPI_SILU, true>(p, g, b, stream);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
}  // namespace

extern "C" hipError_t FFN_LAUNCHER(int role, const ffn::GemmParams* p, int grid, hipStream_t stream) {
    return launch_role<Cfg>(role, p, grid, stream);
}
