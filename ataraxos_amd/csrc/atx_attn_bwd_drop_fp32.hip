// The fp32 attention backward with dropout (atx_attn_bwd_kernels.hpp built
// with DROP), head_dim 48 and 64, both variants, 1, 2, 4 and 8 key chunks;
// the 16-bit kernels are in atx_attn_bwd_drop.hip.
#include "atx_attn_bwd_kernels.hpp"

namespace atx {
namespace {

template <int D, bool LOOP>
int dropf_nkc(int nkc, int grid, size_t lds, hipStream_t st, const BwdArgs& a) {
    switch (nkc) {
        case 1: return launch_bwd(attn_bwd_fp32<D, 1, LOOP, true>, grid, lds, st, a);
        case 2: return launch_bwd(attn_bwd_fp32<D, 2, LOOP, true>, grid, lds, st, a);
        case 4: return launch_bwd(attn_bwd_fp32<D, 4, LOOP, true>, grid, lds, st, a);
        case 8: return launch_bwd(attn_bwd_fp32<D, 8, LOOP, true>, grid, lds, st, a);
    }
    ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: %d key chunks (fp32: 1, 2, 4, 8)", nkc);
}

template <int D>
int dropf_loop(bool loop, int nkc, int grid, size_t lds, hipStream_t st, const BwdArgs& a) {
    return loop ? dropf_nkc<D, true>(nkc, grid, lds, st, a) : dropf_nkc<D, false>(nkc, grid, lds, st, a);
}

}  // namespace

int dispatch_bwd_drop_fp32(bool loop, int D, int nkc, int grid, size_t lds, hipStream_t st, const BwdArgs& a) {
    switch (D) {
        case 48: return dropf_loop<48>(loop, nkc, grid, lds, st, a);
        case 64: return dropf_loop<64>(loop, nkc, grid, lds, st, a);
    }
    ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: dropout needs head_dim 48 or 64 (got %d)", D);
}

}  // namespace atx
