// LOOP instantiations of the 16-bit attention backward: one workgroup per
// (batch, KV head) over the group's query heads in blocks of query rows
// (atx_attn_bwd_kernels.hpp) -- grouped-query attention, and query sequences
// too long to stage at once.  Built for 1, 2, 4 and 8 key chunks.
#include "atx_attn_bwd_kernels.hpp"

namespace atx {
namespace {

template <typename T, int D>
int loop_nkc(int nkc, int grid, size_t lds, hipStream_t st, const BwdArgs& a) {
    switch (nkc) {
        case 1: return launch_bwd(attn_bwd_16bit<T, D, 1, true>, grid, lds, st, a);
        case 2: return launch_bwd(attn_bwd_16bit<T, D, 2, true>, grid, lds, st, a);
        case 4: return launch_bwd(attn_bwd_16bit<T, D, 4, true>, grid, lds, st, a);
        case 8: return launch_bwd(attn_bwd_16bit<T, D, 8, true>, grid, lds, st, a);
        default: ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: %d key chunks (1, 2, 4, 8 in this variant)", nkc);
    }
}

template <typename T>
int loop_d(int D, int nkc, int grid, size_t lds, hipStream_t st, const BwdArgs& a) {
    switch (D) {
        case 16: return loop_nkc<T, 16>(nkc, grid, lds, st, a);
        case 32: return loop_nkc<T, 32>(nkc, grid, lds, st, a);
        case 48: return loop_nkc<T, 48>(nkc, grid, lds, st, a);
        case 64: return loop_nkc<T, 64>(nkc, grid, lds, st, a);
        case 80: return loop_nkc<T, 80>(nkc, grid, lds, st, a);
        case 96: return loop_nkc<T, 96>(nkc, grid, lds, st, a);
        case 112: return loop_nkc<T, 112>(nkc, grid, lds, st, a);
        case 128: return loop_nkc<T, 128>(nkc, grid, lds, st, a);
        default: ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: head_dim %d not supported", D);
    }
}

}  // namespace

int dispatch_bwd16_loop(bool bf16, int D, int nkc, int grid, size_t lds, hipStream_t st, const BwdArgs& a) {
    return bf16 ? loop_d<__bf16>(D, nkc, grid, lds, st, a) : loop_d<_Float16>(D, nkc, grid, lds, st, a);
}

}  // namespace atx
