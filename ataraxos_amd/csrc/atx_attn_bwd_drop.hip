// The attention backward with dropout: the LOOP variants of
// atx_attn_bwd_kernels.hpp (one workgroup per (batch, KV head), query rows in
// blocks) built with DROP, for head_dim 48 and 64 and 1, 2, 4, 8 key chunks.
// Each kernel recomputes the forward's keep decisions from the same
// (seed, offset) key; nothing is read from a stored mask.
#include "atx_attn_bwd_kernels.hpp"

namespace atx {
namespace {

template <int D>
int bwd_drop_nkc(int dtype, int nkc, int grid, size_t lds, hipStream_t st, const BwdArgs& a) {
#define ATX_BWD_DROP_CASE(N)                                                                        \
    case N:                                                                                         \
        switch (dtype) {                                                                            \
            case ATX_DTYPE_BF16: return launch_bwd(attn_bwd_16bit<__bf16, D, N, true, true>, grid, lds, st, a);   \
            case ATX_DTYPE_FP16: return launch_bwd(attn_bwd_16bit<_Float16, D, N, true, true>, grid, lds, st, a); \
            default: return launch_bwd(attn_bwd_fp32<D, N, true, true>, grid, lds, st, a);          \
        }
    switch (nkc) {
        ATX_BWD_DROP_CASE(1)
        ATX_BWD_DROP_CASE(2)
        ATX_BWD_DROP_CASE(4)
        ATX_BWD_DROP_CASE(8)
    }
#undef ATX_BWD_DROP_CASE
    ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: %d key chunks (1, 2, 4, 8 with dropout)", nkc);
}

}  // namespace

int dispatch_bwd_drop(int dtype, int D, int nkc, int grid, size_t lds, hipStream_t st, const BwdArgs& a) {
    switch (D) {
        case 48: return bwd_drop_nkc<48>(dtype, nkc, grid, lds, st, a);
        case 64: return bwd_drop_nkc<64>(dtype, nkc, grid, lds, st, a);
    }
    ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: dropout needs head_dim 48 or 64 (got %d)", D);
}

}  // namespace atx
