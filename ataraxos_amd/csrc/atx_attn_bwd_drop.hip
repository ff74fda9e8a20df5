// The attention backward with dropout (atx_attn_bwd_kernels.hpp built with
// DROP), head_dim 48 and 64: the 16-bit kernels here, both variants (every
// query staged at once for 1..8 key chunks; LOOP for 1, 2, 4, 8), and the
// fp32 ones in atx_attn_bwd_drop_fp32.hip.  Each kernel recomputes the
// forward's keep decisions from the same (seed, offset) key; nothing is read
// from a stored mask.
#include "atx_attn_bwd_kernels.hpp"

namespace atx {
namespace {

template <typename T, int D>
int drop16_nkc(bool loop, int nkc, int grid, size_t lds, hipStream_t st, const BwdArgs& a) {
    if (loop) {
        switch (nkc) {
            case 1: return launch_bwd(attn_bwd_16bit<T, D, 1, true, true>, grid, lds, st, a);
            case 2: return launch_bwd(attn_bwd_16bit<T, D, 2, true, true>, grid, lds, st, a);
            case 4: return launch_bwd(attn_bwd_16bit<T, D, 4, true, true>, grid, lds, st, a);
            case 8: return launch_bwd(attn_bwd_16bit<T, D, 8, true, true>, grid, lds, st, a);
        }
        ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: %d key chunks (1, 2, 4, 8 in this variant)", nkc);
    }
    switch (nkc) {
        case 1: return launch_bwd(attn_bwd_16bit<T, D, 1, false, true>, grid, lds, st, a);
        case 2: return launch_bwd(attn_bwd_16bit<T, D, 2, false, true>, grid, lds, st, a);
        case 3: return launch_bwd(attn_bwd_16bit<T, D, 3, false, true>, grid, lds, st, a);
        case 4: return launch_bwd(attn_bwd_16bit<T, D, 4, false, true>, grid, lds, st, a);
        case 5: return launch_bwd(attn_bwd_16bit<T, D, 5, false, true>, grid, lds, st, a);
        case 6: return launch_bwd(attn_bwd_16bit<T, D, 6, false, true>, grid, lds, st, a);
        case 7: return launch_bwd(attn_bwd_16bit<T, D, 7, false, true>, grid, lds, st, a);
        case 8: return launch_bwd(attn_bwd_16bit<T, D, 8, false, true>, grid, lds, st, a);
    }
    ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: seq_kv needs %d 32-key chunks (<= 8)", nkc);
}

template <typename T>
int drop16_d(bool loop, int D, int nkc, int grid, size_t lds, hipStream_t st, const BwdArgs& a) {
    switch (D) {
        case 48: return drop16_nkc<T, 48>(loop, nkc, grid, lds, st, a);
        case 64: return drop16_nkc<T, 64>(loop, nkc, grid, lds, st, a);
    }
    ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: dropout needs head_dim 48 or 64 (got %d)", D);
}

}  // namespace

int dispatch_bwd_drop(int dtype, bool loop, int D, int nkc, int grid, size_t lds, hipStream_t st, const BwdArgs& a) {
    switch (dtype) {
        case ATX_DTYPE_BF16: return drop16_d<__bf16>(loop, D, nkc, grid, lds, st, a);
        case ATX_DTYPE_FP16: return drop16_d<_Float16>(loop, D, nkc, grid, lds, st, a);
    }
    return dispatch_bwd_drop_fp32(loop, D, nkc, grid, lds, st, a);
}

}  // namespace atx
