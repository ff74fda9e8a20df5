// fp32 instantiations of the attention backward (atx_attn_bwd_kernels.hpp):
// v_mfma_f32_16x16x4_f32 for 1, 2, 4 and 8 key chunks.  This file builds the
// variant that stages every query at once; atx_attn_bwd_fp32_loop.hip
// includes it with ATX_BWD_FP32_LOOP defined for the one that loops over
// query heads and blocks of query rows (two translation units that compile
// in parallel).
// The reference's trainers never enter its AMP helper
// (stratego/training/amp.py is imported by none of them), so its Move, Setup
// and Belief networks train in fp32: this is the backward of that
// (stratego/training/move_trainer.py:140).
#include "atx_attn_bwd_kernels.hpp"

namespace atx {
namespace {

template <int D, bool LOOP>
int f32_nkc(int nkc, int grid, size_t lds, hipStream_t st, const BwdArgs& a) {
    switch (nkc) {
        case 1: return launch_bwd(attn_bwd_fp32<D, 1, LOOP>, grid, lds, st, a);
        case 2: return launch_bwd(attn_bwd_fp32<D, 2, LOOP>, grid, lds, st, a);
        case 4: return launch_bwd(attn_bwd_fp32<D, 4, LOOP>, grid, lds, st, a);
        case 8: return launch_bwd(attn_bwd_fp32<D, 8, LOOP>, grid, lds, st, a);
        default: ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: %d key chunks (fp32: 1, 2, 4, 8)", nkc);
    }
}

template <bool LOOP>
int f32_d(int D, int nkc, int grid, size_t lds, hipStream_t st, const BwdArgs& a) {
    switch (D) {
        case 16: return f32_nkc<16, LOOP>(nkc, grid, lds, st, a);
        case 32: return f32_nkc<32, LOOP>(nkc, grid, lds, st, a);
        case 48: return f32_nkc<48, LOOP>(nkc, grid, lds, st, a);
        case 64: return f32_nkc<64, LOOP>(nkc, grid, lds, st, a);
        case 80: return f32_nkc<80, LOOP>(nkc, grid, lds, st, a);
        case 96: return f32_nkc<96, LOOP>(nkc, grid, lds, st, a);
        case 112: return f32_nkc<112, LOOP>(nkc, grid, lds, st, a);
        case 128: return f32_nkc<128, LOOP>(nkc, grid, lds, st, a);
        default: ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: head_dim %d not supported", D);
    }
}

}  // namespace

#ifdef ATX_BWD_FP32_LOOP
int dispatch_bwd_fp32_loop(int D, int nkc, int grid, size_t lds, hipStream_t st, const BwdArgs& a) {
    return f32_d<true>(D, nkc, grid, lds, st, a);
}
#else
int dispatch_bwd_fp32(bool loop, int D, int nkc, int grid, size_t lds, hipStream_t st, const BwdArgs& a) {
    return loop ? dispatch_bwd_fp32_loop(D, nkc, grid, lds, st, a) : f32_d<false>(D, nkc, grid, lds, st, a);
}
#endif

}  // namespace atx
