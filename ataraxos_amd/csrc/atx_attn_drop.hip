// Attention dropout: the forward kernels of atx_attn_kernels.hpp built with
// DROP (head_dim 48 and 64, the reference networks' head sizes), and
// atx_dropout_mask, which writes the keep decisions those kernels make.
//
// The reference applies nn.Dropout to the softmax weights in training
// (stratego/networks/attention.py:312-313; FA2's dropout_p, :236-253).  Here
// the decision for weight (b, h, i, j) is a counter-based hash of its flat
// index ((b * H + h) * S_q + i) * S_kv + j under a key derived from the
// caller's (seed, offset): nothing is stored between the forward and the
// backward, which recomputes each decision where it needs it.
#include "atx_attn_kernels.hpp"

namespace atx {
namespace {

template <int D>
int fwd_drop_dim(int dtype, int nkc, int grid, hipStream_t st, const AttnArgs& a) {
    switch (dtype) {
        case ATX_DTYPE_BF16: return dispatch_16bit<__bf16, D, true>(nkc, grid, st, a);
        case ATX_DTYPE_FP16: return dispatch_16bit<_Float16, D, true>(nkc, grid, st, a);
        default: return dispatch_fp32<D, true>(nkc, grid, st, a);
    }
}

// keep[idx] for idx in [0, n): 16 consecutive decisions per thread, one
// 16-byte store when the run is whole and the output 16-byte aligned.
__global__ __launch_bounds__(256) void dropout_mask_kernel(uint8_t* keep, uint64_t n, DropKey k) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x * 16;
    const bool al = ((uintptr_t)keep & 15) == 0;
    for (uint64_t base = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) * 16; base < n; base += stride) {
        if (al && base + 16 <= n) {
            uint32_t w[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                uint32_t v = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    v |= (uint32_t)(drop_hash(base + 4 * q + e, k.k0, k.k1) >= k.thresh) << (8 * e);
                w[q] = v;
            }
            *reinterpret_cast<u32x4*>(keep + base) = u32x4{w[0], w[1], w[2], w[3]};
        } else {
            for (uint64_t i = base; i < n && i < base + 16; ++i) keep[i] = drop_hash(i, k.k0, k.k1) >= k.thresh;
        }
    }
}

}  // namespace

int dispatch_fwd_drop(int dtype, int D, int nkc, int grid, hipStream_t st, const AttnArgs& a) {
    switch (D) {
        case 48: return fwd_drop_dim<48>(dtype, nkc, grid, st, a);
        case 64: return fwd_drop_dim<64>(dtype, nkc, grid, st, a);
    }
    ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_fwd: dropout needs head_dim 48 or 64 (got %d)", D);
}

}  // namespace atx

extern "C" int atx_dropout_mask(int32_t batch, int32_t num_heads, int32_t seq_q, int32_t seq_kv, float p, uint64_t seed,
                                uint64_t offset, uint8_t* keep, void* stream) {
    using namespace atx;
    clear_error();
    if (batch < 1 || num_heads < 1 || seq_q < 1 || seq_kv < 1)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_dropout_mask: sizes must be >= 1 (batch %d, heads %d, seq_q %d, seq_kv %d)",
                 batch, num_heads, seq_q, seq_kv);
    if (!(p >= 0.f && p < 1.f)) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_dropout_mask: p must be in [0, 1) (got %g)", (double)p);
    if (!keep) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_dropout_mask: keep is NULL");
    const uint64_t n = (uint64_t)batch * (uint64_t)num_heads * (uint64_t)seq_q * (uint64_t)seq_kv;
    const uint64_t runs = (n + 15) / 16;
    const uint64_t blocks = (runs + 255) / 256;
    const int grid = (int)(blocks < 65536 ? blocks : 65536);
    hipLaunchKernelGGL(dropout_mask_kernel, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream), keep, n,
                       make_drop_key(p, seed, offset));
    ATX_CHECK_LAUNCH("atx_dropout_mask launch");
    return ATX_OK;
}
