// fp32 backward of the key-query policy head for gfx950: the same gradient
// as atx_kq_bwd.hip (dq = scale * dL k, dk = scale * dL^T q, dL the
// gradient of the masked logits) with fp32 q, k and fp32 products
// (v_mfma_f32_16x16x4_f32) -- the precision the reference's Move trainer
// runs its policy head in (stratego/training/move_trainer.py:115-140; its
// trainers never enter the AMP helper).
//
// One workgroup (8 waves) per sample.  dL is kept in LDS as fp32 [RP x RP];
// q and k are staged as fp32 rows of a DC-column slice (DC = 16 or 32; 64
// spills registers at 128 squares), one slice after another.  Rows of 4-float chunks are XOR-swizzled
// (chunk ^ hsw(r)) so that both the 16-byte row reads and the single-element
// "transposed" reads stay spread over the banks.  An MFMA k-step covers one
// element of a 4-float chunk per lane group: the sums over squares run in
// the order (chunk, element), the same for both operands.
#include "atx_kq_bwd.hpp"

namespace atx {
namespace {

constexpr int kThreads = kKqBwdThreads;
constexpr int kWaves = kKqBwdWaves;

template <int W>  // row width in floats
constexpr int kHswMaskW = ((W / 4) % 16 == 0) ? 15 : ((W / 4) % 8 == 0) ? 7 : 3;
template <int W>
__device__ inline int hsw_w(int r) {
    return (((r & 3) << 2) | ((r >> 2) & 3)) & kHswMaskW<W>;
}
template <int W>
__device__ inline int fchunk(int r, int ch) {  // float offset of row r, 4-float chunk ch
    return r * W + ((ch ^ hsw_w<W>(r)) << 2);
}
template <int W>
__device__ inline int felem(int r, int c) {  // float offset of row r, column c
    return r * W + (((c >> 2) ^ hsw_w<W>(r)) << 2) + (c & 3);
}

// RP = squares staged (S <= RP, a multiple of 16); DC = slice width
// (floats).  RP = 112 with 16-column slices (97 to 112 squares, the
// reference's 100 and 101): 63 KB of LDS and at most 128 VGPRs, so two
// workgroups share a CU and one sample's loads and stores run under the
// other's products; the other shapes take 64 to 128 KB, one per CU.
template <int RP>
constexpr int kq_bwd_fp32_occ() {
    return RP == 112 ? 4 : 2;
}
template <int DC, int RP, bool PROBS>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(kq_bwd_fp32_occ<RP>(), 8)))
void kq_bwd_fp32(KqBwdArgs a) {
    constexpr int CH4 = DC / 4;   // 4-float chunks per q / k slice row
    constexpr int NDT = DC / 16;  // output tiles of the slice
    constexpr int QD = DC / 4;    // contiguous outputs per lane
    constexpr int NC = RP / 16;   // 16-square groups of the sums

    lds_t* const sg = lds_base();             // dL, fp32 [RP x RP]
    lds_t* const sq = sg + RP * RP * 4;       // q slice [RP x DC]
    lds_t* const sk = sq + RP * DC * 4;       // k slice
    lds_t* const sred = sk + RP * DC * 4;     // kWaves floats

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int m = lane & 15, g = lane >> 4;
    const int b = blockIdx.x;
    const int S = a.S;

    kq_bwd_dl<RP, PROBS>(
        a, b, sred,
        [&](int i, int c, const float (&dl)[8]) {
            lds_st16(sg + fchunk<RP>(i, 2 * c) * 4, __builtin_bit_cast(u32x4, f32x4{dl[0], dl[1], dl[2], dl[3]}));
            lds_st16(sg + fchunk<RP>(i, 2 * c + 1) * 4, __builtin_bit_cast(u32x4, f32x4{dl[4], dl[5], dl[6], dl[7]}));
        },
        [&](int i, int j, float v) { lds_st4(sg + felem<RP>(i, j) * 4, __builtin_bit_cast(uint32_t, v)); },
        sg, RP * RP * 4);  // dL: free until phase 1 ends

    const rsrc_t rq = make_rsrc(static_cast<const float*>(a.q) + b * a.qsb, (uint32_t)(((S - 1) * a.qss + a.Dfull) * 4));
    const rsrc_t rk = make_rsrc(static_cast<const float*>(a.k) + b * a.ksb, (uint32_t)(((S - 1) * a.kss + a.Dfull) * 4));
    const rsrc_t rdq = make_rsrc(static_cast<const float*>(a.dq) + b * a.dqsb, (uint32_t)(((S - 1) * a.dqss + a.Dfull) * 4));
    const rsrc_t rdk = make_rsrc(static_cast<const float*>(a.dk) + b * a.dksb, (uint32_t)(((S - 1) * a.dkss + a.Dfull) * 4));
    auto dcol = [&](int dt) { return (m >> 2) * QD + 4 * dt + (m & 3); };
    auto ld_elem = [&](const lds_t* base, int r, int c) {
        return __builtin_bit_cast(float, lds_ld4(base + felem<DC>(r, c) * 4));
    };
    const int ntile = (S + 15) >> 4;
    const int ncs = min(NC, ntile);  // 16-square chunks holding squares < S
    // q / k rows of a slice, in registers between the loads and the LDS
    // stores (rows past S read 0): each next slice's loads go out before the
    // current slice's products, so they wait under them
    constexpr int QKU = (RP * CH4 + kThreads - 1) / kThreads;  // chunks per thread and tensor
    u32x4 qn[QKU], kn[QKU];
    auto issue_qk = [&](int c0) {
#pragma unroll
        for (int u = 0; u < QKU; ++u) {
            const int idx = tid + u * kThreads;
            const int r = idx / CH4, c = idx - (idx / CH4) * CH4;
            const bool in = idx < RP * CH4;
            qn[u] = buf_ld16(rq, in ? (uint32_t)(r * a.qss + c0 + c * 4) * 4 : 0xfffffff0u);
            kn[u] = buf_ld16(rk, in ? (uint32_t)(r * a.kss + c0 + c * 4) * 4 : 0xfffffff0u);
        }
    };
    issue_qk(0);

    for (int dc = 0; dc < a.nd; ++dc) {
        const int col0 = dc * DC;
        if (dc > 0) __syncthreads();  // every wave is done with the previous slice
#pragma unroll
        for (int u = 0; u < QKU; ++u) {
            const int idx = tid + u * kThreads;
            const int r = idx / CH4, c = idx - (idx / CH4) * CH4;
            if (idx < RP * CH4) {
                lds_st16(sq + fchunk<DC>(r, c) * 4, qn[u]);
                lds_st16(sk + fchunk<DC>(r, c) * 4, kn[u]);
            }
        }
        __syncthreads();
        if (dc + 1 < a.nd) issue_qk(col0 + DC);
        // wave passes over the output tiles: dq^T tiles 0 .. ntile-1, then dk^T
        for (int t = wave; t < 2 * ntile; t += kWaves) {
            // LDS bases through opaque copies: otherwise every per-lane
            // address of the products is computed once, before the dL phase,
            // and kept live (and spilled) across the whole kernel
            const lds_t* const sgt = lds_opaque(sg);
            const lds_t* const skt = lds_opaque(sk);
            const lds_t* const sqt = lds_opaque(sq);
            f32x4 acc[NDT];
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (t < ntile) {
                // dq^T[d][i] = sum_j k[j][d] dL[i][j]; column i = 16t + m,
                // k-step (c, e) covers j = 16c + 4g' + e
                const int row = t * 16 + m;
                // operands of chunk c + 1 read before the MFMAs of chunk c
                f32x4 dlc;
                float kc[NDT][4];
                auto ld_dq = [&](int c, f32x4& dl, float (&kk)[NDT][4]) {
                    dl = as_f32x4(lds_ld16(sgt + fchunk<RP>(row, 4 * c + g) * 4));
#pragma unroll
                    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                        for (int e = 0; e < 4; ++e) kk[dt][e] = ld_elem(skt, 16 * c + 4 * g + e, dcol(dt));
                };
                ld_dq(0, dlc, kc);
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    if (c >= ncs) break;  // zero rows of dL and k (uniform)
                    f32x4 dln;
                    float kn[NDT][4];
                    if (c + 1 < ncs) ld_dq(c + 1, dln, kn);
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc[dt] = mma_f32(kc[dt][e], dlc[e], acc[dt]);
                    __builtin_amdgcn_sched_barrier(0);
                    dlc = dln;
#pragma unroll
                    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                        for (int e = 0; e < 4; ++e) kc[dt][e] = kn[dt][e];
                }
                const uint32_t base = (uint32_t)(row * a.dqss + col0 + g * QD) * 4;
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt)
                    buf_st16_cached(rdq, base + dt * 16, __builtin_bit_cast(u32x4, f32x4{acc[dt][0] * a.scale,
                                                                                  acc[dt][1] * a.scale,
                                                                                  acc[dt][2] * a.scale,
                                                                                  acc[dt][3] * a.scale}));
            } else {
                // dk^T[d][j] = sum_i q[i][d] dL[i][j]; column j = 16jt + m,
                // k-step (c, e) covers i = 16c + 4g' + e
                const int jt = t - ntile;
                const int col = jt * 16 + m;
                // operands of chunk c + 1 read before the MFMAs of chunk c
                float dlc[4], qc[NDT][4];
                auto ld_dk = [&](int c, float (&dl)[4], float (&qq)[NDT][4]) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        dl[e] = __builtin_bit_cast(float, lds_ld4(sgt + felem<RP>(16 * c + 4 * g + e, col) * 4));
#pragma unroll
                        for (int dt = 0; dt < NDT; ++dt) qq[dt][e] = ld_elem(sqt, 16 * c + 4 * g + e, dcol(dt));
                    }
                };
                ld_dk(0, dlc, qc);
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    if (c >= ncs) break;  // zero rows of dL and q (uniform)
                    float dln[4], qn[NDT][4];
                    if (c + 1 < ncs) ld_dk(c + 1, dln, qn);
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
#pragma unroll
                        for (int dt = 0; dt < NDT; ++dt) acc[dt] = mma_f32(qc[dt][e], dlc[e], acc[dt]);
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        dlc[e] = dln[e];
#pragma unroll
                        for (int dt = 0; dt < NDT; ++dt) qc[dt][e] = qn[dt][e];
                    }
                }
                const uint32_t base = (uint32_t)(col * a.dkss + col0 + g * QD) * 4;
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt)
                    buf_st16_cached(rdk, base + dt * 16, __builtin_bit_cast(u32x4, f32x4{acc[dt][0] * a.scale,
                                                                                  acc[dt][1] * a.scale,
                                                                                  acc[dt][2] * a.scale,
                                                                                  acc[dt][3] * a.scale}));
            }
        }
    }
}

template <typename K>
int launch(K kernel, int grid, size_t lds, hipStream_t st, const KqBwdArgs& a) {
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) ATX_FAIL(ATX_ERR_LAUNCH, "hipFuncSetAttribute(%zu bytes LDS): %s", lds, hipGetErrorString(e));
    }
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kThreads), lds, st, a);
    ATX_CHECK_LAUNCH("atx_kq_bwd launch");
    return ATX_OK;
}

template <int DC, bool PROBS>
int by_rp(int rp, int grid, size_t lds, hipStream_t st, const KqBwdArgs& a) {
    switch (rp) {
        case 64: return launch(kq_bwd_fp32<DC, 64, PROBS>, grid, lds, st, a);
        case 96: return launch(kq_bwd_fp32<DC, 96, PROBS>, grid, lds, st, a);
        case 128: return launch(kq_bwd_fp32<DC, 128, PROBS>, grid, lds, st, a);
        default: ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_kq_bwd: fp32 with %d squares staged, %d-column slices", rp, DC);
    }
}

template <bool PROBS>
int by_dc(int dc, int rp, int grid, size_t lds, hipStream_t st, const KqBwdArgs& a) {
    if (rp == 112) {
        if (dc != 16) ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_kq_bwd: fp32 112 squares need 16-column slices (got %d)", dc);
        return launch(kq_bwd_fp32<16, 112, PROBS>, grid, lds, st, a);
    }
    switch (dc) {
        case 16: return by_rp<16, PROBS>(rp, grid, lds, st, a);
        case 32: return by_rp<32, PROBS>(rp, grid, lds, st, a);
        default: ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_kq_bwd: fp32 slice width %d", dc);
    }
}

}  // namespace

size_t kq_bwd_fp32_lds_bytes(int dslice, int rp) {
    return (size_t)rp * rp * 4 + 2 * (size_t)rp * dslice * 4 + kWaves * 4;
}

int dispatch_kq_bwd_fp32(bool probs, int dslice, int rp, int grid, size_t lds, hipStream_t st, const KqBwdArgs& a) {
    return probs ? by_dc<true>(dslice, rp, grid, lds, st, a) : by_dc<false>(dslice, rp, grid, lds, st, a);
}

}  // namespace atx
