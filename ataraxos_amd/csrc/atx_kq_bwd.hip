// Backward of the key-query policy head for gfx950 (bf16 / fp16 q, k).
//
// Forward (stratego/networks/move_net.py:92-95, plus the callers' softmax):
//   L = scale * q k^T, masked_fill(~mask, -1e10), flattened from-major;
//   P = softmax over the S*S entries (probs mode).
// Given the upstream fp32 gradient G of the logits (or of P), the gradient of
// the masked logits is
//   dL = G                     (logits mode)
//   dL = P * (G - sum(G * P))  (probs mode)
// on legal entries and 0 on illegal ones (masked_fill passes none), and
//   dq = scale * dL k,   dk = scale * dL^T q.
//
// One workgroup (8 waves) per sample.  Phase 1 streams the sample's G (and
// P) rows from HBM, forms dL and stores it as 16-bit MFMA operands in LDS
// ([RP x RP], zero-padded to a multiple of 32); Q and K rows are staged next
// to it.  Phase 2 runs dq^T = K^T dL^T and dk^T = Q^T dL as 16x16x32 MFMA
// tiles, one 16-row output tile per wave pass, with K^T, Q^T and dL (for dk)
// fed by transposing LDS reads.  Rows wider than 128 (the reference's
// policy_d_model = 384, move_net.py:151) are processed in 64-column slices,
// dL staying resident: columns c of dq and dk depend only on columns c of k
// and q.  Every output has one owner and every sum a
// fixed order: the result does not depend on timing.
#include "atx_kq_bwd.hpp"

namespace atx {


namespace {

constexpr int kThreads = 512;
constexpr int kWaves = 8;
constexpr uint32_t kOut = 0xfffffff0u;  // a buffer offset past any slice: loads 0

// Rows of W 16-bit elements: 16-byte chunk c of row r at c ^ ((r >> 1) & 7)
// when a row has 8 or 16 chunks (the 16 rows of an operand read and the
// 4 x 4 rows x column groups of a transposing read land in distinct bank
// groups), else rows padded by one chunk.
template <int W>
constexpr bool kSwzW = (W == 64 || W == 128);
template <int W>
constexpr int row_bytes_w() {
    return kSwzW<W> ? W * 2 : W * 2 + 16;
}
template <int W>
__device__ inline int chunk_off_w(int r, int c) {
    return r * row_bytes_w<W>() + (kSwzW<W> ? (c ^ ((r >> 1) & 7)) : c) * 16;
}
template <int W>
__device__ inline int quad_off_w(int r, int e) {
    return chunk_off_w<W>(r, e >> 3) + (e & 7) * 2;
}

template <int D, int NKC>
constexpr int kq_bwd_occ() {
    return (NKC <= 4 && D <= 64) ? 4 : 2;
}

}  // namespace

inline size_t kq_bwd_lds_bytes(int D, int nkc) {
    const int rp = 32 * nkc;
    const int rs_g = (rp == 64 || rp == 128) ? rp * 2 : rp * 2 + 16;
    const int rs = (D == 64 || D == 128) ? D * 2 : D * 2 + 16;
    return (size_t)rp * rs_g + (size_t)2 * rp * rs + kWaves * 4;
}

// NKC = 32-square chunks (S <= 32 * NKC); PROBS: G is the gradient of P;
// D = the column slice width (a.nd slices of it make a row).
template <typename T, int D, int NKC, bool PROBS>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(kq_bwd_occ<D, NKC>(), 8)))
void kq_bwd_16bit(KqBwdArgs a) {
    using M = Mfma16<T>;
    constexpr int RP = 32 * NKC;     // dL rows / columns and Q / K rows staged
    constexpr int GC = RP / 8;       // 16-byte chunks per dL row
    constexpr int CH = D / 8;        // 16-byte chunks per Q / K row
    constexpr int NDT = D / 16;      // head-dim output tiles
    constexpr int QD = D / 4;        // contiguous outputs per lane
    constexpr int RSG = row_bytes_w<RP>();
    constexpr int RS = row_bytes_w<D>();
    constexpr int PERT = (RP * GC + kThreads - 1) / kThreads;  // dL chunks per thread

    lds_t* const sg = lds_base();
    lds_t* const sq = sg + RP * RSG;
    lds_t* const sk = sq + RP * RS;
    lds_t* const sred = sk + RP * RS;  // kWaves floats

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int m = lane & 15, g = lane >> 4;
    const int b = blockIdx.x;
    const int S = a.S;

    const rsrc_t rq = make_rsrc(static_cast<const T*>(a.q) + b * a.qsb, (uint32_t)(((S - 1) * a.qss + a.Dfull) * 2));
    const rsrc_t rk = make_rsrc(static_cast<const T*>(a.k) + b * a.ksb, (uint32_t)(((S - 1) * a.kss + a.Dfull) * 2));
    // Q and K rows of a column slice, in registers between the loads and the
    // LDS stores (rows past S read 0): the first slice's loads go out before
    // phase 1, each next slice's before the current slice's products, so the
    // loads wait under other work.
    constexpr int QKU = (RP * CH + kThreads - 1) / kThreads;  // chunks per thread and tensor
    u32x4 qn[QKU], kn[QKU];
    auto issue_qk = [&](int c0) {
#pragma unroll
        for (int u = 0; u < QKU; ++u) {
            const int idx = tid + u * kThreads;
            const int r = idx / CH, c = idx - (idx / CH) * CH;
            const bool in = idx < RP * CH;
            qn[u] = buf_ld16(rq, in ? (uint32_t)(r * a.qss + c0 + c * 8) * 2 : kOut);
            kn[u] = buf_ld16(rk, in ? (uint32_t)(r * a.kss + c0 + c * 8) * 2 : kOut);
        }
    };
    auto commit_qk = [&]() {
#pragma unroll
        for (int u = 0; u < QKU; ++u) {
            const int idx = tid + u * kThreads;
            const int r = idx / CH, c = idx - (idx / CH) * CH;
            if (idx < RP * CH) {
                lds_st16(sq + chunk_off_w<D>(r, c), qn[u]);
                lds_st16(sk + chunk_off_w<D>(r, c), kn[u]);
            }
        }
    };
    issue_qk(0);

    lds_t* const sg_ = sg;
    kq_bwd_dl<RP, PROBS>(
        a, b, sred,
        [&](int i, int c, const float (&dl)[8]) {
            lds_st16(sg_ + chunk_off_w<RP>(i, c), u32x4{M::pack2(dl[0], dl[1]), M::pack2(dl[2], dl[3]),
                                                           M::pack2(dl[4], dl[5]), M::pack2(dl[6], dl[7])});
        },
        [&](int i, int j, float v) { lds_st2(sg_ + quad_off_w<RP>(i, j), M::pack2(v, 0.f)); },
        sg_, RP * RSG + 2 * RP * RS);  // dL and the q / k slices: free until phase 1 ends

    // ---- phase 2: dq^T = K^T dL^T, dk^T = Q^T dL --------------------------------
    // Transposing reads of Q / K: input lane a4 + 4t of a 16-lane group points
    // at row 4g + t, elements a4*QD + 4dt .. +3, which hands lane m the four
    // rows 4g .. 4g+3 of head-dim (m/4)*QD + 4dt + m%4.
    int troff[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) troff[dt] = quad_off_w<D>(4 * g + (m >> 2), (m & 3) * QD + 4 * dt);
    const T* const dqbase = static_cast<const T*>(a.dq) + b * a.dqsb;
    const T* const dkbase = static_cast<const T*>(a.dk) + b * a.dksb;
    const rsrc_t rdq = make_rsrc(dqbase, (uint32_t)(((S - 1) * a.dqss + a.Dfull) * 2));
    const rsrc_t rdk = make_rsrc(dkbase, (uint32_t)(((S - 1) * a.dkss + a.Dfull) * 2));
    int col0 = 0;  // first column of the current slice
    auto store_row = [&](rsrc_t r, int ss, int row, const f32x4 (&x)[NDT]) {
        const float mul = a.scale;
        const uint32_t base = (uint32_t)(row * ss + col0 + g * QD) * 2;
        if constexpr (QD % 8 == 0) {
#pragma unroll
            for (int dt = 0; dt < NDT; dt += 2)
                buf_st16_cached(r, base + dt * 8,
                                u32x4{M::pack2(x[dt][0] * mul, x[dt][1] * mul), M::pack2(x[dt][2] * mul, x[dt][3] * mul),
                                      M::pack2(x[dt + 1][0] * mul, x[dt + 1][1] * mul),
                                      M::pack2(x[dt + 1][2] * mul, x[dt + 1][3] * mul)});
        } else {
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
                buf_st8_cached(r, base + dt * 8,
                               u32x2{M::pack2(x[dt][0] * mul, x[dt][1] * mul), M::pack2(x[dt][2] * mul, x[dt][3] * mul)});
        }
    };
    const int ntile = (S + 15) >> 4;
    for (int dc = 0; dc < a.nd; ++dc) {
    col0 = dc * D;
    if (dc > 0) __syncthreads();  // every wave is done with the previous slice
    commit_qk();
    __syncthreads();
    if (dc + 1 < a.nd) issue_qk(col0 + D);
    for (int t = wave; t < 2 * ntile; t += kWaves) {
        f32x4 acc[NDT];
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (t < ntile) {
            // dq^T tile: columns = from-squares 16t + m; k = to-squares
            const int row = t * 16 + m;
#pragma unroll
            for (int c = 0; c < NKC; ++c) {
                const u32x2 blo = lds_ld8(sg + quad_off_w<RP>(row, 32 * c + 4 * g));
                const u32x2 bhi = lds_ld8(sg + quad_off_w<RP>(row, 32 * c + 16 + 4 * g));
                const u32x4 bop = {blo[0], blo[1], bhi[0], bhi[1]};
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) {
                    const u32x2 lo = lds_ld8_tr16(sk + 32 * c * RS + troff[dt]);
                    const u32x2 hi = lds_ld8_tr16(sk + (32 * c + 16) * RS + troff[dt]);
                    acc[dt] = M::mma(u32x4{lo[0], lo[1], hi[0], hi[1]}, bop, acc[dt]);
                }
            }
            store_row(rdq, a.dqss, row, acc);
        } else {
            // dk^T tile: columns = to-squares 16jt + m; k = from-squares
            const int jt = t - ntile;
            const int goff = quad_off_w<RP>(4 * g + (m >> 2), jt * 16 + 4 * (m & 3));
#pragma unroll
            for (int c = 0; c < NKC; ++c) {
                const u32x2 blo = lds_ld8_tr16(sg + 32 * c * RSG + goff);
                const u32x2 bhi = lds_ld8_tr16(sg + (32 * c + 16) * RSG + goff);
                const u32x4 bop = {blo[0], blo[1], bhi[0], bhi[1]};
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) {
                    const u32x2 lo = lds_ld8_tr16(sq + 32 * c * RS + troff[dt]);
                    const u32x2 hi = lds_ld8_tr16(sq + (32 * c + 16) * RS + troff[dt]);
                    acc[dt] = M::mma(u32x4{lo[0], lo[1], hi[0], hi[1]}, bop, acc[dt]);
                }
            }
            store_row(rdk, a.dkss, jt * 16 + m, acc);
        }
    }
    }
}

namespace {

template <typename K>
int launch_kq_bwd(K kernel, int grid, size_t lds, hipStream_t st, const KqBwdArgs& a) {
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) ATX_FAIL(ATX_ERR_LAUNCH, "hipFuncSetAttribute(%zu bytes LDS): %s", lds, hipGetErrorString(e));
    }
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kThreads), lds, st, a);
    ATX_CHECK_LAUNCH("atx_kq_bwd launch");
    return ATX_OK;
}

template <typename T, int D, bool PROBS>
int dispatch_kq_bwd_nkc(int nkc, int grid, size_t lds, hipStream_t st, const KqBwdArgs& a) {
    switch (nkc) {
        case 2: return launch_kq_bwd(kq_bwd_16bit<T, D, 2, PROBS>, grid, lds, st, a);
        case 3: return launch_kq_bwd(kq_bwd_16bit<T, D, 3, PROBS>, grid, lds, st, a);
        case 4: return launch_kq_bwd(kq_bwd_16bit<T, D, 4, PROBS>, grid, lds, st, a);
        default: ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_kq_bwd: %d 32-square chunks", nkc);
    }
}

template <typename T, bool PROBS>
int dispatch_kq_bwd(int D, int nkc, int grid, size_t lds, hipStream_t st, const KqBwdArgs& a) {
    switch (D) {
        case 16: return dispatch_kq_bwd_nkc<T, 16, PROBS>(nkc, grid, lds, st, a);
        case 32: return dispatch_kq_bwd_nkc<T, 32, PROBS>(nkc, grid, lds, st, a);
        case 48: return dispatch_kq_bwd_nkc<T, 48, PROBS>(nkc, grid, lds, st, a);
        case 64: return dispatch_kq_bwd_nkc<T, 64, PROBS>(nkc, grid, lds, st, a);
        case 80: return dispatch_kq_bwd_nkc<T, 80, PROBS>(nkc, grid, lds, st, a);
        case 96: return dispatch_kq_bwd_nkc<T, 96, PROBS>(nkc, grid, lds, st, a);
        case 112: return dispatch_kq_bwd_nkc<T, 112, PROBS>(nkc, grid, lds, st, a);
        case 128: return dispatch_kq_bwd_nkc<T, 128, PROBS>(nkc, grid, lds, st, a);
        default: ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_kq_bwd: dim %d not supported", D);
    }
}

}  // namespace
}  // namespace atx

extern "C" int atx_kq_bwd(const AtxKqBwdParams* p, void* stream) {
    using namespace atx;
    clear_error();
    if (!p) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_kq_bwd: params is NULL");
    if (p->abi_version != ATX_ABI_VERSION)
        ATX_FAIL(ATX_ERR_ABI, "atx_kq_bwd: abi_version %d, library is %d", p->abi_version, ATX_ABI_VERSION);
    if (p->dtype != ATX_DTYPE_BF16 && p->dtype != ATX_DTYPE_FP16 && p->dtype != ATX_DTYPE_FP32)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_kq_bwd: unknown dtype %d", p->dtype);
    const bool f32 = p->dtype == ATX_DTYPE_FP32;
    const int es = f32 ? 4 : 2;
    if (p->batch < 1 || p->seq < 1 || p->dim < 1)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_kq_bwd: sizes must be >= 1 (batch %d, seq %d, dim %d)", p->batch, p->seq,
                 p->dim);
    if (p->out_mode != ATX_KQ_OUT_PROBS && p->out_mode != ATX_KQ_OUT_LOGITS)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_kq_bwd: unknown out_mode %d", p->out_mode);
    const bool probs = p->out_mode == ATX_KQ_OUT_PROBS;
    if (!p->q || !p->k || !p->grad || !p->dq || !p->dk || (probs && !p->probs))
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_kq_bwd: null tensor pointer");
    if (!(p->scale > 0.f) || p->scale == __builtin_inff())
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_kq_bwd: scale must be finite and > 0 (got %g)", (double)p->scale);
    if (p->seq > 128) ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_kq_bwd: seq %d not supported (<= 128)", p->seq);
    if (p->dim % 16 != 0 || (!f32 && p->dim > 128 && p->dim % 64 != 0) || p->dim > 4096)
        ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_kq_bwd: dim %d not supported (multiple of 16 up to 128, of 64 up to 4096%s)",
                 p->dim, f32 ? "" : "; fp32: of 16 up to 4096");
    const int D = p->dim, S = p->seq;
    auto rows16 = [&](const void* base, int64_t sb, int64_t ss) {
        return aligned16(base) && ((sb * es) & 15) == 0 && ((ss * es) & 15) == 0;
    };
    // Row strides of a one-row sample are never used.
    auto sstride = [&](int64_t s) { return S == 1 ? (int64_t)D : s; };
    const int64_t qss = sstride(p->q_stride_s), kss = sstride(p->k_stride_s);
    const int64_t dqss = sstride(p->dq_stride_s), dkss = sstride(p->dk_stride_s);
    if (!rows16(p->q, p->q_stride_b, qss) || !rows16(p->k, p->k_stride_b, kss) || !rows16(p->dq, p->dq_stride_b, dqss) ||
        !rows16(p->dk, p->dk_stride_b, dkss))
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_kq_bwd: every q/k/dq/dk row must start on a 16-byte boundary");
    for (int64_t s : {qss, kss, dqss, dkss})
        if (s < 0 || (int64_t)(S + 32) * s * es + D * es > 0x7fffffffLL)
            ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_kq_bwd: row strides must be >= 0 and one sample < 2 GiB");
    if (dqss < D || dkss < D) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_kq_bwd: dq/dk rows overlap");
    if (((uintptr_t)p->grad & 3) != 0 || p->grad_stride_b < (int64_t)S * S ||
        (probs && (((uintptr_t)p->probs & 3) != 0 || p->probs_stride_b < (int64_t)S * S)))
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_kq_bwd: grad/probs must be 4-byte aligned with stride >= seq*seq");
    if (p->mask && (p->mask_stride_s < 0 || p->mask_stride_b < 0 || (int64_t)S * p->mask_stride_s + S > 0x7fffffffLL))
        ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_kq_bwd: mask strides must be >= 0 and one sample < 2 GiB");

    KqBwdArgs a;
    a.q = p->q; a.k = p->k;
    a.qsb = p->q_stride_b; a.ksb = p->k_stride_b;
    a.qss = (int)qss; a.kss = (int)kss;
    a.mask = p->mask;
    a.msb = p->mask_stride_b;
    a.mss = (int)p->mask_stride_s;
    a.grad = p->grad; a.gsb = p->grad_stride_b;
    a.probs = probs ? p->probs : nullptr;
    a.psb = probs ? p->probs_stride_b : 0;
    a.dq = p->dq; a.dk = p->dk;
    a.dqsb = p->dq_stride_b; a.dksb = p->dk_stride_b;
    a.dqss = (int)dqss; a.dkss = (int)dkss;
    a.S = S;
    a.Dfull = D;
    const int nkc = S <= 64 ? 2 : (S + 31) / 32;
    // fp32 at 97 to 112 squares: 112 staged, 16-column slices (two
    // workgroups per CU); other fp32 shapes 32 * nkc staged
    const int rp32 = (S > 96 && S <= 112) ? 112 : 32 * nkc;
    // 16-bit: rows up to 128 wide in one slice, wider ones in 64-column
    // slices; fp32: slices of 32 or 16 columns
    const int dslice = f32 ? (D % 32 == 0 && rp32 != 112 ? 32 : 16) : (D <= 128 ? D : 64);
    a.nd = D / dslice;
    a.scale = p->scale;
    a.mask_al4 = p->mask && ((uintptr_t)p->mask & 3) == 0 && (p->mask_stride_b & 3) == 0 && (p->mask_stride_s & 3) == 0;
    a.grad_vec = S % 4 == 0 && aligned16(p->grad) && (p->grad_stride_b & 3) == 0 &&
                 (!probs || (aligned16(p->probs) && (p->probs_stride_b & 3) == 0));
    const size_t lds = f32 ? kq_bwd_fp32_lds_bytes(dslice, rp32) : kq_bwd_lds_bytes(dslice, nkc);
    if (lds > 160 * 1024)
        ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_kq_bwd: seq %d, dim %d need %zu bytes of LDS (> 160 KiB)", S, D, lds);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (f32) return dispatch_kq_bwd_fp32(probs, dslice, rp32, p->batch, lds, st, a);
    if (p->dtype == ATX_DTYPE_BF16)
        return probs ? dispatch_kq_bwd<__bf16, true>(dslice, nkc, p->batch, lds, st, a)
                     : dispatch_kq_bwd<__bf16, false>(dslice, nkc, p->batch, lds, st, a);
    return probs ? dispatch_kq_bwd<_Float16, true>(dslice, nkc, p->batch, lds, st, a)
                 : dispatch_kq_bwd<_Float16, false>(dslice, nkc, p->batch, lds, st, a);
}
