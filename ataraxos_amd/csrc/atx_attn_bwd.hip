// Attention backward for gfx950 (bf16 / fp16): dQ, dK, dV of
//   S = scale * Q K^T (masked), P = softmax(S), O = P V
// given Q, K, V, O and dO -- the gradient the reference's training step
// (stratego/training/move_trainer.py:140) takes through
// stratego/networks/attention.py:281-316.  With delta_q = sum_d O[q,d] dO[q,d]:
//   dP = dO V^T,  dS = P * (dP - delta),
//   dQ = scale * dS K,  dK = scale * dS^T Q,  dV = P^T dO.
//
// One workgroup (8 waves) per (batch, head), everything for that pair
// resident in LDS: K, V, Q and dO rows in one layout that serves both 16-byte
// row reads and the transposing reads (ds_read_b64_tr_b16), plus the
// per-query log-sum-exp and delta.
//  * Phase 1, one wave per 16-query tile, in the forward's orientation
//    (S^T = K Q^T: each lane owns one query): delta from the O tile (read
//    straight into registers) and the dO tile, the softmax and its
//    log-sum-exp, then dP^T = V dO^T, dS^T, and dQ^T = K^T dS^T with dS^T
//    fed from registers the way the forward feeds P^T.
//  * Phase 2, one wave per 16-key tile (S = Q K^T: each lane owns one key):
//    recompute P from the log-sum-exp, dP = dO V^T and dS, and accumulate
//    dV^T = dO^T P and dK^T = Q^T dS over pairs of query tiles, with P and dS
//    fed from registers.
// Every output tile has one owner: no atomics, no cross-wave reductions, and
// the result does not depend on timing.
// Masked scores get dS = 0 (the gradient of masked_fill); a query that sees
// no key has P = NaN, so its dO reaches dV as NaN, as autograd through the
// reference's math gives.  Key tiles that are fully usable (or unusable) for
// a whole wave skip the per-score masking (or the whole tile).
#include "atx_attn_bwd_kernels.hpp"

namespace atx {
namespace {

template <typename T, int D>
int dispatch_bwd_nkc(int nkc, int grid, size_t lds, hipStream_t st, const BwdArgs& a) {
    switch (nkc) {
        case 1: return launch_bwd(attn_bwd_16bit<T, D, 1, false>, grid, lds, st, a);
        case 2: return launch_bwd(attn_bwd_16bit<T, D, 2, false>, grid, lds, st, a);
        case 3: return launch_bwd(attn_bwd_16bit<T, D, 3, false>, grid, lds, st, a);
        case 4: return launch_bwd(attn_bwd_16bit<T, D, 4, false>, grid, lds, st, a);
        case 5: return launch_bwd(attn_bwd_16bit<T, D, 5, false>, grid, lds, st, a);
        case 6: return launch_bwd(attn_bwd_16bit<T, D, 6, false>, grid, lds, st, a);
        case 7: return launch_bwd(attn_bwd_16bit<T, D, 7, false>, grid, lds, st, a);
        case 8: return launch_bwd(attn_bwd_16bit<T, D, 8, false>, grid, lds, st, a);
        default: ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: seq_kv needs %d 32-key chunks (<= 8)", nkc);
    }
}

template <typename T>
int dispatch_bwd16(int D, int nkc, int grid, size_t lds, hipStream_t st, const BwdArgs& a) {
    switch (D) {
        case 16: return dispatch_bwd_nkc<T, 16>(nkc, grid, lds, st, a);
        case 32: return dispatch_bwd_nkc<T, 32>(nkc, grid, lds, st, a);
        case 48: return dispatch_bwd_nkc<T, 48>(nkc, grid, lds, st, a);
        case 64: return dispatch_bwd_nkc<T, 64>(nkc, grid, lds, st, a);
        case 80: return dispatch_bwd_nkc<T, 80>(nkc, grid, lds, st, a);
        case 96: return dispatch_bwd_nkc<T, 96>(nkc, grid, lds, st, a);
        case 112: return dispatch_bwd_nkc<T, 112>(nkc, grid, lds, st, a);
        case 128: return dispatch_bwd_nkc<T, 128>(nkc, grid, lds, st, a);
        default: ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: head_dim %d not supported", D);
    }
}

bool rows16(const void* base, int64_t sb, int64_t ss, int64_t sh, int es) {
    return aligned16(base) && ((sb * es) & 15) == 0 && ((ss * es) & 15) == 0 && ((sh * es) & 15) == 0;
}

}  // namespace
}  // namespace atx

extern "C" int atx_attn_bwd(const AtxAttnBwdParams* p, void* stream) {
    using namespace atx;
    clear_error();
    if (!p) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_bwd: params is NULL");
    if (p->abi_version != ATX_ABI_VERSION)
        ATX_FAIL(ATX_ERR_ABI, "atx_attn_bwd: abi_version %d, library is %d", p->abi_version, ATX_ABI_VERSION);
    if (p->dtype != ATX_DTYPE_BF16 && p->dtype != ATX_DTYPE_FP16 && p->dtype != ATX_DTYPE_FP32)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_bwd: unknown dtype %d", p->dtype);
    const bool f32 = p->dtype == ATX_DTYPE_FP32;
    const int es = f32 ? 4 : 2;
    if (p->batch < 1 || p->seq_q < 1 || p->seq_kv < 1 || p->num_heads < 1 || p->num_kv_heads < 1 || p->head_dim < 1)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_bwd: sizes must be >= 1");
    if (p->num_heads % p->num_kv_heads != 0)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_bwd: num_heads %d not divisible by num_kv_heads %d", p->num_heads,
                 p->num_kv_heads);
    if (!p->q || !p->k || !p->v || !p->o || !p->d_o || !p->dq || !p->dk || !p->dv)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_bwd: null tensor pointer");
    if (!(p->scale > 0.f) || p->scale == __builtin_inff())
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_bwd: scale must be finite and > 0 (got %g)", (double)p->scale);
    if (p->head_dim % 16 != 0 || p->head_dim > 128)
        ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: head_dim %d not supported (multiple of 16, <= 128)", p->head_dim);
    if (p->seq_kv > 256) ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: seq_kv %d not supported (<= 256)", p->seq_kv);
    if (p->seq_q > (1 << 20)) ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: seq_q %d not supported (<= 2^20)", p->seq_q);
    const int64_t grid = (int64_t)p->batch * p->num_kv_heads;  // one workgroup per (batch, KV head)
    if (grid > 0x7fffffff) ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: batch*heads too large");
    // Sequence strides of length-1 sequences are never used.
    auto sstride = [](int64_t s, int seq, int d) { return seq == 1 ? (int64_t)d : s; };
    const int D = p->head_dim;
    const int64_t qss = sstride(p->q_stride_s, p->seq_q, D), oss = sstride(p->o_stride_s, p->seq_q, D);
    const int64_t doss = sstride(p->do_stride_s, p->seq_q, D), dqss = sstride(p->dq_stride_s, p->seq_q, D);
    const int64_t kss = sstride(p->k_stride_s, p->seq_kv, D), vss = sstride(p->v_stride_s, p->seq_kv, D);
    const int64_t dkss = sstride(p->dk_stride_s, p->seq_kv, D), dvss = sstride(p->dv_stride_s, p->seq_kv, D);
    if (!rows16(p->q, p->q_stride_b, qss, p->q_stride_h, es) || !rows16(p->k, p->k_stride_b, kss, p->k_stride_h, es) ||
        !rows16(p->v, p->v_stride_b, vss, p->v_stride_h, es) || !rows16(p->o, p->o_stride_b, oss, p->o_stride_h, es) ||
        !rows16(p->d_o, p->do_stride_b, doss, p->do_stride_h, es) ||
        !rows16(p->dq, p->dq_stride_b, dqss, p->dq_stride_h, es) ||
        !rows16(p->dk, p->dk_stride_b, dkss, p->dk_stride_h, es) ||
        !rows16(p->dv, p->dv_stride_b, dvss, p->dv_stride_h, es))
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_bwd: every row must start on a 16-byte boundary");
    // one (batch, head) slice per descriptor: 32-bit offsets, rows up to the
    // next multiple of 32 past the end; output rows must not overlap
    const int64_t strides_q[] = {qss, oss, doss, dqss}, strides_k[] = {kss, vss, dkss, dvss};
    for (int64_t s : strides_q)
        if (s < 0 || (p->seq_q + 32) * s * es + D * es > 0x7fffffffLL)
            ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: sequence strides must be >= 0 and one slice < 2 GiB");
    for (int64_t s : strides_k)
        if (s < 0 || (p->seq_kv + 32) * s * es + D * es > 0x7fffffffLL)
            ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: sequence strides must be >= 0 and one slice < 2 GiB");
    if (dqss < D || dkss < D || dvss < D)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_bwd: gradient rows overlap");
    if (!(p->dropout_p >= 0.f && p->dropout_p < 1.f))
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_bwd: dropout_p must be in [0, 1) (got %g)", (double)p->dropout_p);
    const bool drop = p->dropout_p > 0.f;
    if (drop && D != 48 && D != 64)
        ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: dropout needs head_dim 48 or 64 (got %d)", D);

    // Variant: every query staged at once (one pass), or LOOP -- query heads
    // of a group and blocks of QB query rows one after another (GQA, or too
    // many query rows for LDS).  The LOOP and fp32 variants exist for 1, 2, 4
    // and 8 key chunks.
    const bool gqa = p->num_heads != p->num_kv_heads;
    const size_t kLds = 160 * 1024;
    const int nkc_exact = (p->seq_kv + 31) / 32;
    const int qalign = f32 ? 16 : 32;  // query rows per staging unit
    const int rq_all = (int)(((int64_t)p->seq_q + qalign - 1) / qalign * qalign);
    auto lds_of = [&](int nkc_, int rq_) {
        return f32 ? bwd_lds_bytes_fp32(D, nkc_ * 32, rq_) : bwd_lds_bytes(D, nkc_ * 32, rq_);
    };
    int nkc = f32 ? bwd_nkc_pow2(nkc_exact) : nkc_exact;
    const bool loop = gqa || p->seq_q > 256 || lds_of(nkc, rq_all) > kLds;
    int qb = 0;
    if (loop) {
        nkc = bwd_nkc_pow2(nkc_exact);
        qb = rq_all < 256 ? rq_all : 256;
        while (qb > qalign && lds_of(nkc, qb) > kLds) qb -= qalign;
    }
    const size_t lds = lds_of(nkc, loop ? qb : rq_all);
    if (lds > kLds)
        ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: seq_kv %d, head_dim %d%s need %zu bytes of LDS (> 160 KiB)",
                 p->seq_kv, D, f32 ? " (fp32)" : "", lds);

    BwdArgs a;
    a.q = p->q; a.k = p->k; a.v = p->v; a.o = p->o; a.dout = p->d_o;
    a.dq = p->dq; a.dk = p->dk; a.dv = p->dv;
    a.qsb = p->q_stride_b; a.qsh = p->q_stride_h; a.ksb = p->k_stride_b; a.ksh = p->k_stride_h;
    a.vsb = p->v_stride_b; a.vsh = p->v_stride_h; a.osb = p->o_stride_b; a.osh = p->o_stride_h;
    a.dosb = p->do_stride_b; a.dosh = p->do_stride_h; a.dqsb = p->dq_stride_b; a.dqsh = p->dq_stride_h;
    a.dksb = p->dk_stride_b; a.dksh = p->dk_stride_h; a.dvsb = p->dv_stride_b; a.dvsh = p->dv_stride_h;
    a.qss = (int)qss; a.kss = (int)kss; a.vss = (int)vss; a.oss = (int)oss;
    a.doss = (int)doss; a.dqss = (int)dqss; a.dkss = (int)dkss; a.dvss = (int)dvss;
    a.kpad = p->key_pad;
    a.kpsb = p->key_pad_stride_b;
    a.H = p->num_heads;
    a.G = p->num_heads / p->num_kv_heads;
    a.QB = qb;
    a.Sq = p->seq_q;
    a.Skv = p->seq_kv;
    a.c2 = p->scale * kLog2e;
    a.scale = p->scale;
    a.causal = p->causal != 0;
    a.drop = make_drop_key(drop ? p->dropout_p : 0.f, p->dropout_seed, p->dropout_offset);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (drop) return dispatch_bwd_drop(p->dtype, loop, D, nkc, (int)grid, lds, st, a);
    if (f32) return dispatch_bwd_fp32(loop, D, nkc, (int)grid, lds, st, a);
    if (loop) return dispatch_bwd16_loop(p->dtype == ATX_DTYPE_BF16, D, nkc, (int)grid, lds, st, a);
    if (p->dtype == ATX_DTYPE_BF16) return dispatch_bwd16<__bf16>(D, nkc, (int)grid, lds, st, a);
    return dispatch_bwd16<_Float16>(D, nkc, (int)grid, lds, st, a);
}
