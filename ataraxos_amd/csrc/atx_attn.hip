// Fused attention forward for gfx950 (MI355X).
//
// Semantics follow the math fallback of the reference,
// stratego/networks/attention.py:281-316: S = (Q K^T) * scale, top-left causal
// mask (torch.triu(ones(S_q, S_kv), 1) -> -inf), softmax over keys, O = P V,
// with GQA mapping query head h to KV head h / (H / H_kv) as the
// repeat_interleave of attention.py:210-220 does.
//
// One workgroup (4 waves) owns one (batch, head) pair.  The whole key range
// (<= 256 keys) is resident at once, so the softmax is computed in a single
// pass from registers: no running-max rescaling.
//
// Work layout (16-bit types, MFMA v_mfma_f32_16x16x32_{bf16,f16}):
//   * K rows are staged in LDS, row stride 2*D+16 bytes (an odd number of
//     16-byte units, so the 16 rows an MFMA operand read touches fall in
//     distinct bank groups).
//   * V is staged TRANSPOSED in LDS (V^T[d][key]) because the PV product
//     reduces over keys and the MFMA wants the reduction index contiguous per
//     lane.  Keys are permuted inside each 32-key chunk so that the 8 keys one
//     lane needs for one PV MFMA are one 16-byte block, and blocks are
//     XOR-swizzled by the reading lane's row so the 16 lanes of a read hit 16
//     distinct bank groups.
//   * Each wave takes 16-query tiles.  Per tile it computes S^T = K Q^T
//     (keys on MFMA rows, queries on columns): lane (m = l%16, g = l/16) then
//     holds query m against keys 16*kt + 4*g + i, i.e. one query per lane, so
//     the row softmax needs only in-lane work plus two cross-lane steps.
//   * P (bf16/fp16) feeds O^T = V^T P^T as the B operand straight from
//     registers.  MFMA row r of output tile dt stands for head-dim index
//     (r/4)*(D/4) + 4*dt + r%4, which leaves every lane with D/4 contiguous
//     outputs of one query, stored with wide writes.
#include "atx_attn_kernels.hpp"

namespace atx {

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------
namespace {

template <typename T>
int dispatch_dim(int D, int nkc, int grid, hipStream_t st, const AttnArgs& a) {
    switch (D) {
        case 16: return dispatch_16bit<T, 16>(nkc, grid, st, a);
        case 32: return dispatch_16bit<T, 32>(nkc, grid, st, a);
        case 48: return dispatch_16bit<T, 48>(nkc, grid, st, a);
        case 64: return dispatch_16bit<T, 64>(nkc, grid, st, a);
        case 80: return dispatch_16bit<T, 80>(nkc, grid, st, a);
        case 96: return dispatch_16bit<T, 96>(nkc, grid, st, a);
        case 112: return dispatch_16bit<T, 112>(nkc, grid, st, a);
        case 128: return dispatch_16bit<T, 128>(nkc, grid, st, a);
    }
    ATX_FAIL(ATX_ERR_UNSUPPORTED, "head_dim %d", D);
}

int dispatch_dim_fp32(int D, int nkc, int grid, hipStream_t st, const AttnArgs& a) {
    switch (D) {
        case 16: return dispatch_fp32<16>(nkc, grid, st, a);
        case 32: return dispatch_fp32<32>(nkc, grid, st, a);
        case 48: return dispatch_fp32<48>(nkc, grid, st, a);
        case 64: return dispatch_fp32<64>(nkc, grid, st, a);
        case 80: return dispatch_fp32<80>(nkc, grid, st, a);
        case 96: return dispatch_fp32<96>(nkc, grid, st, a);
        case 112: return dispatch_fp32<112>(nkc, grid, st, a);
        case 128: return dispatch_fp32<128>(nkc, grid, st, a);
    }
    ATX_FAIL(ATX_ERR_UNSUPPORTED, "head_dim %d", D);
}

// Every row of a [B, S, H, D] view starts on a 16-byte boundary.
bool rows_aligned(const void* base, int64_t sb, int64_t ss, int64_t sh, int esize) {
    return aligned16(base) && ((sb * esize) & 15) == 0 && ((ss * esize) & 15) == 0 && ((sh * esize) & 15) == 0;
}

}  // namespace
}  // namespace atx

extern "C" int atx_attn_fwd(const AtxAttnParams* p, void* stream) {
    using namespace atx;
    clear_error();
    if (!p) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_fwd: params is NULL");
    if (p->abi_version != ATX_ABI_VERSION)
        ATX_FAIL(ATX_ERR_ABI, "atx_attn_fwd: abi_version %d, library is %d", p->abi_version, ATX_ABI_VERSION);
    if (p->dtype != ATX_DTYPE_BF16 && p->dtype != ATX_DTYPE_FP16 && p->dtype != ATX_DTYPE_FP32)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_fwd: unknown dtype %d", p->dtype);
    if (p->batch < 1 || p->seq_q < 1 || p->seq_kv < 1 || p->num_heads < 1 || p->num_kv_heads < 1 || p->head_dim < 1)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT,
                 "atx_attn_fwd: sizes must be >= 1 (batch %d, seq_q %d, seq_kv %d, heads %d, kv_heads %d, head_dim %d)",
                 p->batch, p->seq_q, p->seq_kv, p->num_heads, p->num_kv_heads, p->head_dim);
    if (p->num_heads % p->num_kv_heads != 0)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_fwd: num_heads %d not divisible by num_kv_heads %d",
                 p->num_heads, p->num_kv_heads);
    if (!p->q || !p->k || !p->v || !p->o) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_fwd: null tensor pointer");
    if (!(p->scale > 0.f) || p->scale == __builtin_inff())
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_fwd: scale must be finite and > 0 (got %g)", (double)p->scale);
    if (p->head_dim % 16 != 0 || p->head_dim > 128)
        ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_fwd: head_dim %d not supported (multiple of 16, <= 128)", p->head_dim);
    if (p->seq_kv > 256)
        ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_fwd: seq_kv %d not supported (<= 256)", p->seq_kv);
    const int64_t grid = (int64_t)p->batch * p->num_heads;
    if (grid > 0x7fffffff) ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_fwd: batch*heads %lld too large", (long long)grid);
    const int es = p->dtype == ATX_DTYPE_FP32 ? 4 : 2;
    // The 16-bit kernels address one (batch, head) slice through a buffer
    // descriptor that ends at the last valid row: rows past the sequence read
    // as zero and output rows past it are dropped. That needs 32-bit byte
    // offsets (rows up to the next multiple of 16 past the end) and output
    // rows that do not overlap. A length-1 sequence's stride is never used
    // to reach a valid row, so it is replaced by one row's extent.
    const int64_t qss = p->seq_q == 1 ? p->head_dim : p->q_stride_s;
    const int64_t oss = p->seq_q == 1 ? p->head_dim : p->o_stride_s;
    const int64_t kss = p->seq_kv == 1 ? p->head_dim : p->k_stride_s;
    const int64_t vss = p->seq_kv == 1 ? p->head_dim : p->v_stride_s;
    if (!rows_aligned(p->q, p->q_stride_b, qss, p->q_stride_h, es) ||
        !rows_aligned(p->k, p->k_stride_b, kss, p->k_stride_h, es) ||
        !rows_aligned(p->v, p->v_stride_b, vss, p->v_stride_h, es) ||
        !rows_aligned(p->o, p->o_stride_b, oss, p->o_stride_h, es))
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_fwd: every Q/K/V/O row must start on a 16-byte boundary");
    auto slice_fits = [&](int64_t stride_s, int64_t seq) {
        return stride_s >= 0 && (seq + 16) * stride_s * es + (int64_t)p->head_dim * es <= 0x7fffffffLL;
    };
    if (!slice_fits(qss, p->seq_q) || !slice_fits(oss, p->seq_q) || !slice_fits(kss, p->seq_kv) ||
        !slice_fits(vss, p->seq_kv))
        ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_fwd: sequence strides must be >= 0 and one (batch, head) slice < 2 GiB");
    if (oss < p->head_dim)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_fwd: output rows overlap (o_stride_s %lld < head_dim %d)",
                 (long long)p->o_stride_s, p->head_dim);
    if (!(p->dropout_p >= 0.f && p->dropout_p < 1.f))
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_fwd: dropout_p must be in [0, 1) (got %g)", (double)p->dropout_p);
    const bool drop = p->dropout_p > 0.f;
    if (drop && p->head_dim != 48 && p->head_dim != 64)
        ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_fwd: dropout needs head_dim 48 or 64 (got %d)", p->head_dim);

    AttnArgs a;
    a.q = p->q;
    a.k = p->k;
    a.v = p->v;
    a.o = p->o;
    a.qsb = p->q_stride_b; a.qss = qss; a.qsh = p->q_stride_h;
    a.ksb = p->k_stride_b; a.kss = kss; a.ksh = p->k_stride_h;
    a.vsb = p->v_stride_b; a.vss = vss; a.vsh = p->v_stride_h;
    a.osb = p->o_stride_b; a.oss = oss; a.osh = p->o_stride_h;
    a.kpad = p->key_pad;
    a.kpsb = p->key_pad_stride_b;
    a.kpad_w4 = p->key_pad && ((uintptr_t)p->key_pad % 4 == 0) && (p->key_pad_stride_b % 4 == 0);
    a.H = p->num_heads;
    a.group = p->num_heads / p->num_kv_heads;
    a.Sq = p->seq_q;
    a.Skv = p->seq_kv;
    a.nkt = (p->seq_kv + 15) / 16;
    a.c2 = p->scale * kLog2e;
    a.causal = p->causal != 0;
    a.xcd_remap = p->num_heads % 8 == 0;
    a.drop = make_drop_key(drop ? p->dropout_p : 0.f, p->dropout_seed, p->dropout_offset);
    const int nkc = (p->seq_kv + 31) / 32;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (drop) return dispatch_fwd_drop(p->dtype, p->head_dim, nkc, (int)grid, st, a);
    switch (p->dtype) {
        case ATX_DTYPE_BF16: return dispatch_dim<__bf16>(p->head_dim, nkc, (int)grid, st, a);
        case ATX_DTYPE_FP16: return dispatch_dim<_Float16>(p->head_dim, nkc, (int)grid, st, a);
        default: return dispatch_dim_fp32(p->head_dim, nkc, (int)grid, st, a);
    }
}
