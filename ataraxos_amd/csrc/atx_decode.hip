// Single-query attention over a KV cache (incremental causal decode) for
// gfx950.  The reference has no cache: SetupNetwork recomputes the causal
// attention over the whole prefix for every new token
// (stratego/training/selfplay.py:139-146,181, stratego/networks/setup_net.py:117,
// stratego/networks/attention.py:281-316 with is_causal = True).  The last
// row of that recompute is softmax(q_t . K[0:t]^T * scale) . V[0:t], which is
// what this kernel returns.
//
// One wave per (batch, head).  A key row is split over LPK lanes (one 16-byte
// chunk each), so a wave covers 64/LPK keys per step with fully coalesced
// 16-byte loads.  Each lane keeps an online softmax (running max, running sum,
// accumulator for its chunk of V) over the keys of its lane slot; the slots
// are merged with cross-lane exchanges at the end.  The work is pure
// streaming (about 1 FLOP per byte), so it is bound by HBM bandwidth.
#include "atx_common.hpp"

namespace atx {

struct DecArgs {
    const void* q;
    void* kc;
    void* vc;
    const void* kn;
    const void* vn;
    void* o;
    int64_t qsb, qsh;
    int64_t ksb, ksh, kss;
    int64_t vsb, vsh, vss;
    int64_t knb, knh, vnb, vnh;
    int64_t osb, osh;
    const int32_t* lens;
    int B, H, group, len, cap;
    float c2;
};

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;

constexpr int pow2ceil(int x) {
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}

template <typename T>
struct Elem;
template <>
struct Elem<float> {
    static constexpr int N = 4;
    __device__ static inline void unpack(u32x4 v, float (&f)[4]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) f[i] = as_f32x4(v)[i];
    }
    __device__ static inline u32x4 pack(const float (&f)[4]) {
        return u32x4{__builtin_bit_cast(uint32_t, f[0]), __builtin_bit_cast(uint32_t, f[1]),
                     __builtin_bit_cast(uint32_t, f[2]), __builtin_bit_cast(uint32_t, f[3])};
    }
};
template <typename T16>
struct Elem16 {
    static constexpr int N = 8;
    __device__ static inline void unpack(u32x4 v, float (&f)[8]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[2 * i] = Mfma16<T16>::to_float(static_cast<uint16_t>(v[i] & 0xffffu));
            f[2 * i + 1] = Mfma16<T16>::to_float(static_cast<uint16_t>(v[i] >> 16));
        }
    }
    __device__ static inline u32x4 pack(const float (&f)[8]) {
        return u32x4{Mfma16<T16>::pack2(f[0], f[1]), Mfma16<T16>::pack2(f[2], f[3]),
                     Mfma16<T16>::pack2(f[4], f[5]), Mfma16<T16>::pack2(f[6], f[7])};
    }
};
template <>
struct Elem<__bf16> : Elem16<__bf16> {};
template <>
struct Elem<_Float16> : Elem16<_Float16> {};

}  // namespace

template <typename T, int D>
__global__ __launch_bounds__(kThreads) void attn_decode(DecArgs a) {
    using E = Elem<T>;
    constexpr int EPC = E::N;             // elements per 16-byte chunk
    constexpr int CH = D / EPC;           // chunks per row
    constexpr int LPK = pow2ceil(CH);     // lanes per key
    constexpr int KPI = 64 / LPK;         // keys per wave step
    constexpr int U = KPI >= 8 ? 2 : 4;   // steps whose loads are issued together

    const int lane = threadIdx.x & 63;
    const int wid = blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (wid >= a.B * a.H) return;
    const int b = wid / a.H, h = wid - (wid / a.H) * a.H;
    const int hk = h / a.group;
    const int slot = lane / LPK, dc = lane % LPK;
    const bool active = dc < CH;

    int n = a.lens ? a.lens[b] : a.len;
    n = n < a.cap ? n : a.cap;

    const T* kb = static_cast<const T*>(a.kc) + b * a.ksb + hk * a.ksh;
    const T* vb = static_cast<const T*>(a.vc) + b * a.vsb + hk * a.vsh;
    const T* knew = a.kn ? static_cast<const T*>(a.kn) + b * a.knb + hk * a.knh : nullptr;
    const T* vnew = a.vn ? static_cast<const T*>(a.vn) + b * a.vnb + hk * a.vnh : nullptr;

    float qf[EPC];
    {
        const T* qrow = static_cast<const T*>(a.q) + b * a.qsb + h * a.qsh;
        u32x4 qv = active ? ld16(qrow + dc * EPC) : u32x4{0, 0, 0, 0};
        E::unpack(qv, qf);
#pragma unroll
        for (int e = 0; e < EPC; ++e) qf[e] *= a.c2;  // scores come out in log2 units
    }

    const float kNegInf = -__builtin_inff();
    float mrun = kNegInf, lrun = 0.f;
    float acc[EPC];
#pragma unroll
    for (int e = 0; e < EPC; ++e) acc[e] = 0.f;

    for (int base = 0; base < n; base += U * KPI) {
        u32x4 kv[U], vv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int key = base + u * KPI + slot;
            const bool ok = active && key < n;
            const bool fresh = knew && key == n - 1;
            const T* kp = fresh ? knew : kb + key * a.kss;
            const T* vp = fresh ? vnew : vb + key * a.vss;
            kv[u] = ok ? ld16(kp + dc * EPC) : u32x4{0, 0, 0, 0};
            vv[u] = ok ? ld16(vp + dc * EPC) : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int key = base + u * KPI + slot;
            float kf[EPC];
            E::unpack(kv[u], kf);
            float dot = 0.f;
#pragma unroll
            for (int e = 0; e < EPC; ++e) dot = __builtin_fmaf(qf[e], kf[e], dot);
#pragma unroll
            for (int off = 1; off < LPK; off <<= 1) dot += shfl_xor(dot, off);
            if (key < n) {
                const float mnew = fmaxf(mrun, dot);
                const float alpha = fast_exp2(mrun - mnew);  // 0 while mrun = -inf
                const float p = fast_exp2(dot - mnew);
                float vf[EPC];
                E::unpack(vv[u], vf);
                lrun = lrun * alpha + p;
#pragma unroll
                for (int e = 0; e < EPC; ++e) acc[e] = __builtin_fmaf(p, vf[e], acc[e] * alpha);
                mrun = mnew;
            }
        }
    }

    // Merge the KPI key slots.
#pragma unroll
    for (int off = LPK; off < 64; off <<= 1) {
        const float mo = shfl_xor(mrun, off);
        const float lo = shfl_xor(lrun, off);
        const float mnew = fmaxf(mrun, mo);
        const bool empty = (mnew == kNegInf);
        const float a1 = empty ? 0.f : fast_exp2(mrun - mnew);
        const float a2 = empty ? 0.f : fast_exp2(mo - mnew);
        lrun = lrun * a1 + lo * a2;
#pragma unroll
        for (int e = 0; e < EPC; ++e) {
            const float ao = shfl_xor(acc[e], off);
            acc[e] = acc[e] * a1 + ao * a2;
        }
        mrun = mnew;
    }

    if (slot == 0 && active) {
        // n < 1 leaves lrun = 0 and the result NaN, as a softmax over no keys.
        const float inv = 1.0f / lrun;
        float r[EPC];
#pragma unroll
        for (int e = 0; e < EPC; ++e) r[e] = acc[e] * inv;
        T* orow = static_cast<T*>(a.o) + b * a.osb + h * a.osh;
        st16(orow + dc * EPC, E::pack(r));
        // The first query head of each KV group appends the new row.
        if (knew && n >= 1 && h % a.group == 0) {
            st16(static_cast<T*>(a.kc) + b * a.ksb + hk * a.ksh + (n - 1) * a.kss + dc * EPC, ld16(knew + dc * EPC));
            st16(static_cast<T*>(a.vc) + b * a.vsb + hk * a.vsh + (n - 1) * a.vss + dc * EPC, ld16(vnew + dc * EPC));
        }
    }
}

namespace {

template <typename T>
int dispatch_decode(int D, int grid, hipStream_t st, const DecArgs& a) {
    switch (D) {
#define ATX_DEC_CASE(N)                                                                  \
    case N:                                                                              \
        hipLaunchKernelGGL((attn_decode<T, N>), dim3(grid), dim3(kThreads), 0, st, a); \
        break;
        ATX_DEC_CASE(8)
        ATX_DEC_CASE(16)
        ATX_DEC_CASE(24)
        ATX_DEC_CASE(32)
        ATX_DEC_CASE(48)
        ATX_DEC_CASE(64)
        ATX_DEC_CASE(96)
        ATX_DEC_CASE(128)
        ATX_DEC_CASE(256)
#undef ATX_DEC_CASE
        default:
            ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_decode_fwd: head_dim %d not supported", D);
    }
    ATX_CHECK_LAUNCH("atx_attn_decode_fwd launch");
    return ATX_OK;
}

}  // namespace
}  // namespace atx

extern "C" int atx_attn_decode_fwd(const AtxDecodeParams* p, void* stream) {
    using namespace atx;
    clear_error();
    if (!p) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_decode_fwd: params is NULL");
    if (p->abi_version != ATX_ABI_VERSION)
        ATX_FAIL(ATX_ERR_ABI, "atx_attn_decode_fwd: abi_version %d, library is %d", p->abi_version, ATX_ABI_VERSION);
    if (p->dtype != ATX_DTYPE_BF16 && p->dtype != ATX_DTYPE_FP16 && p->dtype != ATX_DTYPE_FP32)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_decode_fwd: unknown dtype %d", p->dtype);
    if (p->batch < 1 || p->num_heads < 1 || p->num_kv_heads < 1 || p->head_dim < 1 || p->kv_capacity < 1)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_decode_fwd: sizes must be >= 1");
    if (p->num_heads % p->num_kv_heads != 0)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_decode_fwd: num_heads %d not divisible by num_kv_heads %d",
                 p->num_heads, p->num_kv_heads);
    if (!p->kv_lens && (p->kv_len < 1 || p->kv_len > p->kv_capacity))
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_decode_fwd: kv_len %d outside [1, kv_capacity %d]", p->kv_len,
                 p->kv_capacity);
    if (!p->q || !p->k_cache || !p->v_cache || !p->o)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_decode_fwd: null tensor pointer");
    if ((p->k_new == nullptr) != (p->v_new == nullptr))
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_decode_fwd: k_new and v_new must be given together");
    if (!(p->scale > 0.f) || p->scale == __builtin_inff())
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_decode_fwd: scale must be finite and > 0 (got %g)",
                 (double)p->scale);
    const int es = p->dtype == ATX_DTYPE_FP32 ? 4 : 2;
    const int epc = 16 / es;
    if (p->head_dim % epc != 0)
        ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_decode_fwd: head_dim %d must be a multiple of %d", p->head_dim, epc);
    auto al = [&](const void* ptr, int64_t s1, int64_t s2, int64_t s3) {
        return aligned16(ptr) && ((s1 * es) & 15) == 0 && ((s2 * es) & 15) == 0 && ((s3 * es) & 15) == 0;
    };
    if (!al(p->q, p->q_stride_b, p->q_stride_h, 0) || !al(p->k_cache, p->k_stride_b, p->k_stride_h, p->k_stride_s) ||
        !al(p->v_cache, p->v_stride_b, p->v_stride_h, p->v_stride_s) || !al(p->o, p->o_stride_b, p->o_stride_h, 0) ||
        (p->k_new && (!al(p->k_new, p->k_new_stride_b, p->k_new_stride_h, 0) ||
                      !al(p->v_new, p->v_new_stride_b, p->v_new_stride_h, 0))))
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_decode_fwd: every row must start on a 16-byte boundary");
    const int64_t waves = (int64_t)p->batch * p->num_heads;
    if (waves > 0x7fffffffLL - kWaves)
        ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_decode_fwd: batch*heads %lld too large", (long long)waves);

    DecArgs a;
    a.q = p->q;
    a.kc = p->k_cache;
    a.vc = p->v_cache;
    a.kn = p->k_new;
    a.vn = p->v_new;
    a.o = p->o;
    a.qsb = p->q_stride_b; a.qsh = p->q_stride_h;
    a.ksb = p->k_stride_b; a.ksh = p->k_stride_h; a.kss = p->k_stride_s;
    a.vsb = p->v_stride_b; a.vsh = p->v_stride_h; a.vss = p->v_stride_s;
    a.knb = p->k_new_stride_b; a.knh = p->k_new_stride_h;
    a.vnb = p->v_new_stride_b; a.vnh = p->v_new_stride_h;
    a.osb = p->o_stride_b; a.osh = p->o_stride_h;
    a.lens = p->kv_lens;
    a.B = p->batch;
    a.H = p->num_heads;
    a.group = p->num_heads / p->num_kv_heads;
    a.len = p->kv_len;
    a.cap = p->kv_capacity;
    a.c2 = p->scale * kLog2e;
    const int grid = (int)((waves + kWaves - 1) / kWaves);
    hipStream_t st = static_cast<hipStream_t>(stream);
    switch (p->dtype) {
        case ATX_DTYPE_BF16: return dispatch_decode<__bf16>(p->head_dim, grid, st, a);
        case ATX_DTYPE_FP16: return dispatch_decode<_Float16>(p->head_dim, grid, st, a);
        default: return dispatch_decode<float>(p->head_dim, grid, st, a);
    }
}
