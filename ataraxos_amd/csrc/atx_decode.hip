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
// 16-byte loads.  Keys are taken in blocks of U steps whose loads are all in
// flight together; each lane keeps a softmax (running max, running sum,
// accumulator for its chunk of V) over the keys of its lane slot, rescaled
// once per block; the slots are merged with cross-lane exchanges at the end.
// The work is pure streaming (about 1 FLOP per byte), so it is bound by HBM
// bandwidth and by how many loads are in flight.
#include <algorithm>

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
    uint32_t q_bytes, o_bytes, kc_bytes, vc_bytes, kn_bytes, vn_bytes;  // extents of this launch
};

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;

constexpr int pow2ceil(int x) {
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}

// Chunk operations: a 16-byte chunk of a row, the dot product of a q chunk
// and a k chunk (fp32 accumulate), and the conversion of a v chunk to fp32.
template <typename T>
struct Chunk;
template <>
struct Chunk<float> {
    static constexpr int N = 4;
    __device__ static inline float dot(u32x4 q, u32x4 k) {
        const f32x4 a = as_f32x4(q), b = as_f32x4(k);
        return __builtin_fmaf(a[3], b[3], __builtin_fmaf(a[2], b[2], __builtin_fmaf(a[1], b[1], a[0] * b[0])));
    }
    __device__ static inline void unpack(u32x4 v, float (&f)[4]) {
        const f32x4 x = as_f32x4(v);
#pragma unroll
        for (int i = 0; i < 4; ++i) f[i] = x[i];
    }
    __device__ static inline u32x4 pack(const float (&f)[4]) {
        return __builtin_bit_cast(u32x4, f32x4{f[0], f[1], f[2], f[3]});
    }
};
template <typename T16>
struct Chunk16 {
    static constexpr int N = 8;
    typedef T16 v8 __attribute__((ext_vector_type(8)));
    typedef T16 v2 __attribute__((ext_vector_type(2)));
    // Products of two 16-bit floats are exact in fp32; v_dot2 adds two of
    // them to an fp32 accumulator.  (Sub-vectors are taken with shuffles of
    // the whole vector, never by casting single elements.)
    __device__ static inline float dot(u32x4 q, u32x4 k) {
        const v8 a = __builtin_bit_cast(v8, q), b = __builtin_bit_cast(v8, k);
        float r = 0.f;
        r = dot2(__builtin_shufflevector(a, a, 0, 1), __builtin_shufflevector(b, b, 0, 1), r);
        r = dot2(__builtin_shufflevector(a, a, 2, 3), __builtin_shufflevector(b, b, 2, 3), r);
        r = dot2(__builtin_shufflevector(a, a, 4, 5), __builtin_shufflevector(b, b, 4, 5), r);
        r = dot2(__builtin_shufflevector(a, a, 6, 7), __builtin_shufflevector(b, b, 6, 7), r);
        return r;
    }
    __device__ static inline float dot2(v2 x, v2 y, float c);
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
__device__ inline float Chunk16<__bf16>::dot2(v2 x, v2 y, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(x, y, c, false);
}
template <>
__device__ inline float Chunk16<_Float16>::dot2(v2 x, v2 y, float c) {
    return __builtin_amdgcn_fdot2(x, y, c, false);
}
template <>
struct Chunk<__bf16> : Chunk16<__bf16> {};
template <>
struct Chunk<_Float16> : Chunk16<_Float16> {};

}  // namespace

// Waves needed for P (batch, head) pairs at head_dim D.
template <typename T>
constexpr int dec_slots_per_wave(int D) {
    return 64 / pow2ceil(D / Chunk<T>::N);
}

#ifndef ATX_DEC_KEYS
#define ATX_DEC_KEYS 2
#endif
#ifndef ATX_DEC_WAVES
#define ATX_DEC_WAVES 8
#endif

template <typename T, int D>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(ATX_DEC_WAVES, 8)))
void attn_decode(DecArgs a) {
    using C = Chunk<T>;
    constexpr int EPC = C::N;             // elements per 16-byte chunk
    constexpr int CH = D / EPC;           // chunks per row
    constexpr int LPK = pow2ceil(CH);     // lanes per slot (one row per step)
    constexpr int SPW = 64 / LPK;         // slots = (batch, head) pairs per wave
    constexpr int U = ATX_DEC_KEYS;       // keys per block: all their loads in flight together

    const int lane = threadIdx.x & 63;
    const int slot = lane / LPK, dc = lane % LPK;
    const int pair = (blockIdx.x * kWaves + (threadIdx.x >> 6)) * SPW + slot;
    const bool valid = pair < a.B * a.H;
    const bool active = valid && dc < CH;
    const int pr = valid ? pair : 0;
    const int b = pr / a.H, h = pr - (pr / a.H) * a.H;
    const int hk = h / a.group;

    int n = valid ? (a.lens ? a.lens[b] : a.len) : 0;
    n = n < a.cap ? n : a.cap;
    int nmax = n;  // the wave's trip count
#pragma unroll
    for (int off = LPK; off < 64; off <<= 1) nmax = max(nmax, __builtin_bit_cast(int, shfl_xor(__builtin_bit_cast(float, nmax), off)));
    nmax = __builtin_amdgcn_readfirstlane(nmax);

    // One buffer descriptor per tensor (uniform), 32-bit per-lane byte
    // offsets (the host keeps every extent of one launch below 4 GiB).  A
    // masked-out access gets an offset past the extent: loads return zero and
    // stores are dropped by the range check, with no branches.
    constexpr uint32_t es = sizeof(T);
    constexpr uint32_t kOut = 0xfffffff0u;
    const rsrc_t rk = make_rsrc(a.kc, a.kc_bytes), rv = make_rsrc(a.vc, a.vc_bytes);
    const uint32_t chunk = (uint32_t)dc * 16;
    const uint32_t koff = (uint32_t)(b * a.ksb + hk * a.ksh) * es + chunk;
    const uint32_t voff = (uint32_t)(b * a.vsb + hk * a.vsh) * es + chunk;
    const uint32_t kstep = (uint32_t)a.kss * es, vstep = (uint32_t)a.vss * es;
    const bool has_new = a.kn != nullptr;
    const u32x4 qv = buf_ld16(make_rsrc(a.q, a.q_bytes), active ? (uint32_t)(b * a.qsb + h * a.qsh) * es + chunk : kOut);
    // the newest row, when given, comes from k_new / v_new
    u32x4 knv = u32x4{0, 0, 0, 0}, vnv = u32x4{0, 0, 0, 0};
    if (has_new) {
        knv = buf_ld16(make_rsrc(a.kn, a.kn_bytes), active ? (uint32_t)(b * a.knb + hk * a.knh) * es + chunk : kOut);
        vnv = buf_ld16(make_rsrc(a.vn, a.vn_bytes), active ? (uint32_t)(b * a.vnb + hk * a.vnh) * es + chunk : kOut);
    }

    const float kNegInf = -__builtin_inff();
    float mrun = kNegInf, lrun = 0.f;
    float acc[EPC];
#pragma unroll
    for (int e = 0; e < EPC; ++e) acc[e] = 0.f;

    for (int base = 0; base < nmax; base += U) {
        u32x4 kv[U], vv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int key = base + u;
            const bool fresh = has_new && key == n - 1;
            const bool ok = active && key < n && !fresh;
            kv[u] = buf_ld16(rk, ok ? koff + (uint32_t)key * kstep : kOut);
            vv[u] = buf_ld16(rv, ok ? voff + (uint32_t)key * vstep : kOut);
            if (fresh) {
                kv[u] = knv;
                vv[u] = vnv;
            }
        }
        // scores of the block in log2 units (keys past n: -inf), one rescale
        float sc[U];
        float mblk = kNegInf;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float d = C::dot(qv, kv[u]);
#pragma unroll
            for (int off = 1; off < LPK; off <<= 1) d += shfl_xor(d, off);
            sc[u] = base + u < n ? d * a.c2 : kNegInf;
            mblk = fmaxf(mblk, sc[u]);
        }
        const float mnew = fmaxf(mrun, mblk);
        const float ms = mnew == kNegInf ? 0.f : mnew;  // no key yet: stays empty
        const float alpha = fast_exp2(mrun - ms);
        lrun *= alpha;
#pragma unroll
        for (int e = 0; e < EPC; ++e) acc[e] *= alpha;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const float p = fast_exp2(sc[u] - ms);
            float vf[EPC];
            C::unpack(vv[u], vf);
            lrun += p;
#pragma unroll
            for (int e = 0; e < EPC; ++e) acc[e] = __builtin_fmaf(p, vf[e], acc[e]);
        }
        mrun = mnew;
    }

    if (active) {
        // n < 1 leaves lrun = 0 and the result NaN, as a softmax over no keys.
        const float inv = 1.0f / lrun;
        float r[EPC];
#pragma unroll
        for (int e = 0; e < EPC; ++e) r[e] = acc[e] * inv;
        buf_st16(make_rsrc(a.o, a.o_bytes), (uint32_t)(b * a.osb + h * a.osh) * es + chunk, C::pack(r));
        // The first query head of each KV group appends the new row.
        if (has_new && n >= 1 && h % a.group == 0) {
            buf_st16(rk, koff + (uint32_t)(n - 1) * kstep, knv);
            buf_st16(rv, voff + (uint32_t)(n - 1) * vstep, vnv);
        }
    }
}

namespace {

template <typename T, int D>
int launch_decode(hipStream_t st, const DecArgs& a) {
    constexpr int spw = dec_slots_per_wave<T>(D);
    const int64_t waves = ((int64_t)a.B * a.H + spw - 1) / spw;
    const int64_t grid = (waves + kWaves - 1) / kWaves;
    if (grid > 0x7fffffff) ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_decode_fwd: batch*heads too large");
    hipLaunchKernelGGL((attn_decode<T, D>), dim3((unsigned)grid), dim3(kThreads), 0, st, a);
    ATX_CHECK_LAUNCH("atx_attn_decode_fwd launch");
    return ATX_OK;
}

template <typename T>
int dispatch_decode(int D, hipStream_t st, const DecArgs& a) {
    switch (D) {
        case 8: return launch_decode<T, 8>(st, a);
        case 16: return launch_decode<T, 16>(st, a);
        case 24: return launch_decode<T, 24>(st, a);
        case 32: return launch_decode<T, 32>(st, a);
        case 48: return launch_decode<T, 48>(st, a);
        case 64: return launch_decode<T, 64>(st, a);
        case 96: return launch_decode<T, 96>(st, a);
        case 128: return launch_decode<T, 128>(st, a);
        case 256: return launch_decode<T, 256>(st, a);
        default: ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_decode_fwd: head_dim %d not supported", D);
    }
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
    // The kernel addresses each tensor with 32-bit byte offsets: launch over
    // batch chunks whose every tensor extent stays below 4 GiB.
    const int64_t D = p->head_dim, Hq = p->num_heads, Hk = p->num_kv_heads, T = p->kv_capacity;
    struct Extent {
        int64_t sb, rest;  // bytes per batch step; bytes of one batch element's slice
    };
    const Extent ext[] = {
        {p->q_stride_b * es, ((Hq - 1) * p->q_stride_h + D) * es},
        {p->o_stride_b * es, ((Hq - 1) * p->o_stride_h + D) * es},
        {p->k_stride_b * es, ((Hk - 1) * p->k_stride_h + (T - 1) * p->k_stride_s + D) * es},
        {p->v_stride_b * es, ((Hk - 1) * p->v_stride_h + (T - 1) * p->v_stride_s + D) * es},
        {p->k_new ? p->k_new_stride_b * es : 0, p->k_new ? ((Hk - 1) * p->k_new_stride_h + D) * es : 0},
        {p->v_new ? p->v_new_stride_b * es : 0, p->v_new ? ((Hk - 1) * p->v_new_stride_h + D) * es : 0},
    };
    const int64_t lim = 0xffffff00LL;  // below the out-of-range offset the kernel uses for masked lanes
    int64_t nb = p->batch;
    for (const Extent& e : ext) {
        if (e.sb < 0 || e.rest < 0 || e.rest > lim)
            ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_decode_fwd: strides must be >= 0 and one batch element < 4 GiB");
        if (e.sb > 0) nb = std::min<int64_t>(nb, 1 + (lim - e.rest) / e.sb);
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    for (int64_t b0 = 0; b0 < p->batch; b0 += nb) {
        DecArgs c = a;
        c.B = (int)std::min<int64_t>(nb, p->batch - b0);
        c.q = static_cast<const char*>(p->q) + b0 * ext[0].sb;
        c.o = static_cast<char*>(p->o) + b0 * ext[1].sb;
        c.kc = static_cast<char*>(p->k_cache) + b0 * ext[2].sb;
        c.vc = static_cast<char*>(p->v_cache) + b0 * ext[3].sb;
        if (p->k_new) {
            c.kn = static_cast<const char*>(p->k_new) + b0 * ext[4].sb;
            c.vn = static_cast<const char*>(p->v_new) + b0 * ext[5].sb;
        }
        if (p->kv_lens) c.lens = p->kv_lens + b0;
        auto bytes = [&](const Extent& e) { return (uint32_t)((c.B - 1) * e.sb + e.rest); };
        c.q_bytes = bytes(ext[0]);
        c.o_bytes = bytes(ext[1]);
        c.kc_bytes = bytes(ext[2]);
        c.vc_bytes = bytes(ext[3]);
        c.kn_bytes = p->k_new ? bytes(ext[4]) : 0;
        c.vn_bytes = p->v_new ? bytes(ext[5]) : 0;
        int rc;
        switch (p->dtype) {
            case ATX_DTYPE_BF16: rc = dispatch_decode<__bf16>(p->head_dim, st, c); break;
            case ATX_DTYPE_FP16: rc = dispatch_decode<_Float16>(p->head_dim, st, c); break;
            default: rc = dispatch_decode<float>(p->head_dim, st, c); break;
        }
        if (rc != ATX_OK) return rc;
    }
    return ATX_OK;
}
