// Key-query policy head for gfx950: logits + legal-move mask (+ softmax over
// the whole from x to board), one workgroup per sample.
//
// Semantics: stratego/networks/move_net.py:92-95 computes
//   logits = (q @ k^T) / sqrt(d); logits.masked_fill(~mask, -1e10);
//   logits.reshape(B, S*S)          (from-major: index i*S + j)
// and every caller then takes softmax(dim=-1) over the S*S entries
// (stratego/training/selfplay.py:284, stratego/training/move_trainer.py:118).
//
// Layout: the S x S logits of one sample are computed as 16x16 MFMA tiles of
// L^T = K Q^T, so lane (m, g) of a tile holds from-square 16*it + m against
// the four consecutive to-squares 16*jt + 4g .. +3: one 16-byte fp32 store and
// one 4-byte mask load per tile and lane.  The whole sample (<= 128 x 128
// logits) stays in registers across the two block reductions (max, sum), so
// the logits are never written to memory.
#include "atx_common.hpp"

namespace atx {

struct KqArgs {
    const void* q;
    const void* k;
    int64_t qsb, qss, ksb, kss;
    const uint8_t* mask;
    int64_t msb, mss;
    float* out;
    int64_t osb;
    int S, nchunks;  // nchunks: 16-byte chunks per q/k row
    float scale, c2;
    int probs;
    int mask_vec;  // 4-byte mask loads are aligned
    int out_vec;   // 16-byte output stores are aligned
};

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kSliceChunks = 8;            // 16-byte chunks per staged slice
constexpr int kRowBytes = kSliceChunks * 16 + 16;  // padded LDS row (odd number of 16B units)

template <typename T>
struct KqMma;

template <>
struct KqMma<__bf16> {
    __device__ static inline f32x4 slice(const char* krow, const char* qrow, int g, f32x4 acc) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const u32x4 a = *reinterpret_cast<const u32x4*>(krow + (4 * i + g) * 16);
            const u32x4 b = *reinterpret_cast<const u32x4*>(qrow + (4 * i + g) * 16);
            acc = Mfma16<__bf16>::mma(a, b, acc);
        }
        return acc;
    }
};

template <>
struct KqMma<_Float16> {
    __device__ static inline f32x4 slice(const char* krow, const char* qrow, int g, f32x4 acc) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const u32x4 a = *reinterpret_cast<const u32x4*>(krow + (4 * i + g) * 16);
            const u32x4 b = *reinterpret_cast<const u32x4*>(qrow + (4 * i + g) * 16);
            acc = Mfma16<_Float16>::mma(a, b, acc);
        }
        return acc;
    }
};

template <>
struct KqMma<float> {
    __device__ static inline f32x4 slice(const char* krow, const char* qrow, int g, f32x4 acc) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const f32x4 a = as_f32x4(*reinterpret_cast<const u32x4*>(krow + (4 * i + g) * 16));
            const f32x4 b = as_f32x4(*reinterpret_cast<const u32x4*>(qrow + (4 * i + g) * 16));
#pragma unroll
            for (int j = 0; j < 4; ++j) acc = mma_f32(a[j], b[j], acc);
        }
        return acc;
    }
};

__device__ inline float wave_max(float v) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) v = fmaxf(v, shfl_xor(v, off));
    return v;
}
__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) v += shfl_xor(v, off);
    return v;
}

}  // namespace

// NT = number of 16-square tiles per side (S <= 16*NT).
template <typename T, int NT>
__global__ __launch_bounds__(kThreads) void kq_policy(KqArgs a) {
    constexpr int NTILE = NT * NT;
    constexpr int TPW = (NTILE + kWaves - 1) / kWaves;
    constexpr int ROWS = NT * 16;

    __shared__ __attribute__((aligned(16))) char sq[ROWS * kRowBytes];
    __shared__ __attribute__((aligned(16))) char sk[ROWS * kRowBytes];
    __shared__ float red[kWaves];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int m = lane & 15, g = lane >> 4;
    const int b = blockIdx.x;
    const int S = a.S;

    const char* qb = static_cast<const char*>(a.q) + (int64_t)b * a.qsb * sizeof(T);
    const char* kb = static_cast<const char*>(a.k) + (int64_t)b * a.ksb * sizeof(T);
    const int64_t qrs = a.qss * (int64_t)sizeof(T), krs = a.kss * (int64_t)sizeof(T);

    // ---- legality bytes, fetched before the products -------------------
    uint32_t mbits[TPW];
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
        const int t = wave + kWaves * u;
        const int it = t / NT, jt = t - (t / NT) * NT;
        const int i = it * 16 + m, j0 = jt * 16 + 4 * g;
        uint32_t w = 0;
        if (t < NTILE && i < S && j0 < S) {
            if (!a.mask) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (j0 + e < S) w |= 1u << (8 * e);
            } else {
                const uint8_t* mrow = a.mask + (int64_t)b * a.msb + (int64_t)i * a.mss;
                if (a.mask_vec) {
                    w = *reinterpret_cast<const uint32_t*>(mrow + j0);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (j0 + e < S) w |= (uint32_t)(mrow[j0 + e] != 0) << (8 * e);
                }
            }
        }
        mbits[u] = w;
    }

    // ---- logits: loop over 8-chunk slices of the feature dimension --------
    f32x4 acc[TPW];
#pragma unroll
    for (int u = 0; u < TPW; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int sc = 0; sc < a.nchunks; sc += kSliceChunks) {
        if (sc) __syncthreads();
        for (int idx = tid; idx < S * kSliceChunks; idx += kThreads) {
            const int r = idx >> 3, c = idx & 7;
            const bool in = sc + c < a.nchunks;
            const u32x4 qv = in ? ld16(qb + r * qrs + (sc + c) * 16) : u32x4{0, 0, 0, 0};
            const u32x4 kv = in ? ld16(kb + r * krs + (sc + c) * 16) : u32x4{0, 0, 0, 0};
            *reinterpret_cast<u32x4*>(sq + r * kRowBytes + c * 16) = qv;
            *reinterpret_cast<u32x4*>(sk + r * kRowBytes + c * 16) = kv;
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < TPW; ++u) {
            const int t = wave + kWaves * u;
            if (t < NTILE) {
                const int it = t / NT, jt = t - (t / NT) * NT;
                acc[u] = KqMma<T>::slice(sk + (jt * 16 + m) * kRowBytes, sq + (it * 16 + m) * kRowBytes, g, acc[u]);
            }
        }
    }

    float* ob = a.out + (int64_t)b * a.osb;
    const float kNegInf = -__builtin_inff();

    if (!a.probs) {
#pragma unroll
        for (int u = 0; u < TPW; ++u) {
            const int t = wave + kWaves * u;
            const int it = t / NT, jt = t - (t / NT) * NT;
            const int i = it * 16 + m, j0 = jt * 16 + 4 * g;
            if (t < NTILE && i < S && j0 < S) {
                float r[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) r[e] = ((mbits[u] >> (8 * e)) & 0xff) ? acc[u][e] * a.scale : -1e10f;
                float* dst = ob + (int64_t)i * S + j0;
                if (a.out_vec) {
                    st16(dst, __builtin_bit_cast(u32x4, f32x4{r[0], r[1], r[2], r[3]}));
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (j0 + e < S) dst[e] = r[e];
                }
            }
        }
        return;
    }

    // ---- softmax over the S*S legal entries ------------------------------
    float mx = kNegInf;
#pragma unroll
    for (int u = 0; u < TPW; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if ((mbits[u] >> (8 * e)) & 0xff) mx = fmaxf(mx, acc[u][e]);
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();

    const bool none_legal = (mx == kNegInf);
    const float mb = mx * a.c2;
    float lsum = 0.f;
#pragma unroll
    for (int u = 0; u < TPW; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const bool legal = (mbits[u] >> (8 * e)) & 0xff;
            const float p = legal ? fast_exp2(__builtin_fmaf(acc[u][e], a.c2, -mb)) : 0.f;
            acc[u][e] = p;
            lsum += p;
        }
    lsum = wave_sum(lsum);
    if (lane == 0) red[wave] = lsum;
    __syncthreads();
    lsum = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = 1.0f / lsum;
    const float uniform = 1.0f / (float)(S * S);

#pragma unroll
    for (int u = 0; u < TPW; ++u) {
        const int t = wave + kWaves * u;
        const int it = t / NT, jt = t - (t / NT) * NT;
        const int i = it * 16 + m, j0 = jt * 16 + 4 * g;
        if (t < NTILE && i < S && j0 < S) {
            float r[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) r[e] = none_legal ? uniform : acc[u][e] * inv;
            float* dst = ob + (int64_t)i * S + j0;
            if (a.out_vec) {
                st16(dst, __builtin_bit_cast(u32x4, f32x4{r[0], r[1], r[2], r[3]}));
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (j0 + e < S) dst[e] = r[e];
            }
        }
    }
}

namespace {

template <typename T>
int dispatch_kq(int nt, int grid, hipStream_t st, const KqArgs& a) {
    switch (nt) {
#define ATX_KQ_CASE(N)                                                             \
    case N:                                                                        \
        hipLaunchKernelGGL((kq_policy<T, N>), dim3(grid), dim3(kThreads), 0, st, a); \
        break;
        ATX_KQ_CASE(1)
        ATX_KQ_CASE(2)
        ATX_KQ_CASE(3)
        ATX_KQ_CASE(4)
        ATX_KQ_CASE(5)
        ATX_KQ_CASE(6)
        ATX_KQ_CASE(7)
        ATX_KQ_CASE(8)
#undef ATX_KQ_CASE
        default:
            ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_kq_masked_softmax_fwd: %d tiles", nt);
    }
    ATX_CHECK_LAUNCH("atx_kq_masked_softmax_fwd launch");
    return ATX_OK;
}

}  // namespace
}  // namespace atx

extern "C" int atx_kq_masked_softmax_fwd(const AtxKqParams* p, void* stream) {
    using namespace atx;
    clear_error();
    if (!p) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_kq_masked_softmax_fwd: params is NULL");
    if (p->abi_version != ATX_ABI_VERSION)
        ATX_FAIL(ATX_ERR_ABI, "atx_kq_masked_softmax_fwd: abi_version %d, library is %d", p->abi_version,
                 ATX_ABI_VERSION);
    if (p->dtype != ATX_DTYPE_BF16 && p->dtype != ATX_DTYPE_FP16 && p->dtype != ATX_DTYPE_FP32)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_kq_masked_softmax_fwd: unknown dtype %d", p->dtype);
    if (p->batch < 1 || p->seq < 1 || p->dim < 1)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_kq_masked_softmax_fwd: sizes must be >= 1 (batch %d, seq %d, dim %d)",
                 p->batch, p->seq, p->dim);
    if (p->out_mode != ATX_KQ_OUT_PROBS && p->out_mode != ATX_KQ_OUT_LOGITS)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_kq_masked_softmax_fwd: unknown out_mode %d", p->out_mode);
    if (!p->q || !p->k || !p->out) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_kq_masked_softmax_fwd: null tensor pointer");
    if (!(p->scale > 0.f) || p->scale == __builtin_inff())
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_kq_masked_softmax_fwd: scale must be finite and > 0 (got %g)",
                 (double)p->scale);
    if (p->seq > 128) ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_kq_masked_softmax_fwd: seq %d not supported (<= 128)", p->seq);
    if (p->dim % 8 != 0)
        ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_kq_masked_softmax_fwd: dim %d not supported (multiple of 8)", p->dim);
    const int es = p->dtype == ATX_DTYPE_FP32 ? 4 : 2;
    if (!aligned16(p->q) || !aligned16(p->k) || ((p->q_stride_b * es) & 15) || ((p->q_stride_s * es) & 15) ||
        ((p->k_stride_b * es) & 15) || ((p->k_stride_s * es) & 15))
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_kq_masked_softmax_fwd: every q/k row must start on a 16-byte boundary");
    if (((uintptr_t)p->out & 3) != 0 || p->out_stride_b < (int64_t)p->seq * p->seq)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_kq_masked_softmax_fwd: out must be 4-byte aligned with stride >= seq*seq");

    KqArgs a;
    a.q = p->q;
    a.k = p->k;
    a.qsb = p->q_stride_b; a.qss = p->q_stride_s;
    a.ksb = p->k_stride_b; a.kss = p->k_stride_s;
    a.mask = p->mask;
    a.msb = p->mask_stride_b; a.mss = p->mask_stride_s;
    a.out = p->out;
    a.osb = p->out_stride_b;
    a.S = p->seq;
    a.nchunks = p->dim * es / 16;
    a.scale = p->scale;
    a.c2 = p->scale * kLog2e;
    a.probs = p->out_mode == ATX_KQ_OUT_PROBS;
    a.mask_vec = p->mask && (((uintptr_t)p->mask & 3) == 0) && (p->mask_stride_b % 4 == 0) &&
                 (p->mask_stride_s % 4 == 0) && (p->seq % 4 == 0);
    a.out_vec = aligned16(p->out) && (p->out_stride_b % 4 == 0) && (p->seq % 4 == 0);
    const int nt = (p->seq + 15) / 16;
    hipStream_t st = static_cast<hipStream_t>(stream);
    switch (p->dtype) {
        case ATX_DTYPE_BF16: return dispatch_kq<__bf16>(nt, p->batch, st, a);
        case ATX_DTYPE_FP16: return dispatch_kq<_Float16>(nt, p->batch, st, a);
        default: return dispatch_kq<float>(nt, p->batch, st, a);
    }
}
