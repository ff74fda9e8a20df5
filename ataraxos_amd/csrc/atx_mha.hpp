// Device helpers shared by the fused self-attention layer kernels
// (atx_mha.hip: one workgroup per sample, all waves on one phase at a time;
// atx_mha_ws.hip: persistent, producer and consumer waves).
#pragma once

#include "ataraxos_attn.h"
#include "atx_common.hpp"

namespace atx {

struct MhaArgs {
    const void* x;
    int64_t xsb;
    int xss;
    const void* w[4];  // q, k, v, out: [E, E] row-major (out features x in features)
    const void* bias[4];
    void* y;
    int64_t ysb;
    int yss;
    int L;
    float c2;  // scale * log2(e)
    const void* ln_w;  // pre-LN weight [E] (NULL: no LayerNorm)
    const void* ln_b;  // pre-LN bias [E] (NULL: zero)
    float ln_eps;
    int residual;      // 1: y = x + layer output
    int ws_spin;       // atx_mha_ws.hip: polls before a wait gives up (set by mha_ws_launch)
};

namespace {

#ifndef ATX_MHA_WAVES
#define ATX_MHA_WAVES 8
#endif
constexpr int kWaves = ATX_MHA_WAVES;  // per workgroup (one workgroup per CU)
constexpr int kThreads = kWaves * 64;
constexpr int kD = 64;  // head_dim
#ifndef ATX_MHA_PREFETCH
#define ATX_MHA_PREFETCH 1
#endif
constexpr int PFD = ATX_MHA_PREFETCH;  // k-steps of weight loads in flight ahead of the MFMAs

// Row r of 64 16-bit elements (Q, K, V): 16-byte chunk c at c ^ ((r >> 1) & 7).
template <int W>
__device__ inline int xoff(int r, int c) {
    return r * W * 2 + ((c & ~7) | ((c ^ (r >> 1)) & 7)) * 16;
}
template <int W>
__device__ inline int xquad(int r, int e) {
    return xoff<W>(r, e >> 3) + (e & 7) * 2;
}
// Row r of E 16-bit elements (X, then O; E a multiple of 128): chunk c at
// (c & ~15) | ((c ^ r) & 15).  An operand read (rows 16p + m, one chunk per
// 16-lane group) then covers all 16 bank groups of a 256-byte LDS cycle.
template <int W>
__device__ inline int eoff(int r, int c) {
    return r * W * 2 + ((c & ~15) | ((c ^ r) & 15)) * 16;
}

}  // namespace

// Weights are read either as the nn.Linear matrix [E, E] (row-major: one
// operand load covers 16 rows x 64 bytes, half of each 128-byte line) or in
// the packed tile order that atx_mha_pack_weight writes: for row tile rt (16
// output features) and k-step kt (32 inputs), the 64 lanes' 16-byte operand
// chunks lie contiguous, lane 16 g + m holding row 16 rt + m, inputs
// 32 kt + 8 g .. + 7, so one load covers 8 whole lines.  Offsets in bytes of
// a lane's chunk at k-step 0, and the stride of one k-step:
template <int E, bool PK>
__device__ inline uint32_t wtile_off(int rt, int m, int g) {
    return PK ? (uint32_t)((rt * (E / 32) * 64 + 16 * g + m) * 16) : (uint32_t)((rt * 16 + m) * E + 8 * g) * 2;
}
template <bool PK>
constexpr uint32_t kWStep = PK ? 1024 : 64;
// (In both orders the next head's rows, 4 row tiles on, lie kD * E * 2 bytes
// further.)

namespace {

// Attention of one head for query tile qt (rows 16 qt .. 16 qt + 15): S^T =
// K Q^T, row softmax in registers, O^T = V^T P^T with V^T from transposing LDS
// reads.  Returns the lane's O elements 16g .. 16g + 15 of row 16 qt + m,
// rounded to T (where the reference's attention output is rounded), as two
// 16-byte chunks.
template <typename T, int NP, bool CAUSAL>
__device__ __forceinline__ void attend_tile(const lds_t* sq, const lds_t* sk, const lds_t* sv, const int (&troff)[4],
                                            int qt, int L, float c2, int m, int g, u32x4 (&out)[2]) {
    using M = Mfma16<T>;
    constexpr int NKC = (NP + 1) / 2;  // 32-key chunks
    const float kNegInf = -__builtin_inff();
    const int qrow = qt * 16 + m;
    u32x4 qop[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) qop[i] = lds_ld16(sq + xoff<kD>(qrow, 4 * i + g));
    const int kend = CAUSAL ? min(L, qt * 16 + 16) : L;  // keys >= kend are unusable for the whole tile
    // Without the causal mask every key tile (and 32-key chunk) below NP holds
    // a key < L, since 16 (NP - 1) < L: those tests are then compile-time
    // constants and the tiles' MFMAs form one straight-line block.  Only the
    // last key tile can hold keys >= L.
    const auto live = [&](int k0) { return !CAUSAL || k0 < kend; };
    f32x4 s[NP];
    float mx = kNegInf;
#pragma unroll
    for (int kt = 0; kt < NP; ++kt) {
        if (live(kt * 16)) {
            f32x4 acc = M::mma(lds_ld16(sk + xoff<kD>(kt * 16 + m, g)), qop[0], f32x4{0.f, 0.f, 0.f, 0.f});
            acc = M::mma(lds_ld16(sk + xoff<kD>(kt * 16 + m, 4 + g)), qop[1], acc);
            if (CAUSAL ? kt * 16 + 16 > min(L, qt * 16 + 1) : kt == NP - 1) {
                u32x4 ab = __builtin_bit_cast(u32x4, acc);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int key = kt * 16 + 4 * g + i;
                    const bool ok = key < L && (!CAUSAL || key <= qrow);
                    ab[i] = ok ? ab[i] : 0xff800000u;
                }
                acc = __builtin_bit_cast(f32x4, ab);
            }
            mx = fmaxf(fmaxf(mx, acc[0]), acc[1]);
            mx = fmaxf(fmaxf(mx, acc[2]), acc[3]);
            s[kt] = acc;
        }
    }
    mx = colgroup_max(mx);
    const float nb = -mx * c2;  // every query sees key 0: mx is finite
    float sum = 0.f;
#pragma unroll
    for (int kt = 0; kt < NP; ++kt) {
        if (live(kt * 16)) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                s[kt][i] = fast_exp2(__builtin_fmaf(s[kt][i], c2, nb));
                sum += s[kt][i];
            }
        }
    }
    sum = colgroup_sum(sum);
    const float rs = 1.f / sum;
    // P^T packed per 32-key chunk (unnormalised; 1/sum applied to O)
    u32x4 pk[NKC];
#pragma unroll
    for (int c = 0; c < NKC; ++c) {
        float pv[8];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int kt = 2 * c + hh;
#pragma unroll
            for (int i = 0; i < 4; ++i) pv[4 * hh + i] = (kt < NP && live(kt * 16)) ? s[kt < NP ? kt : 0][i] : 0.f;
        }
        pk[c] = u32x4{M::pack2(pv[0], pv[1]), M::pack2(pv[2], pv[3]), M::pack2(pv[4], pv[5]), M::pack2(pv[6], pv[7])};
    }
    // O^T = V^T P^T: lane m (query) gets d = 16g + 4dt + i
    f32x4 o[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NKC; ++c) {
            if (live(c * 32)) {
                const u32x2 lo = lds_ld8_tr16(sv + 32 * c * kD * 2 + troff[dt]);
                const u32x2 hi = lds_ld8_tr16(sv + (32 * c + 16) * kD * 2 + troff[dt]);
                acc = M::mma(u32x4{lo[0], lo[1], hi[0], hi[1]}, pk[c], acc);
            }
        }
        o[dt] = acc;
    }
#pragma unroll
    for (int half = 0; half < 2; ++half)
        out[half] = u32x4{M::pack2(o[2 * half][0] * rs, o[2 * half][1] * rs), M::pack2(o[2 * half][2] * rs, o[2 * half][3] * rs),
                          M::pack2(o[2 * half + 1][0] * rs, o[2 * half + 1][1] * rs),
                          M::pack2(o[2 * half + 1][2] * rs, o[2 * half + 1][3] * rs)};
}

// Y^T += Wo[:, 64h .. 64h+63] O_h^T over the wave's FT feature tiles and every
// position tile (K = 64: two k-steps); `wo` holds the Wo operands of head h.
template <typename T, int FT, int NP>
__device__ __forceinline__ void out_proj_head(f32x4 (&yacc)[FT][NP], const u32x4 (&wo)[2][FT], const lds_t* so, int m,
                                              int g) {
    using M = Mfma16<T>;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const u32x4 ob = lds_ld16(so + xoff<kD>(p * 16 + m, 4 * j + g));
#pragma unroll
            for (int f = 0; f < FT; ++f) yacc[f][p] = M::mma(wo[j][f], ob, yacc[f][p]);
        }
}

}  // namespace

// The persistent producer/consumer form of the layer (atx_mha_ws.hip): LDS
// bytes it needs (0 where the shape is outside it) and its launch over
// `batch` samples.
size_t mha_ws_lds_bytes(int E, int L);
int mha_ws_launch(int L, bool causal, bool bf16, bool packed, int batch, size_t lds, hipStream_t st, const MhaArgs& a);

}  // namespace atx
