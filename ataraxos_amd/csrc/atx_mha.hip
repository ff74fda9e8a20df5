// Fused multi-head self-attention layer for gfx950 (bf16 / fp16):
//   Y = out_proj(attention(q_proj(X), k_proj(X), v_proj(X)))
// for one sample per workgroup -- the whole of MultiHeadAttention.forward
// (stratego/networks/attention.py:152-204) with key_value = None, head_dim
// 64 and num_kv_heads = num_heads.
//
// The sample's X rows stay in LDS while Q, K, V of one head at a time are
// produced into LDS by MFMA and attended over.  Q, K, V never leave the CU;
// HBM sees X once and Y once, and the weights come from L2 (1.2 MB for
// E = 384, shared by every CU).
//
// Per head h (8 waves):
//  A. [Q_h | K_h | V_h]^T = W_h X^T: 12 feature tiles x NP position tiles,
//     K = E; each wave owns whole feature tiles (2 or 1) for every position,
//     so the weight operand streams from L2 once per sample (16-byte loads,
//     the next k-step in flight), X from LDS.  Results are rounded to the
//     16-bit type (where nn.Linear rounds them) and stored row-major.
//  B. Attention, one 16-query tile per wave, as the attention kernel does
//     it: S^T = K Q^T, row softmax in registers, O^T = V^T P^T with V^T from
//     transposing LDS reads; O_h (the reference's attn_out columns
//     64h .. 64h+63) is rounded.
// The output projection Y^T = Wo O^T has wave w owning H / 2 feature tiles of
// Y for every position, in one of two forms:
//  * Y in registers (C3's shape): O_h goes to one of two LDS buffers, and
//    while head h is attended over, every wave adds Wo[:, 64(h-1) ..] O_{h-1}^T
//    (K = 64) into accumulators it keeps across the head loop;
//  * parked (where the accumulators or the second O buffer do not fit, or
//    where that form measured slower): O_h is stored to the sample's rows of
//    y, which the workgroup alone owns; after the last head those rows come
//    back into LDS in place of X and the projection runs as one GEMM (K = E).
// Both accumulate over the same k order, so they give identical results.
// Rounding points match the reference's bf16 modules: Q, K, V and O are
// rounded to the 16-bit type, every product accumulates in fp32, Y is
// rounded once at the end.
#include <stdlib.h>
#include <string.h>

#include <mutex>

#include "atx_mha.hpp"

namespace atx {

// LDS of one workgroup: X [16 np, E], Q and K [16 np, 64], V [32 ceil(np/2), 64]
// (padding rows zero), and, when Y accumulates in registers, two O_h buffers
// [16 np, 64].
constexpr size_t kMhaLdsMax = 160 * 1024;
constexpr size_t mha_lds_core(int E, int np) {
    return (size_t)16 * np * E * 2 + (size_t)(2 * 16 * np + 32 * ((np + 1) / 2)) * kD * 2;
}
constexpr size_t mha_lds_o(int np) { return (size_t)16 * np * kD * 2; }
// Y accumulated in registers across heads (H/2 feature tiles x np position
// tiles per wave, at most 84 VGPRs) when the double-buffered O_h fits in LDS;
// otherwise each head's O is parked in y and projected after the last head.
// Measured on MI355X, the register form is slower for 4 and 6 heads at
// np = 4 and for 8 heads at np <= 3 (the per-head Wo loads are exposed
// there), so those park too.
constexpr bool mha_y_in_regs(int H, int np) {
    return (H / 2) * np * 4 <= 84 && mha_lds_core(64 * H, np) + 2 * mha_lds_o(np) <= kMhaLdsMax &&
           !((H == 4 || H == 6) && np == 4) && !(H == 8 && np <= 3);
}
inline size_t mha_lds_bytes(int E, int np) {
    return mha_lds_core(E, np) + (mha_y_in_regs(E / 64, np) ? 2 * mha_lds_o(np) : 0);
}


// [Q_h | K_h | V_h]^T feature tiles (of 12: Q 0-3, K 4-7, V 8-11): tile fta
// for every position tile and, when NF = 2, tile ftb for position tiles
// PB1 .. PB1 + PN1 - 1.  X^T rows come from LDS (one read per position tile
// serves both tiles), the weight rows from memory with the next k-step in
// flight.  Results (+ bias) are rounded and stored row-major into sq / sk / sv
// after a workgroup barrier (all waves call this once per head).
template <typename T, int E, int NP, int NF, int PB1, int PN1, bool PK, int D = kD>
__device__ __forceinline__ void project_head(const lds_t* sx, lds_t* sq, lds_t* sk, lds_t* sv, const int (&xlane)[4],
                                             rsrc_t rq, rsrc_t rk, rsrc_t rv, const void* const (&bias)[4], int h,
                                             int H, int fta, int ftb, int m, int g, u32x4 (&wpre)[NF]) {
    using M = Mfma16<T>;
    constexpr int KS = E / 32;
    constexpr int TPH = D / 16;  // feature tiles per head in each of Q, K, V
    // tile f covers position tile p
    auto covers = [](int f, int p) constexpr { return f == 0 || (p >= PB1 && p < PB1 + PN1); };
    f32x4 acc[NF][NP];
#pragma unroll
    for (int f = 0; f < NF; ++f)
#pragma unroll
        for (int p = 0; p < NP; ++p) acc[f][p] = f32x4{0.f, 0.f, 0.f, 0.f};
    rsrc_t wr[NF];
    uint32_t wrow[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        const int ft = f == 0 ? fta : ftb;
        wr[f] = ft / TPH == 0 ? rq : (ft / TPH == 1 ? rk : rv);
        wrow[f] = wtile_off<E, PK>(h * TPH + ft % TPH, m, g);
    }
    // Weight k-steps stay PF ahead of the MFMAs: each iteration issues step
    // kk + PF first, and a scheduling barrier keeps the compiler from
    // sinking those loads to their use.
    // From 6 position tiles on, step 0 comes from `wpre`, loaded by the
    // previous head's call (so its L2 latency passes under that head's
    // attention), or here for head 0.  (At shorter lengths this measured
    // slower on MI355X: each head loads step 0 at its start.)
    constexpr bool WPRE = NP >= 6;
    constexpr int PF = KS < PFD ? KS : PFD;
    u32x4 wbuf[PF][NF];
    if (!WPRE || h == 0)
#pragma unroll
        for (int f = 0; f < NF; ++f) wpre[f] = buf_ld16_keep(wr[f], wrow[f]);
#pragma unroll
    for (int s = 0; s < PF; ++s)
#pragma unroll
        for (int f = 0; f < NF; ++f) wbuf[s][f] = s == 0 ? wpre[f] : buf_ld16_keep(wr[f], wrow[f] + s * kWStep<PK>);
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
        u32x4 cur[NF], nxt[NF];
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            cur[f] = wbuf[kk % PF][f];
            if (kk + PF < KS) nxt[f] = buf_ld16_keep(wr[f], wrow[f] + (kk + PF) * kWStep<PK>);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const u32x4 xb = lds_ld16(sx + xlane[kk & 3] + p * 16 * E * 2 + (kk >> 2) * 256);
#pragma unroll
            for (int f = 0; f < NF; ++f)
                if (covers(f, p)) acc[f][p] = M::mma(cur[f], xb, acc[f][p]);
        }
        if (kk + PF < KS)
#pragma unroll
            for (int f = 0; f < NF; ++f) wbuf[kk % PF][f] = nxt[f];
    }
    // Step 0 of head h + 1 (its rows start D rows further down).
    if (WPRE && h + 1 < H)
#pragma unroll
        for (int f = 0; f < NF; ++f) wpre[f] = buf_ld16_keep(wr[f], wrow[f] + D * E * 2);
    __syncthreads();  // every wave is done with the previous head's Q, K, V
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        const int ft = f == 0 ? fta : ftb;
        f32x4 bv = f32x4{0.f, 0.f, 0.f, 0.f};  // bias of features 4g .. 4g+3 of the tile
        const T* bp = static_cast<const T*>(bias[ft / TPH]);
        if (bp) {
            const int feat = h * D + (ft % TPH) * 16 + 4 * g;
#pragma unroll
            for (int i = 0; i < 4; ++i) bv[i] = static_cast<float>(bp[feat + i]);
        }
        lds_t* const dst = ft < TPH ? sq : (ft < 2 * TPH ? sk : sv);
#pragma unroll
        for (int p = 0; p < NP; ++p)
            if (covers(f, p))
            lds_st8(dst + xquad<kD>(p * 16 + m, (ft % TPH) * 16 + 4 * g),
                    u32x2{M::pack2(acc[f][p][0] + bv[0], acc[f][p][1] + bv[1]),
                          M::pack2(acc[f][p][2] + bv[2], acc[f][p][3] + bv[3])});
    }
}

// H heads of D (64, or 48 with 8 heads), NP 16-row position tiles (L <= 16 NP).
// With D = 48 the head's Q, K, V rows keep the 64-element LDS rows of D = 64
// with elements 48 .. 63 zero, so the attention runs unchanged (the padded
// dot-product terms and output columns are exact zeros; those columns are
// not stored), and O always takes the parked form.
template <typename T, int H, int NP, bool CAUSAL, bool PK, int D = kD>
__global__ __launch_bounds__(kThreads) void mha_fused(MhaArgs a) {
    using M = Mfma16<T>;
    static_assert(D == kD || (D == 48 && H == 8), "head_dim 64, or 48 with 8 heads");
    constexpr int E = H * D;
    constexpr int LP = NP * 16;
    constexpr int NKC = (NP + 1) / 2;  // 32-key chunks
    constexpr int LV = NKC * 32;       // V rows staged
    constexpr int KS = E / 32;         // k-steps of a projection
    constexpr int FT = E / 128;        // output feature tiles of a wave (E / 16 over 8 waves)
    constexpr int PF = KS < PFD ? KS : PFD;  // weight prefetch depth (k-steps)
    constexpr int XC = E / 8;          // 16-byte chunks per X row
    constexpr bool YREG = D == kD && mha_y_in_regs(H, NP);
    static_assert(H % 2 == 0 && H <= 8, "H even, at most 8");
    static_assert(kWaves == 8, "wave roles assume 8 waves");

    lds_t* const sx0 = lds_base();
    lds_t* const sq0 = sx0 + LP * E * 2;  // Q_h
    lds_t* const sk0 = sq0 + LP * kD * 2;
    lds_t* const sv0 = sk0 + LP * kD * 2;
    lds_t* const so0 = sv0 + LV * kD * 2;  // O_h, buffer h & 1 (Y in registers only)

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar descriptors per wave
    const int m = lane & 15, g = lane >> 4;
    const int b = blockIdx.x;
    const int L = a.L;

    // ---- X rows (rows past L read 0), V padding rows zeroed --------------------
    {
        const rsrc_t rx = make_rsrc(static_cast<const T*>(a.x) + b * a.xsb, (uint32_t)(((L - 1) * a.xss + E) * 2));
        constexpr int N = LP * XC;
        constexpr int U = (N + kThreads - 1) / kThreads;
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int idx = u * kThreads + tid;
            const int r = idx / XC, c = idx - (idx / XC) * XC;
            v[u] = buf_ld16(rx, idx < N ? (uint32_t)(r * a.xss + c * 8) * 2 : 0xfffffff0u);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int idx = u * kThreads + tid;
            const int r = idx / XC, c = idx - (idx / XC) * XC;
            if (idx < N) lds_st16(sx0 + eoff<E>(r, c), v[u]);
        }
        for (int idx = tid; idx < (LV - LP) * 8; idx += kThreads)
            lds_st16(sv0 + LP * kD * 2 + idx * 16, u32x4{0, 0, 0, 0});
        if constexpr (D < kD)  // elements D .. 63 of every Q, K and V row: zero, never written
            for (int idx = tid; idx < (2 * LP + LV) * (kD - D) / 8; idx += kThreads) {
                const int r = idx / ((kD - D) / 8), c = D / 8 + idx % ((kD - D) / 8);
                lds_st16(sq0 + xoff<kD>(r, c), u32x4{0, 0, 0, 0});
            }
    }

    const rsrc_t ry = make_rsrc(static_cast<const T*>(a.y) + b * a.ysb, (uint32_t)(((L - 1) * a.yss + E) * 2));
    // Weight descriptors (each matrix E x E).
    rsrc_t rw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) rw[i] = make_rsrc(a.w[i], (uint32_t)(E * E * 2));

    // Transposing-read offsets into V (rows 4g + t, elements a4*16 + 4dt).
    int troff[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) troff[dt] = xquad<kD>(4 * g + (m >> 2), (m & 3) * 16 + 4 * dt);

    // X / O rows in LDS: row pt*16 + m, logical chunk kk*4 + g sits at
    // xlane[kk & 3] + pt*16*E*2 + (kk >> 2)*256 (the swizzle term depends on
    // m only, since 16 pt is a multiple of 16).
    int xlane[4];
#pragma unroll
    for (int par = 0; par < 4; ++par) xlane[par] = m * E * 2 + (((4 * par + g) ^ m) & 15) * 16;

    // Output projection: wave w owns Y feature tiles FT w .. FT w + FT - 1 for
    // every position.
    uint32_t orow[FT];
#pragma unroll
    for (int f = 0; f < FT; ++f) orow[f] = wtile_off<E, PK>(wave * FT + f, m, g);
    f32x4 yacc[FT][NP];
#pragma unroll
    for (int f = 0; f < FT; ++f)
#pragma unroll
        for (int p = 0; p < NP; ++p) yacc[f][p] = f32x4{0.f, 0.f, 0.f, 0.f};

    u32x4 wpre[2], wpre1[1];  // step-0 weights of the next head (Q/K waves, V waves)

    __syncthreads();

    for (int h = 0; h < H; ++h) {
        // LDS bases re-derived per head through an opaque copy: otherwise the
        // compiler hoists every per-tile address of both phases out of the
        // head loop and runs out of registers.
        lds_t* const sx = lds_opaque(sx0);
        lds_t* const sq = lds_opaque(sq0);
        lds_t* const sk = lds_opaque(sk0);
        lds_t* const sv = lds_opaque(sv0);
        // ---- A: [Q_h | K_h | V_h]^T: waves 0..3 own feature tiles 2w, 2w+1
        // (Q, K), waves 4..7 tile 4 + w (V), each for every position, so every
        // weight element crosses from L2 once per sample and each SIMD holds
        // one 2-tile and one 1-tile wave.
        if constexpr (D == kD) {
            if (wave < 4)
                project_head<T, E, NP, 2, 0, NP, PK>(sx, sq, sk, sv, xlane, rw[0], rw[1], rw[2], a.bias, h, H, 2 * wave, 2 * wave + 1, m, g, wpre);
            else
                project_head<T, E, NP, 1, 0, 0, PK>(sx, sq, sk, sv, xlane, rw[0], rw[1], rw[2], a.bias, h, H, 4 + wave, 0, m, g, wpre1);
        } else {
            // 9 feature tiles (Q 0-2, K 3-5, V 6-8): wave w owns tile w, wave 0 also tile 8.
            if (wave == 0)
                project_head<T, E, NP, 2, 0, NP, PK, D>(sx, sq, sk, sv, xlane, rw[0], rw[1], rw[2], a.bias, h, H, 0, 8, m, g, wpre);
            else
                project_head<T, E, NP, 1, 0, 0, PK, D>(sx, sq, sk, sv, xlane, rw[0], rw[1], rw[2], a.bias, h, H, wave, 0, m, g, wpre1);
        }
        __syncthreads();

        // ---- B: attention of head h, one query tile per wave -------------------
        if constexpr (YREG) {
            // O_h into LDS buffer h & 1; meanwhile the output projection of head
            // h - 1 reads buffer (h - 1) & 1, complete since the barrier above
            // and not written again before the barrier after the next
            // projections.
            lds_t* const so = lds_opaque(so0);
            u32x4 wo[2][FT];  // Wo operands of head h - 1, in flight during the attention
            if (h > 0)
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int f = 0; f < FT; ++f)
                        wo[j][f] = buf_ld16_keep(rw[3], orow[f] + (uint32_t)(2 * h - 2 + j) * kWStep<PK>);
            if (wave < NP) {
                u32x4 out[2];
                attend_tile<T, NP, CAUSAL>(sq, sk, sv, troff, wave, L, a.c2, m, g, out);
#pragma unroll
                for (int half = 0; half < 2; ++half)
                    lds_st16(so + (h & 1) * LP * kD * 2 + xoff<kD>(wave * 16 + m, 2 * g + half), out[half]);
            }
            if (h > 0) out_proj_head<T, FT, NP>(yacc, wo, so + ((h - 1) & 1) * LP * kD * 2, m, g);
        } else {
            // O_h parked in the sample's own rows of y (the reference's
            // attn_out columns 64h .. 64h + 63; rows past L are dropped).
            if (wave < NP) {
                u32x4 out[2];
                attend_tile<T, NP, CAUSAL>(sq, sk, sv, troff, wave, L, a.c2, m, g, out);
                if (16 * g < D)
#pragma unroll
                    for (int half = 0; half < 2; ++half)
                        buf_st16_cached(ry, (uint32_t)((wave * 16 + m) * a.yss + h * D + 16 * g + 8 * half) * 2, out[half]);
            }
        }
    }

    if constexpr (YREG) {
        __syncthreads();  // every O_{H-1} row is in LDS
        u32x4 wo[2][FT];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int f = 0; f < FT; ++f) wo[j][f] = buf_ld16_keep(rw[3], orow[f] + (uint32_t)(2 * H - 2 + j) * kWStep<PK>);
        out_proj_head<T, FT, NP>(yacc, wo, lds_opaque(so0) + ((H - 1) & 1) * LP * kD * 2, m, g);
    } else {
        // Every head's O store has completed (s_waitcnt 0: acknowledged by the
        // L2 this CU writes through) before any wave of the workgroup reads the
        // rows back with L1-bypassing loads.  Only this workgroup touches these
        // rows, so no wider fence (which would write back and invalidate L2) is
        // needed.
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        // O (all heads) back into LDS in place of X: reads bypass L1
        {
            constexpr int N = LP * XC;
            constexpr int U = (N + kThreads - 1) / kThreads;
            u32x4 v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int idx = u * kThreads + tid;
                const int r = idx / XC, c = idx - (idx / XC) * XC;
                v[u] = __builtin_amdgcn_raw_buffer_load_b128(ry, (int)(idx < N ? (uint32_t)(r * a.yss + c * 8) * 2 : 0xfffffff0u),
                                                             0, kAuxGlc);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int idx = u * kThreads + tid;
                const int r = idx / XC, c = idx - (idx / XC) * XC;
                if (idx < N) lds_st16(sx0 + eoff<E>(r, c), v[u]);
            }
        }
        __syncthreads();
        // Y^T = Wo O^T as one GEMM over all heads (K = E)
        u32x4 wbuf[PF][FT];
#pragma unroll
        for (int s2 = 0; s2 < PF; ++s2)
#pragma unroll
            for (int f = 0; f < FT; ++f) wbuf[s2][f] = buf_ld16_keep(rw[3], orow[f] + (uint32_t)s2 * kWStep<PK>);
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
            u32x4 wa[FT], nxt[FT];
#pragma unroll
            for (int f = 0; f < FT; ++f) {
                wa[f] = wbuf[kk % PF][f];
                if (kk + PF < KS) nxt[f] = buf_ld16_keep(rw[3], orow[f] + (uint32_t)(kk + PF) * kWStep<PK>);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                const u32x4 ob = lds_ld16(sx0 + xlane[kk & 3] + p * 16 * E * 2 + (kk >> 2) * 256);
#pragma unroll
                for (int f = 0; f < FT; ++f) yacc[f][p] = M::mma(wa[f], ob, yacc[f][p]);
            }
            if (kk + PF < KS)
#pragma unroll
                for (int f = 0; f < FT; ++f) wbuf[kk % PF][f] = nxt[f];
        }
    }

    // ---- Y (+ bias), rounded once; rows past L are dropped -------------------------
    const T* const bo = static_cast<const T*>(a.bias[3]);
#pragma unroll
    for (int f = 0; f < FT; ++f) {
        const int feat = (wave * FT + f) * 16 + 4 * g;
        f32x4 bv = f32x4{0.f, 0.f, 0.f, 0.f};
        if (bo)
#pragma unroll
            for (int i = 0; i < 4; ++i) bv[i] = static_cast<float>(bo[feat + i]);
#pragma unroll
        for (int p = 0; p < NP; ++p)
            buf_st8_cached(ry, (uint32_t)((p * 16 + m) * a.yss + feat) * 2,
                           u32x2{M::pack2(yacc[f][p][0] + bv[0], yacc[f][p][1] + bv[1]),
                                 M::pack2(yacc[f][p][2] + bv[2], yacc[f][p][3] + bv[3])});
    }
}

namespace {

template <typename K>
int launch_mha(K kernel, int grid, size_t lds, hipStream_t st, const MhaArgs& a) {
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) ATX_FAIL(ATX_ERR_LAUNCH, "hipFuncSetAttribute(%zu bytes LDS): %s", lds, hipGetErrorString(e));
    }
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kThreads), lds, st, a);
    ATX_CHECK_LAUNCH("atx_mha_fwd launch");
    return ATX_OK;
}

template <typename T, int H, bool CAUSAL, bool PK, int D = kD>
int dispatch_mha_np(int np, int grid, size_t lds, hipStream_t st, const MhaArgs& a) {
    switch (np) {
        case 1: return launch_mha(mha_fused<T, H, 1, CAUSAL, PK, D>, grid, lds, st, a);
        case 2: return launch_mha(mha_fused<T, H, 2, CAUSAL, PK, D>, grid, lds, st, a);
        case 3: return launch_mha(mha_fused<T, H, 3, CAUSAL, PK, D>, grid, lds, st, a);
        case 4: return launch_mha(mha_fused<T, H, 4, CAUSAL, PK, D>, grid, lds, st, a);
        case 5: return launch_mha(mha_fused<T, H, 5, CAUSAL, PK, D>, grid, lds, st, a);
        case 6: return launch_mha(mha_fused<T, H, 6, CAUSAL, PK, D>, grid, lds, st, a);
        case 7: return launch_mha(mha_fused<T, H, 7, CAUSAL, PK, D>, grid, lds, st, a);
        case 8: return launch_mha(mha_fused<T, H, 8, CAUSAL, PK, D>, grid, lds, st, a);
        default: ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_mha_fwd: %d position tiles", np);
    }
}

// head_dim 64: 2, 4, 6 or 8 heads; head_dim 48: 8 heads (embed_dim 384).
template <typename T, bool CAUSAL, bool PK>
int dispatch_mha(int H, int D, int np, int grid, size_t lds, hipStream_t st, const MhaArgs& a) {
    if (D == 48) {
        if (H == 8) return dispatch_mha_np<T, 8, CAUSAL, PK, 48>(np, grid, lds, st, a);
        ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_mha_fwd: head_dim 48 with %d heads (8 only)", H);
    }
    switch (H) {
        case 2: return dispatch_mha_np<T, 2, CAUSAL, PK>(np, grid, lds, st, a);
        case 4: return dispatch_mha_np<T, 4, CAUSAL, PK>(np, grid, lds, st, a);
        case 6: return dispatch_mha_np<T, 6, CAUSAL, PK>(np, grid, lds, st, a);
        case 8: return dispatch_mha_np<T, 8, CAUSAL, PK>(np, grid, lds, st, a);
        default: ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_mha_fwd: %d heads not supported (2, 4, 6, 8)", H);
    }
}

}  // namespace
}  // namespace atx

namespace atx {
namespace {

// Validates `p` for entry point `fn` and fills the kernel arguments, the
// position-tile count and the LDS size; no HIP call.
int mha_check(const AtxMhaParams* p, const char* fn, MhaArgs& a, int& np, size_t& lds) {
    if (!p) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "%s: params is NULL", fn);
    if (p->abi_version != ATX_ABI_VERSION)
        ATX_FAIL(ATX_ERR_ABI, "%s: abi_version %d, library is %d", fn, p->abi_version, ATX_ABI_VERSION);
    if (p->dtype != ATX_DTYPE_BF16 && p->dtype != ATX_DTYPE_FP16) {
        if (p->dtype == ATX_DTYPE_FP32) ATX_FAIL(ATX_ERR_UNSUPPORTED, "%s: fp32 is not supported", fn);
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "%s: unknown dtype %d", fn, p->dtype);
    }
    if (p->batch < 1 || p->seq < 1 || p->num_heads < 1)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "%s: sizes must be >= 1", fn);
    const bool d48 = p->num_heads == 8 && p->embed_dim == 384;  // the reference Move network's 8 x 48
    if (p->embed_dim != p->num_heads * 64 && !d48)
        ATX_FAIL(ATX_ERR_UNSUPPORTED, "%s: head_dim %d not supported (64; 48 with 8 heads)", fn,
                 p->num_heads > 0 ? p->embed_dim / p->num_heads : 0);
    if (p->num_heads != 2 && p->num_heads != 4 && p->num_heads != 6 && p->num_heads != 8)
        ATX_FAIL(ATX_ERR_UNSUPPORTED, "%s: %d heads not supported (2, 4, 6, 8)", fn, p->num_heads);
    if (!p->x || !p->w_q || !p->w_k || !p->w_v || !p->w_o || !p->y)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "%s: null tensor pointer", fn);
    if (!(p->scale > 0.f) || p->scale == __builtin_inff())
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "%s: scale must be finite and > 0 (got %g)", fn, (double)p->scale);
    if (p->seq > 128) ATX_FAIL(ATX_ERR_UNSUPPORTED, "%s: seq %d not supported (<= 128)", fn, p->seq);
    const int E = p->embed_dim, L = p->seq;
    const int64_t xss = L == 1 ? E : p->x_stride_s, yss = L == 1 ? E : p->y_stride_s;
    if (!aligned16(p->x) || !aligned16(p->y) || ((p->x_stride_b * 2) & 15) || ((xss * 2) & 15) ||
        ((p->y_stride_b * 2) & 15) || ((yss * 2) & 15))
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "%s: x/y rows must start on a 16-byte boundary", fn);
    if (!aligned16(p->w_q) || !aligned16(p->w_k) || !aligned16(p->w_v) || !aligned16(p->w_o))
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "%s: weights must be 16-byte aligned, contiguous [E, E]", fn);
    if (xss < 0 || yss < E || (int64_t)(L + 16) * xss * 2 + E * 2 > 0x7fffffffLL ||
        (int64_t)(L + 16) * yss * 2 + E * 2 > 0x7fffffffLL)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "%s: row strides must be >= 0 (y: >= embed_dim) and one sample < 2 GiB", fn);
    np = (L + 15) / 16;
    lds = d48 ? mha_lds_core(E, np) : mha_lds_bytes(E, np);  // head_dim 48: O parked, no O buffers
    if (lds > 160 * 1024)
        ATX_FAIL(ATX_ERR_UNSUPPORTED, "%s: seq %d, embed_dim %d need %zu bytes of LDS (> 160 KiB)", fn, L, E, lds);

    a.x = p->x; a.xsb = p->x_stride_b; a.xss = (int)xss;
    a.w[0] = p->w_q; a.w[1] = p->w_k; a.w[2] = p->w_v; a.w[3] = p->w_o;
    a.bias[0] = p->b_q; a.bias[1] = p->b_k; a.bias[2] = p->b_v; a.bias[3] = p->b_o;
    a.y = p->y; a.ysb = p->y_stride_b; a.yss = (int)yss;
    a.L = L;
    a.c2 = p->scale * kLog2e;
    // The attention half of a pre-LN block: the persistent form only.
    if (p->ln_bias && !p->ln_weight) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "%s: ln_bias without ln_weight", fn);
    if (p->residual != 0 && p->residual != 1) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "%s: residual must be 0 or 1", fn);
    if (p->ln_weight || p->residual) {
        if (!(p->num_heads == 6 && E == 6 * kD && mha_ws_lds_bytes(E, L)))
            ATX_FAIL(ATX_ERR_UNSUPPORTED, "%s: pre-LN / residual need 6 heads of 64 at 65..101 positions (got %d heads, embed_dim %d, seq %d)",
                     fn, p->num_heads, E, L);
        if (p->ln_weight && (!aligned16(p->ln_weight) || (p->ln_bias && !aligned16(p->ln_bias))))
            ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "%s: ln_weight / ln_bias must be 16-byte aligned [embed_dim]", fn);
        if (p->ln_weight && !(p->ln_eps >= 0.f && p->ln_eps < __builtin_inff()))
            ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "%s: ln_eps must be finite and >= 0 (got %g)", fn, (double)p->ln_eps);
    }
    a.ln_w = p->ln_weight;
    a.ln_b = p->ln_bias;
    a.ln_eps = p->ln_eps;
    a.residual = p->residual;
    return ATX_OK;
}

int mha_launch(const AtxMhaParams* p, const MhaArgs& a, int np, size_t lds, hipStream_t st, bool packed) {
    const int H = p->num_heads;
    const int D = p->embed_dim / H;
    const bool bf = p->dtype == ATX_DTYPE_BF16;
    // The persistent form (6 heads of 64) where it applies, unless
    // ATX_MHA_PERSISTENT=0 (both forms give identical results; the switch
    // exists to compare them).
    if (const size_t wl = H == 6 && D == kD ? mha_ws_lds_bytes(p->embed_dim, p->seq) : 0) {
        const char* env = getenv("ATX_MHA_PERSISTENT");
        if (!env || strcmp(env, "0") != 0 || a.ln_w || a.residual)
            return mha_ws_launch(p->seq, p->causal != 0, bf, packed, p->batch, wl, st, a);
    }
    if (packed) {
        if (bf) return p->causal ? dispatch_mha<__bf16, true, true>(H, D, np, p->batch, lds, st, a)
                                 : dispatch_mha<__bf16, false, true>(H, D, np, p->batch, lds, st, a);
        return p->causal ? dispatch_mha<_Float16, true, true>(H, D, np, p->batch, lds, st, a)
                         : dispatch_mha<_Float16, false, true>(H, D, np, p->batch, lds, st, a);
    }
    if (bf) return p->causal ? dispatch_mha<__bf16, true, false>(H, D, np, p->batch, lds, st, a)
                             : dispatch_mha<__bf16, false, false>(H, D, np, p->batch, lds, st, a);
    return p->causal ? dispatch_mha<_Float16, true, false>(H, D, np, p->batch, lds, st, a)
                     : dispatch_mha<_Float16, false, false>(H, D, np, p->batch, lds, st, a);
}

int mha_fwd(const AtxMhaParams* p, void* stream, bool packed) {
    const char* const fn = packed ? "atx_mha_fwd_packed" : "atx_mha_fwd";
    clear_error();
    MhaArgs a;
    int np = 0;
    size_t lds = 0;
    if (const int rc = mha_check(p, fn, a, np, lds)) return rc;
    return mha_launch(p, a, np, lds, static_cast<hipStream_t>(stream), packed);
}

// Packed tile order of one [E, E] weight (see wtile_off): thread i writes
// 16-byte chunk i of the packed matrix.
__global__ __launch_bounds__(256) void mha_pack_weight(const uint16_t* __restrict__ w, uint16_t* __restrict__ out, int E) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int ks = E / 32;
    if (i >= E * ks * 4) return;  // E * E / 8 chunks
    const int lane = i & 63, t = i >> 6;
    const int kt = t % ks, rt = t / ks;
    const int m = lane & 15, g = lane >> 4;
    st16(out + (size_t)i * 8, ld16(w + (size_t)(rt * 16 + m) * E + kt * 32 + g * 8));
}

// The four weights of a layer into consecutive packed [E, E] matrices in one
// launch (blockIdx.y = q, k, v, out).
struct Pack4Args {
    const uint16_t* w[4];
    uint16_t* out;
    int E;
};
__global__ __launch_bounds__(256) void mha_pack_weights4(Pack4Args a) {
    const int which = blockIdx.y;
    const uint16_t* const w = which == 0 ? a.w[0] : which == 1 ? a.w[1] : which == 2 ? a.w[2] : a.w[3];
    const int E = a.E;
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int ks = E / 32;
    if (i >= E * ks * 4) return;
    const int lane = i & 63, t = i >> 6;
    const int kt = t % ks, rt = t / ks;
    const int m = lane & 15, g = lane >> 4;
    st16(a.out + (size_t)which * E * E + (size_t)i * 8, ld16(w + (size_t)(rt * 16 + m) * E + kt * 32 + g * 8));
}

inline bool overlaps(const void* a, size_t na, const void* b, size_t nb) {
    const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    return x < y + nb && y < x + na;
}

// Shared body of atx_mha_fwd_ws and atx_mha_fwd_noalloc: validate, check the
// workspace against the layer, pack the four row-major weights into it (one
// launch), run the packed-order kernel from it.
int mha_fwd_repack(const AtxMhaParams* p, void* ws, int64_t ws_bytes, hipStream_t st, const char* fn) {
    MhaArgs a;
    int np = 0;
    size_t lds = 0;
    if (const int rc = mha_check(p, fn, a, np, lds)) return rc;
    const int E = p->embed_dim;
    const size_t mat = (size_t)E * E * 2, need = 4 * mat;
    if (!ws) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "%s: workspace is NULL", fn);
    if (reinterpret_cast<uintptr_t>(ws) & 255) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "%s: workspace must be 256-byte aligned", fn);
    if (ws_bytes < 0 || (size_t)ws_bytes < need)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "%s: workspace of %lld bytes, embed_dim %d needs %zu", fn, (long long)ws_bytes, E,
                 need);
    const void* const w[4] = {p->w_q, p->w_k, p->w_v, p->w_o};
    for (int i = 0; i < 4; ++i)
        if (overlaps(ws, need, w[i], mat)) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "%s: workspace overlaps a weight", fn);
    // extents of x and y (first to last element touched, strides >= 0)
    const auto extent = [&](int64_t sb, int64_t ss) {
        return (size_t)(((int64_t)(p->batch - 1) * (sb > 0 ? sb : 0) + (int64_t)(p->seq - 1) * ss + E) * 2);
    };
    if (overlaps(ws, need, p->x, extent(p->x_stride_b, a.xss)) || overlaps(ws, need, p->y, extent(p->y_stride_b, a.yss)))
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "%s: workspace overlaps x or y", fn);
    Pack4Args pa;
    for (int i = 0; i < 4; ++i) pa.w[i] = static_cast<const uint16_t*>(w[i]);
    pa.out = static_cast<uint16_t*>(ws);
    pa.E = E;
    const int chunks = E * E / 8;
    hipLaunchKernelGGL(mha_pack_weights4, dim3((chunks + 255) / 256, 4), dim3(256), 0, st, pa);
    ATX_CHECK_LAUNCH("atx_mha pack launch");
    for (int i = 0; i < 4; ++i) a.w[i] = static_cast<const char*>(ws) + i * mat;
    return mha_launch(p, a, np, lds, st, true);
}

}  // namespace
}  // namespace atx

extern "C" int atx_mha_fwd(const AtxMhaParams* p, void* stream) { return atx::mha_fwd(p, stream, false); }

extern "C" int atx_mha_fwd_packed(const AtxMhaParams* p, void* stream) { return atx::mha_fwd(p, stream, true); }

extern "C" int64_t atx_mha_workspace_bytes(int32_t embed_dim) {
    return embed_dim > 0 ? 4 * (int64_t)embed_dim * embed_dim * 2 : 0;
}

extern "C" int atx_mha_fwd_ws(const AtxMhaParams* p, void* workspace, int64_t workspace_bytes, void* stream) {
    atx::clear_error();
    return atx::mha_fwd_repack(p, workspace, workspace_bytes, static_cast<hipStream_t>(stream), "atx_mha_fwd_ws");
}

// ---- the allocate-nothing variant -------------------------------------------
// Device memory of atx_mha_fwd_noalloc: the four packed weights of one layer
// (embed_dim <= 512).  Each GPU the library runs on holds its own copy until
// the process ends.  In host code `scratch` names a host-side stand-in, not a
// device address: only the per-device pointer from hipGetSymbolAddress is
// ever handed to a kernel.
static __device__ __align__(256) unsigned char scratch[ATX_MHA_NOALLOC_SCRATCH_BYTES];

namespace atx {
namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};  // device address of `scratch`, per device

// The current device's address of `scratch`, resolved once per device (with
// that device current) on its first call.
int scratch_for_current_device(hipStream_t st, void** out, const char* fn) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) ATX_FAIL(ATX_ERR_LAUNCH, "%s: hipGetDevice: %s", fn, hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) ATX_FAIL(ATX_ERR_UNSUPPORTED, "%s: device %d (at most %d devices)", fn, dev, kMaxDevices);
    if (st) {
        int sdev = -1;
        e = hipStreamGetDevice(st, &sdev);
        if (e != hipSuccess) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "%s: hipStreamGetDevice: %s", fn, hipGetErrorString(e));
        if (sdev != dev)
            ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "%s: the stream belongs to device %d, the current device is %d", fn, sdev, dev);
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            ATX_FAIL(ATX_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch) on device %d: %s", fn, dev, hipGetErrorString(e));
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return ATX_OK;
}
}  // namespace
}  // namespace atx

extern "C" int atx_mha_fwd_noalloc(const AtxMhaParams* p, void* stream) {
    using namespace atx;
    const char* const fn = "atx_mha_fwd_noalloc";
    clear_error();
    if (!p) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "%s: params is NULL", fn);
    const int64_t need = atx_mha_workspace_bytes(p->embed_dim);
    if (need > (int64_t)ATX_MHA_NOALLOC_SCRATCH_BYTES)
        ATX_FAIL(ATX_ERR_UNSUPPORTED, "%s: embed_dim %d needs %lld bytes of scratch, the maximum is %lld (embed_dim <= 512)",
                 fn, p->embed_dim, (long long)need, (long long)ATX_MHA_NOALLOC_SCRATCH_BYTES);
    {
        // everything about the layer is checked before the first HIP call
        MhaArgs a;
        int np = 0;
        size_t lds = 0;
        if (const int rc = mha_check(p, fn, a, np, lds)) return rc;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    void* ptr = nullptr;
    if (const int rc = scratch_for_current_device(st, &ptr, fn)) return rc;
    return mha_fwd_repack(p, ptr, (int64_t)ATX_MHA_NOALLOC_SCRATCH_BYTES, st, fn);
}

extern "C" int atx_mha_pack_weight(int dtype, int dim, const void* w, void* packed, void* stream) {
    using namespace atx;
    clear_error();
    if (dtype != ATX_DTYPE_BF16 && dtype != ATX_DTYPE_FP16)
        ATX_FAIL(dtype == ATX_DTYPE_FP32 ? ATX_ERR_UNSUPPORTED : ATX_ERR_INVALID_ARGUMENT,
                 "atx_mha_pack_weight: dtype %d (16-bit only)", dtype);
    if (dim < 32 || dim % 32 || dim > 4096)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_mha_pack_weight: dim %d must be a multiple of 32 in [32, 4096]", dim);
    if (!w || !packed) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_mha_pack_weight: null tensor pointer");
    if (!aligned16(w) || !aligned16(packed))
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_mha_pack_weight: weights must be 16-byte aligned");
    const uintptr_t wa = reinterpret_cast<uintptr_t>(w), pa = reinterpret_cast<uintptr_t>(packed);
    const uintptr_t bytes = (uintptr_t)dim * dim * 2;
    if (wa < pa + bytes && pa < wa + bytes) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_mha_pack_weight: w and packed overlap");
    const int chunks = dim * dim / 8;
    hipLaunchKernelGGL(mha_pack_weight, dim3((chunks + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint16_t*>(w), static_cast<uint16_t*>(packed), dim);
    ATX_CHECK_LAUNCH("atx_mha_pack_weight launch");
    return ATX_OK;
}
