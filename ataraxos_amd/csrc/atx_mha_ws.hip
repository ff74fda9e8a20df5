// Fused multi-head self-attention layer, persistent with producer and
// consumer waves (bf16 / fp16), for 6 heads of 64 (embed_dim 384) at 65 to
// 101 positions -- C3's Move-network layer:
//   Y = out_proj(attention(q_proj(X), k_proj(X), v_proj(X)))
// (stratego/networks/attention.py:152-204 with key_value = None), with the
// arithmetic of atx_mha.hip: the same rounding points (Q, K, V and O rounded
// to the 16-bit type, fp32 accumulation, Y rounded once) and the same k order
// of every accumulation, so both kernels give identical results.
//
// One workgroup per CU loops over the samples b = blockIdx.x + i * gridDim.x.
// Its 8 waves take two roles, one wave of each role on every SIMD:
//  * producers (waves 0..3) project: wave p computes feature tile p of Q_h, of
//    K_h and of V_h ([Q|K|V]^T = W X^T; one X^T operand read from LDS feeds
//    three MFMAs) for every position tile and stores them into LDS slot h & 1;
//  * consumers (waves 4..7) attend over head h - 1 in slot (h - 1) & 1, query
//    tiles c and c + 4 of wave 4 + c, writing O over the Q rows it came from.
// So while one head's projections keep the MFMA pipes busy, the previous
// head's softmax (VALU, LDS and latency bound) runs beside them on the same
// SIMDs.  Every wave also owns 3 of the 24 feature tiles of Y in registers
// and adds Wo[:, 64h ..] O_h^T into them one step after head h's attention.
//
// The waves synchronise through progress counters in LDS (one word per wave
// and kind, written only by that wave) instead of workgroup barriers, so
// neither role waits for the other's whole step: a producer projects head h
// (registers only), waits until slot h & 1 is free and stores into it; a
// consumer waits for that store, attends, and out-projects head h one step
// later; producers out-project head h two steps later, after projecting the
// next head (ws_producer / ws_consumer list what each wait protects).  Every
// wait is bounded (ws_wait).
//
// LDS: X (L rows, swizzled as eoff), then per slot Q and K (L rows rounded up
// to even) and V (32 ceil(NP / 2) rows).  Operand reads of the last position
// tile run past the end of a buffer into the next one; those rows only reach
// results that are dropped or replaced: Q rows past L give output rows past
// L, which the bounds of y's buffer resource drop; key scores past L are set
// to -inf before the softmax; V rows L .. are stored as zeros (rows past
// 16 NP are zeroed once), so the probability-0 keys add exact zeros.  Each
// MFMA output column depends only on its own position's operand column, so
// the values read past a buffer (even non-finite ones) stay in those columns.
#include <mutex>
#include <stdlib.h>

#include "atx_mha.hpp"

namespace atx {

namespace {

constexpr int kWsH = 6;
constexpr int kWsE = kWsH * kD;
// Y feature tiles of a producer wave (of the 24: the consumers hold the rest,
// 6 - ws_ftp each).  Measured at C3: 3 / 3 is 1.8 % faster than 2 / 4 (the
// consumers' attention is the longer chain); with the residual add, or with
// weights in the nn.Linear order (wider weight addressing), the 3 / 3 split
// spills, so those kernels keep 2 / 4.
template <bool RES, bool PK>
constexpr int ws_ftp() { return (PK && !RES) ? 3 : 2; }
#ifndef ATX_MHA_WS_PF
#define ATX_MHA_WS_PF 2
#endif
constexpr int kWsPF = ATX_MHA_WS_PF;  // weight k-steps in flight in the projections

// Progress counters, one 32-bit word per wave and kind, each written only by
// its wave and only ever increased.
constexpr int kSyncStore = 0;    // [4] producer p: heads stored into a slot
constexpr int kSyncAttn = 4;     // [4] consumer c: heads attended (O written)
constexpr int kSyncOutP = 8;     // [4] producer p: heads out-projected
constexpr int kSyncOutC = 12;    // [4] consumer c: heads out-projected
constexpr int kSyncXfree = 16;   // [4] producer p: samples whose X it has read for the last time
constexpr int kSyncXready = 20;  // [4] producer p: samples whose X rows it has written (and normalised)
constexpr int kSyncAbort = 24;   // nonzero once any wait gave up (see ws_wait)
constexpr int kSyncSpin = 25;    // polls before a wait gives up (MhaArgs::ws_spin)
constexpr int kSyncWords = 28;

constexpr int ws_lq(int L) { return (L + 1) & ~1; }
constexpr int ws_lv(int np) { return 32 * ((np + 1) / 2); }
constexpr size_t ws_slot(int L) { return (size_t)(2 * ws_lq(L) + ws_lv((L + 15) / 16)) * kD * 2; }
constexpr size_t ws_lds(int L) { return (size_t)L * kWsE * 2 + 2 * ws_slot(L) + kSyncWords * 4; }

// Publishes count v of this wave: every LDS access the wave issued before
// (reads included) has completed before the count is visible.
__device__ inline void ws_post(lds_t* sync, int word, uint32_t v) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    *reinterpret_cast<volatile __attribute__((address_space(3))) uint32_t*>(sync + 4 * word) = v;
}
// Waits until each of the NW (4 or 8) counts from `word` on is >= target;
// each poll reads them with NW / 4 16-byte LDS reads issued together.
// Bounded: a wait gives up after kWsSpin polls (about a million cycles, two
// orders of magnitude above the longest legitimate wait, one role's step),
// so the kernel ends even if the schedule were wrong.  The limit sits in LDS
// word kSyncSpin, read only once a first poll has failed (a kernel-long
// register for it costs the MFMA loops spills, and a read on every entry
// costs a satisfied wait its latency).  A wait that gives up sets the
// workgroup's abort word, and the workgroup then overwrites all of
// its samples' Y with NaN before it ends (mha_ws): a broken schedule shows
// as NaN output, never as plausible wrong numbers.
constexpr uint32_t kWsSpin = 1u << 14;  // (ATX_MHA_WS_SPIN overrides it, for the tests of this path)
#ifndef ATX_MHA_WS_SLEEP
#define ATX_MHA_WS_SLEEP 1  // s_sleep argument between polls (units of 64 cycles)
#endif
template <int NW = 4>
__device__ inline void ws_wait(const lds_t* sync, int word, uint32_t target) {
    static_assert(NW == 4 || NW == 8, "4 or 8 counters");
    typedef const volatile __attribute__((address_space(3))) u32x4 vu32x4;
    vu32x4* w = reinterpret_cast<vu32x4*>(sync + 4 * word);
    uint32_t spin = 0;
    for (uint32_t n = 1;; ++n) {
        const u32x4 a = w[0];
        uint32_t lo = min(min(a[0], a[1]), min(a[2], a[3]));
        if constexpr (NW == 8) {
            const u32x4 b = w[1];
            lo = min(lo, min(min(b[0], b[1]), min(b[2], b[3])));
        }
        if (__builtin_amdgcn_readfirstlane(lo) >= target) break;
        if (n == 1) spin = __builtin_amdgcn_readfirstlane(lds_ld4(sync + 4 * kSyncSpin));  // (off the fast path)
        if (n >= spin) {
            *reinterpret_cast<volatile __attribute__((address_space(3))) uint32_t*>(const_cast<lds_t*>(sync) + 4 * kSyncAbort) = 1u;
            break;
        }
        __builtin_amdgcn_s_sleep(ATX_MHA_WS_SLEEP);
    }
    asm volatile("" ::: "memory");  // no LDS access of the caller moves above the wait
}

// Producer p, head h: feature tile p of Q_h, K_h and V_h for every position
// tile, accumulated over the E inputs in 12 k-steps of 32.  The weight rows of
// the three tiles sit at the same offset in the three matrices; weights run
// kWsPF k-steps ahead of the MFMAs, and each X^T operand of the next k-step is
// read right after the three MFMAs that used the same register, so an LDS
// read's latency passes under the rest of the k-step.
template <typename T, int NP, bool PK>
__device__ __forceinline__ void ws_project(const lds_t* sx, int m, int g, const rsrc_t (&rw)[4], uint32_t wrow,
                                           f32x4 (&acc)[3][NP]) {
    using M = Mfma16<T>;
    constexpr int KS = kWsE / 32;
    constexpr int PF = kWsPF;
    // X^T operand rows: logical chunk kk*4 + g of row pt*16 + m sits at
    // xlane[kk & 3] + pt*16*E*2 + (kk >> 2)*256.
    int xlane[4];
#pragma unroll
    for (int par = 0; par < 4; ++par) xlane[par] = m * kWsE * 2 + (((4 * par + g) ^ m) & 15) * 16;
#pragma unroll
    for (int f = 0; f < 3; ++f)
#pragma unroll
        for (int q = 0; q < NP; ++q) acc[f][q] = f32x4{0.f, 0.f, 0.f, 0.f};
    u32x4 wbuf[PF][3];
#pragma unroll
    for (int q = 0; q < PF; ++q)
#pragma unroll
        for (int f = 0; f < 3; ++f) wbuf[q][f] = buf_ld16_keep(rw[f], wrow + q * kWStep<PK>);
    u32x4 xb[NP];
#pragma unroll
    for (int q = 0; q < NP; ++q) xb[q] = lds_ld16(sx + xlane[0] + q * 16 * kWsE * 2);
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
        u32x4 cur[3];
#pragma unroll
        for (int f = 0; f < 3; ++f) cur[f] = wbuf[kk % PF][f];
        if (kk + PF < KS)
#pragma unroll
            for (int f = 0; f < 3; ++f) wbuf[kk % PF][f] = buf_ld16_keep(rw[f], wrow + (kk + PF) * kWStep<PK>);
        // Scheduling barriers pin the loads where they are issued (the
        // compiler would otherwise sink each one to its use and wait on it).
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < NP; ++q) {
#pragma unroll
            for (int f = 0; f < 3; ++f) acc[f][q] = M::mma(cur[f], xb[q], acc[f][q]);
            if (kk + 1 < KS)
                xb[q] = lds_ld16(sx + xlane[(kk + 1) & 3] + q * 16 * kWsE * 2 + ((kk + 1) >> 2) * 256);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// Attention of one head for query tile qt (rows 16 qt .. 16 qt + 15), as
// attend_tile computes it (S^T = K Q^T, row softmax in registers, O^T = V^T
// P^T with V^T from transposing reads; same operations in the same order), with
// the LDS reads issued ahead of their MFMAs: every K operand before the S^T
// MFMAs, every V^T operand before the softmax.  Returns the lane's O elements
// 16g .. 16g + 15 of row 16 qt + m, rounded to T, as two 16-byte chunks.
template <typename T, int NP, bool CAUSAL>
__device__ __forceinline__ void ws_attend_tile(const lds_t* sq, const lds_t* sk, const lds_t* sv, int qt, int L, float c2,
                                               int m, int g, u32x4 (&out)[2]) {
    using M = Mfma16<T>;
    constexpr int NKC = (NP + 1) / 2;  // 32-key chunks
    const float kNegInf = -__builtin_inff();
    const int qrow = qt * 16 + m;
    const int kend = CAUSAL ? min(L, qt * 16 + 16) : L;  // keys >= kend are unusable for the whole tile
    // Without the causal mask every key tile (and 32-key chunk) below NP holds
    // a key < L, since 16 (NP - 1) < L: those tests are then compile-time
    // constants and the tiles' MFMAs form one straight-line block.  Only the
    // last key tile can hold keys >= L.
    const auto live = [&](int k0) { return !CAUSAL || k0 < kend; };
    u32x4 qop[2], kop[NP][2];
#pragma unroll
    for (int i = 0; i < 2; ++i) qop[i] = lds_ld16(sq + xoff<kD>(qrow, 4 * i + g));
#pragma unroll
    for (int kt = 0; kt < NP; ++kt)
        if (live(kt * 16))
#pragma unroll
            for (int i = 0; i < 2; ++i) kop[kt][i] = lds_ld16(sk + xoff<kD>(kt * 16 + m, 4 * i + g));
    __builtin_amdgcn_sched_barrier(0);
    f32x4 sc[NP];
    float mx = kNegInf;
#pragma unroll
    for (int kt = 0; kt < NP; ++kt) {
        if (live(kt * 16)) {
            f32x4 acc = M::mma(kop[kt][0], qop[0], f32x4{0.f, 0.f, 0.f, 0.f});
            acc = M::mma(kop[kt][1], qop[1], acc);
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
            sc[kt] = acc;
        }
    }
    // V^T operands (rows 4g + t of each 16-key half-chunk, elements
    // (m & 3) * 16 + 4 dt), in flight during the softmax.
    u32x2 vop[4][NKC][2];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
        const int troff = xquad<kD>(4 * g + (m >> 2), (m & 3) * 16 + 4 * dt);
#pragma unroll
        for (int c = 0; c < NKC; ++c)
            if (live(c * 32))
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) vop[dt][c][hh] = lds_ld8_tr16(sv + (32 * c + 16 * hh) * kD * 2 + troff);
    }
    __builtin_amdgcn_sched_barrier(0);
    mx = colgroup_max(mx);
    const float nb = -mx * c2;  // every query sees key 0: mx is finite
    float sum = 0.f;
#pragma unroll
    for (int kt = 0; kt < NP; ++kt) {
        if (live(kt * 16)) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sc[kt][i] = fast_exp2(__builtin_fmaf(sc[kt][i], c2, nb));
                sum += sc[kt][i];
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
            for (int i = 0; i < 4; ++i) pv[4 * hh + i] = (kt < NP && live(kt * 16)) ? sc[kt < NP ? kt : 0][i] : 0.f;
        }
        pk[c] = u32x4{M::pack2(pv[0], pv[1]), M::pack2(pv[2], pv[3]), M::pack2(pv[4], pv[5]), M::pack2(pv[6], pv[7])};
    }
    // O^T = V^T P^T: lane m (query) gets d = 16g + 4dt + i
    f32x4 o[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NKC; ++c)
            if (live(c * 32))
                acc = M::mma(u32x4{vop[dt][c][0][0], vop[dt][c][0][1], vop[dt][c][1][0], vop[dt][c][1][1]}, pk[c], acc);
        o[dt] = acc;
    }
#pragma unroll
    for (int half = 0; half < 2; ++half)
        out[half] = u32x4{M::pack2(o[2 * half][0] * rs, o[2 * half][1] * rs), M::pack2(o[2 * half][2] * rs, o[2 * half][3] * rs),
                          M::pack2(o[2 * half + 1][0] * rs, o[2 * half + 1][1] * rs),
                          M::pack2(o[2 * half + 1][2] * rs, o[2 * half + 1][3] * rs)};
}

// Two query tiles qa, qb of one head at once (no causal mask): the steps of
// ws_attend_tile for each tile, in the same order, with every K and V^T
// operand read once for both and the two tiles' chains side by side.
template <typename T, int NP>
__device__ __forceinline__ void ws_attend_pair(const lds_t* sq, const lds_t* sk, const lds_t* sv, int qa, int qb, int L, float c2,
                                               int m, int g, u32x4 (&outa)[2], u32x4 (&outb)[2]) {
    using M = Mfma16<T>;
    constexpr int NKC = (NP + 1) / 2;  // 32-key chunks
    const float kNegInf = -__builtin_inff();
    u32x4 qopa[2], qopb[2], kop[NP][2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        qopa[i] = lds_ld16(sq + xoff<kD>(qa * 16 + m, 4 * i + g));
        qopb[i] = lds_ld16(sq + xoff<kD>(qb * 16 + m, 4 * i + g));
    }
#pragma unroll
    for (int kt = 0; kt < NP; ++kt)
#pragma unroll
        for (int i = 0; i < 2; ++i) kop[kt][i] = lds_ld16(sk + xoff<kD>(kt * 16 + m, 4 * i + g));
    __builtin_amdgcn_sched_barrier(0);
    f32x4 sa[NP], sb[NP];
    float mxa = kNegInf, mxb = kNegInf;
#pragma unroll
    for (int kt = 0; kt < NP; ++kt) {
        f32x4 acca = M::mma(kop[kt][0], qopa[0], f32x4{0.f, 0.f, 0.f, 0.f});
        f32x4 accb = M::mma(kop[kt][0], qopb[0], f32x4{0.f, 0.f, 0.f, 0.f});
        acca = M::mma(kop[kt][1], qopa[1], acca);
        accb = M::mma(kop[kt][1], qopb[1], accb);
        if (kt == NP - 1) {  // the only key tile that can hold keys >= L
            u32x4 ba = __builtin_bit_cast(u32x4, acca), bb = __builtin_bit_cast(u32x4, accb);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bool ok = kt * 16 + 4 * g + i < L;
                ba[i] = ok ? ba[i] : 0xff800000u;
                bb[i] = ok ? bb[i] : 0xff800000u;
            }
            acca = __builtin_bit_cast(f32x4, ba);
            accb = __builtin_bit_cast(f32x4, bb);
        }
        mxa = fmaxf(fmaxf(mxa, acca[0]), acca[1]);
        mxa = fmaxf(fmaxf(mxa, acca[2]), acca[3]);
        mxb = fmaxf(fmaxf(mxb, accb[0]), accb[1]);
        mxb = fmaxf(fmaxf(mxb, accb[2]), accb[3]);
        sa[kt] = acca;
        sb[kt] = accb;
    }
    u32x2 vop[4][NKC][2];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
        const int troff = xquad<kD>(4 * g + (m >> 2), (m & 3) * 16 + 4 * dt);
#pragma unroll
        for (int c = 0; c < NKC; ++c)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) vop[dt][c][hh] = lds_ld8_tr16(sv + (32 * c + 16 * hh) * kD * 2 + troff);
    }
    __builtin_amdgcn_sched_barrier(0);
    mxa = colgroup_max(mxa);
    mxb = colgroup_max(mxb);
    const float nba = -mxa * c2, nbb = -mxb * c2;  // every query sees key 0: both maxima are finite
    float suma = 0.f, sumb = 0.f;
#pragma unroll
    for (int kt = 0; kt < NP; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sa[kt][i] = fast_exp2(__builtin_fmaf(sa[kt][i], c2, nba));
            suma += sa[kt][i];
            sb[kt][i] = fast_exp2(__builtin_fmaf(sb[kt][i], c2, nbb));
            sumb += sb[kt][i];
        }
    suma = colgroup_sum(suma);
    sumb = colgroup_sum(sumb);
    const float rsa = 1.f / suma, rsb = 1.f / sumb;
    u32x4 pka[NKC], pkb[NKC];
#pragma unroll
    for (int c = 0; c < NKC; ++c) {
        float pa[8], pb[8];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int kt = 2 * c + hh;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                pa[4 * hh + i] = kt < NP ? sa[kt < NP ? kt : 0][i] : 0.f;
                pb[4 * hh + i] = kt < NP ? sb[kt < NP ? kt : 0][i] : 0.f;
            }
        }
        pka[c] = u32x4{M::pack2(pa[0], pa[1]), M::pack2(pa[2], pa[3]), M::pack2(pa[4], pa[5]), M::pack2(pa[6], pa[7])};
        pkb[c] = u32x4{M::pack2(pb[0], pb[1]), M::pack2(pb[2], pb[3]), M::pack2(pb[4], pb[5]), M::pack2(pb[6], pb[7])};
    }
    f32x4 oa[4], ob[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
        f32x4 acca = f32x4{0.f, 0.f, 0.f, 0.f}, accb = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NKC; ++c) {
            const u32x4 v = u32x4{vop[dt][c][0][0], vop[dt][c][0][1], vop[dt][c][1][0], vop[dt][c][1][1]};
            acca = M::mma(v, pka[c], acca);
            accb = M::mma(v, pkb[c], accb);
        }
        oa[dt] = acca;
        ob[dt] = accb;
    }
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        outa[half] = u32x4{M::pack2(oa[2 * half][0] * rsa, oa[2 * half][1] * rsa), M::pack2(oa[2 * half][2] * rsa, oa[2 * half][3] * rsa),
                           M::pack2(oa[2 * half + 1][0] * rsa, oa[2 * half + 1][1] * rsa),
                           M::pack2(oa[2 * half + 1][2] * rsa, oa[2 * half + 1][3] * rsa)};
        outb[half] = u32x4{M::pack2(ob[2 * half][0] * rsb, ob[2 * half][1] * rsb), M::pack2(ob[2 * half][2] * rsb, ob[2 * half][3] * rsb),
                           M::pack2(ob[2 * half + 1][0] * rsb, ob[2 * half + 1][1] * rsb),
                           M::pack2(ob[2 * half + 1][2] * rsb, ob[2 * half + 1][3] * rsb)};
    }
}

// Producer p's tiles of head h (+ bias), rounded, into Q, K, V of the slot:
// Q and K rows below L, V rows below L and zeros for rows L .. 16 NP - 1.
template <typename T, int NP>
__device__ __forceinline__ void ws_store(const f32x4 (&acc)[3][NP], lds_t* sq, lds_t* sk, lds_t* sv,
                                         const void* const (&bias)[4], int h, int p, int L, int m, int g) {
    using M = Mfma16<T>;
#pragma unroll
    for (int f = 0; f < 3; ++f) {
        f32x4 bv = f32x4{0.f, 0.f, 0.f, 0.f};  // bias of features 4g .. 4g+3 of the tile
        const T* bp = static_cast<const T*>(bias[f]);
        if (bp) {
            const int feat = h * kD + p * 16 + 4 * g;
#pragma unroll
            for (int i = 0; i < 4; ++i) bv[i] = static_cast<float>(bp[feat + i]);
        }
        lds_t* const dst = f == 0 ? sq : (f == 1 ? sk : sv);
#pragma unroll
        for (int pt = 0; pt < NP; ++pt) {
            const int row = pt * 16 + m;
            const u32x2 v = u32x2{M::pack2(acc[f][pt][0] + bv[0], acc[f][pt][1] + bv[1]),
                                  M::pack2(acc[f][pt][2] + bv[2], acc[f][pt][3] + bv[3])};
            if (row < L)
                lds_st8(dst + xquad<kD>(row, p * 16 + 4 * g), v);
            else if (f == 2)
                lds_st8(dst + xquad<kD>(row, p * 16 + 4 * g), u32x2{0u, 0u});
        }
    }
}

// 16-bit pair w (as the layer rounded it) + residual pair r, rounded again:
// x + attn(...) of transformer.py:143 in the 16-bit type.
template <typename T>
__device__ inline uint32_t add_res2(uint32_t w, uint32_t r) {
    using M = Mfma16<T>;
    return M::pack2(M::to_float((uint16_t)(w & 0xffffu)) + M::to_float((uint16_t)(r & 0xffffu)),
                    M::to_float((uint16_t)(w >> 16)) + M::to_float((uint16_t)(r >> 16)));
}

// Y feature tiles ft0 .. ft0 + FT - 1 (+ bias) of sample b, rounded once (and,
// with RES, added to x and rounded again); rows past L are dropped.
// In the MFMA layout a lane holds 4 consecutive features (8 bytes) of one row
// per tile.  For each pair of tiles, two lane swaps across the 16-lane groups
// (pairing groups 0,1 with 2,3, then 0 with 1 and 2 with 3) leave lane group
// g with features 8g .. 8g + 7 of the pair's 32, so each store writes 16
// bytes per lane and 64 contiguous bytes per row: half the store
// instructions and write requests of 8-byte stores.  With RES the residual
// pieces of x the stores cover are loaded one pair of tiles at a time, the
// next pair's in flight while the current pair is stored (all at once they
// would not fit in registers beside the accumulators).
template <typename T, int FT, int NP, bool RES>
__device__ __forceinline__ void ws_store_y(const f32x4 (&yacc)[FT][NP], const MhaArgs& a, int b, int ft0, int m, int g) {
    using M = Mfma16<T>;
    const int L = a.L;
    const rsrc_t ry = make_rsrc(static_cast<const T*>(a.y) + b * a.ysb, (uint32_t)(((L - 1) * a.yss + kWsE) * 2));
    const rsrc_t rx = make_rsrc(static_cast<const T*>(a.x) + b * a.xsb, (uint32_t)(((L - 1) * a.xss + kWsE) * 2));
    const T* const bo = static_cast<const T*>(a.bias[3]);
    constexpr int NPAIR = FT / 2;
    // Residual pieces of pair fp, position tile q: the 16 bytes a lane stores.
    const auto res_ld = [&](int fp, int q) {
        return buf_ld16_keep(rx, (uint32_t)((q * 16 + m) * a.xss + (ft0 + 2 * fp) * 16 + 8 * g) * 2);
    };
    u32x4 rcur[NP], rnext[NP];
    if constexpr (RES && NPAIR > 0)
#pragma unroll
        for (int q = 0; q < NP; ++q) rcur[q] = res_ld(0, q);
    // Bias of features 16 (ft0 + f) + 4g .. + 3, read before any store (a
    // wait for the loads would otherwise wait for the stores too).
    f32x4 bv[FT];
#pragma unroll
    for (int f = 0; f < FT; ++f) {
        bv[f] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (bo)
#pragma unroll
            for (int i = 0; i < 4; ++i) bv[f][i] = static_cast<float>(bo[(ft0 + f) * 16 + 4 * g + i]);
    }
#pragma unroll
    for (int fp = 0; fp < NPAIR; ++fp) {
        if constexpr (RES)
            if (fp + 1 < NPAIR)
#pragma unroll
                for (int q = 0; q < NP; ++q) rnext[q] = res_ld(fp + 1, q);
#pragma unroll
        for (int q = 0; q < NP; ++q) {
            const f32x4& ya = yacc[2 * fp][q];
            const f32x4& yb = yacc[2 * fp + 1][q];
            const f32x4& ba = bv[2 * fp];
            const f32x4& bb = bv[2 * fp + 1];
            uint32_t x0 = M::pack2(ya[0] + ba[0], ya[1] + ba[1]), x1 = M::pack2(ya[2] + ba[2], ya[3] + ba[3]);
            uint32_t y0 = M::pack2(yb[0] + bb[0], yb[1] + bb[1]), y1 = M::pack2(yb[2] + bb[2], yb[3] + bb[3]);
            lane_swap32(x0, y0);
            lane_swap32(x1, y1);
            lane_swap16(x0, y0);
            lane_swap16(x1, y1);
            u32x4 out = u32x4{x0, x1, y0, y1};
            if constexpr (RES)
#pragma unroll
                for (int i = 0; i < 4; ++i) out[i] = add_res2<T>(out[i], rcur[q][i]);
            buf_st16_cached(ry, (uint32_t)((q * 16 + m) * a.yss + (ft0 + 2 * fp) * 16 + 8 * g) * 2, out);
        }
        if constexpr (RES)
            if (fp + 1 < NPAIR)
#pragma unroll
                for (int q = 0; q < NP; ++q) rcur[q] = rnext[q];
    }
    if constexpr (FT % 2 == 1) {  // an odd last tile: 8 bytes per lane
        u32x2 rodd[NP];
        if constexpr (RES)
#pragma unroll
            for (int q = 0; q < NP; ++q)
                rodd[q] = __builtin_amdgcn_raw_buffer_load_b64(rx, (int)((q * 16 + m) * a.xss + (ft0 + FT - 1) * 16 + 4 * g) * 2, 0, 0);
#pragma unroll
        for (int q = 0; q < NP; ++q) {
            const f32x4& y = yacc[FT - 1][q];
            const f32x4& bb = bv[FT - 1];
            u32x2 out = u32x2{M::pack2(y[0] + bb[0], y[1] + bb[1]), M::pack2(y[2] + bb[2], y[3] + bb[3])};
            if constexpr (RES)
#pragma unroll
                for (int i = 0; i < 2; ++i) out[i] = add_res2<T>(out[i], rodd[q][i]);
            buf_st8_cached(ry, (uint32_t)((q * 16 + m) * a.yss + (ft0 + FT - 1) * 16 + 4 * g) * 2, out);
        }
    }
}

// X rows of sample b into LDS (swizzled), by NTHR threads (thread index t).
template <typename T, int NP, int NTHR>
__device__ __forceinline__ void ws_load_x(lds_t* sx, const MhaArgs& a, int b, int t) {
    constexpr int XC = kWsE / 8;
    constexpr int U = (NP * 16 * XC + NTHR - 1) / NTHR;
    // Opaque copies: called inside the sample loop, the per-pass offsets
    // would otherwise be hoisted out of it and held (or spilled) throughout.
    const int L = opaque_s(a.L);
    t = opaque_v(t);
    const int N = L * XC;
    const rsrc_t rx = make_rsrc(static_cast<const T*>(a.x) + b * a.xsb, (uint32_t)(((L - 1) * a.xss + kWsE) * 2));
    u32x4 v[U];
    // Whole passes are uniform branches; only the last pass tests its lanes.
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int idx = u * NTHR + t;
        const int r = idx / XC, c = idx - (idx / XC) * XC;
        if (u * NTHR < N) v[u] = buf_ld16(rx, idx < N ? (uint32_t)(r * a.xss + c * 8) * 2 : 0xfffffff0u);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int idx = u * NTHR + t;
        const int r = idx / XC, c = idx - (idx / XC) * XC;
        if (u * NTHR + NTHR <= N)
            lds_st16(sx + eoff<kWsE>(r, c), v[u]);
        else if (u * NTHR < N && idx < N)
            lds_st16(sx + eoff<kWsE>(r, c), v[u]);
    }
}

// The next sample's X rows in two halves for the producers: the loads go out
// right after the last head's projection MFMAs, into registers, and land in
// LDS a step later, once every producer is done reading the current X.
// Producer p takes rows p, p + 4, p + 8, ... (whole rows, so that it can
// normalise them itself right after writing them); kWsXU loads per lane
// cover the longest sequence the kernel takes (kWsMaxL rows).
constexpr int kWsMaxL = 101;
#ifndef ATX_MHA_WS_XEARLY
#define ATX_MHA_WS_XEARLY 8
#endif
constexpr int kWsXEarly = ATX_MHA_WS_XEARLY;  // loads issued before the last head's store
template <int NP>
constexpr int ws_xu() {
    return (((16 * NP < kWsMaxL ? 16 * NP : kWsMaxL) + 3) / 4 * (kWsE / 8) + 63) / 64;
}
template <typename T, int UX, int U0, int U1>
__device__ __forceinline__ void ws_x_issue(u32x4 (&v)[UX], const MhaArgs& a, int b, int p, int lane) {
    constexpr int XC = kWsE / 8;
    const int L = opaque_s(a.L);
    lane = opaque_v(lane);
    const rsrc_t rx = make_rsrc(static_cast<const T*>(a.x) + b * a.xsb, (uint32_t)(((L - 1) * a.xss + kWsE) * 2));
    // No branches (a load past the rows reads zero): registers defined on
    // every path stay in registers across the code between issue and commit.
#pragma unroll
    for (int u = U0; u < U1; ++u) {
        const int j = u * 64 + lane;
        const int r = p + 4 * (j / XC), c = j - (j / XC) * XC;
        v[u] = buf_ld16(rx, r < L ? (uint32_t)(r * a.xss + c * 8) * 2 : 0xfffffff0u);
    }
}
template <int UX>
__device__ __forceinline__ void ws_x_commit(const u32x4 (&v)[UX], lds_t* sx, int L, int p, int lane) {
    constexpr int XC = kWsE / 8;
    L = opaque_s(L);
    lane = opaque_v(lane);
#pragma unroll
    for (int u = 0; u < UX; ++u) {
        const int j = u * 64 + lane;
        const int r = p + 4 * (j / XC), c = j - (j / XC) * XC;
        if (r < L) lds_st16(sx + eoff<kWsE>(r, c), v[u]);
    }
}

// Pre-LN of transformer.py:143 (nn.LayerNorm(embed_dim)) on X rows r0,
// r0 + rstep, ... below L, in place in LDS, by one wave: per row the fp32
// mean and biased variance over the E elements, (x - mean) * rsqrt(var +
// eps) * weight + bias, rounded to T.  Four rows per pass: lanes 16k .. 16k +
// 15 hold row r0 + rstep (4 pass + k), lane i its 16-byte chunks i, i + 16,
// i + 32; row sums over the 16 lanes by DPP butterflies.
template <typename T>
__device__ __forceinline__ void ws_layernorm_rows(lds_t* sx, const MhaArgs& a, int r0, int rstep, int lane) {
    using M = Mfma16<T>;
    constexpr int XC = kWsE / 8;
    constexpr int CPL = XC / 16;  // chunks per lane
    const int L = opaque_s(a.L);
    lane = opaque_v(lane);
    const int k = lane >> 4, i = lane & 15;
    const rsrc_t rg = make_rsrc(a.ln_w, kWsE * 2), rb = make_rsrc(a.ln_b, a.ln_b ? kWsE * 2 : 0);
    u32x4 gw[CPL], gb[CPL];  // this lane's columns of weight and bias (a NULL bias reads zeros)
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        gw[j] = buf_ld16_keep(rg, (uint32_t)(i + 16 * j) * 16);
        gb[j] = buf_ld16_keep(rb, (uint32_t)(i + 16 * j) * 16);
    }
    const auto lo = [](uint32_t w) { return M::to_float((uint16_t)(w & 0xffffu)); };
    const auto hi = [](uint32_t w) { return M::to_float((uint16_t)(w >> 16)); };
    const float inv_e = 1.f / (float)kWsE;
    for (int base = r0; base < L; base += 4 * rstep) {
        const int r = base + rstep * k;
        const bool ok = r < L;
        float xv[CPL][8];
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const u32x4 c = ok ? lds_ld16(sx + eoff<kWsE>(r, i + 16 * j)) : u32x4{0, 0, 0, 0};
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                xv[j][2 * w] = lo(c[w]);
                xv[j][2 * w + 1] = hi(c[w]);
            }
        }
        float sum = 0.f;
#pragma unroll
        for (int j = 0; j < CPL; ++j)
#pragma unroll
            for (int e = 0; e < 8; ++e) sum += xv[j][e];
        sum = row16_sum(sum);
        const float mean = sum * inv_e;
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < CPL; ++j)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                xv[j][e] -= mean;
                ss = __builtin_fmaf(xv[j][e], xv[j][e], ss);
            }
        ss = row16_sum(ss);
        const float rstd = __builtin_amdgcn_rsqf(ss * inv_e + a.ln_eps);
        if (ok)
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                u32x4 c;
#pragma unroll
                for (int w = 0; w < 4; ++w)
                    c[w] = M::pack2(__builtin_fmaf(xv[j][2 * w] * rstd, lo(gw[j][w]), lo(gb[j][w])),
                                    __builtin_fmaf(xv[j][2 * w + 1] * rstd, hi(gw[j][w]), hi(gb[j][w])));
                lds_st16(sx + eoff<kWsE>(r, i + 16 * j), c);
            }
    }
}

// Y^T += Wo[:, 64h ..] O_h^T for Y feature tiles ft0 .. ft0 + FT - 1: the Wo
// operands of head h (two k-steps), loaded one step ahead of their use.
template <int FT, bool PK>
__device__ __forceinline__ void ws_load_wo(u32x4 (&wo)[2][FT], rsrc_t rwo, int ft0, int m, int g, int h) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int f = 0; f < FT; ++f)
            wo[j][f] = buf_ld16_keep(rwo, wtile_off<kWsE, PK>(ft0 + f, m, g) + (uint32_t)(2 * h + j) * kWStep<PK>);
}

struct WsCtx {
    lds_t* sx0;  // X
    lds_t* ss0;  // slot 0 (slot 1 follows at +slot)
    lds_t* sync; // progress counters (after slot 1)
    int slot;    // bytes per slot
    int LQ;      // Q / K rows per slot
    int lane;
    int batch;
};

// ---------------------------------------------------------------------------
// The two roles.  Heads are numbered t = 6 i + s over the workgroup's samples
// i; head t uses slot t & 1.  What each wait protects:
//  * a producer stores head t into slot t & 1 once all eight waves have
//    out-projected head t - 2 from it (which each does only after every
//    consumer has attended head t - 2 there);
//  * a consumer attends head t once every producer has stored it;
//  * every wave out-projects head h once every consumer has attended it;
//  * a producer overwrites X with the next sample's rows once every producer
//    has projected the last head from it, and projects the next sample once
//    every producer has written (and normalised) its rows.
// Producers out-project head t - 2 before projecting head t, consumers head
// t - 1 right after attending it; consumers never read X.
template <typename T, int NP, bool PK, bool RES>
__device__ __forceinline__ void ws_producer(const WsCtx& c, const MhaArgs& a, const rsrc_t (&rw)[4], int p) {
    constexpr int FT = ws_ftp<RES, PK>();
    const int ft0 = FT * p;
    const int grid = gridDim.x;
    f32x4 yacc[FT][NP];
#pragma unroll
    for (int f = 0; f < FT; ++f)
#pragma unroll
        for (int q = 0; q < NP; ++q) yacc[f][q] = f32x4{0.f, 0.f, 0.f, 0.f};
    u32x4 wo[2][FT];
    // Out-projection of head t - 2 (at s = 1 the previous sample's last head,
    // then that sample's Y).
    const auto out_proj = [&](int b, int s, uint32_t t, int m, int g) {
        ws_wait(c.sync, kSyncAttn, t - 1);
        out_proj_head<T, FT, NP>(yacc, wo, lds_opaque(c.ss0) + ((t - 2) & 1) * c.slot, m, g);
        ws_post(c.sync, kSyncOutP + p, t - 1);
        if (s == 1) {
            ws_store_y<T, FT, NP, RES>(yacc, a, b - grid, ft0, m, g);
#pragma unroll
            for (int f = 0; f < FT; ++f)
#pragma unroll
                for (int q = 0; q < NP; ++q) yacc[f][q] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    };
    // Head t into slot t & 1 once all eight waves have out-projected head t - 2.
    const auto store = [&](int s, uint32_t t, int m, int g, const f32x4 (&acc)[3][NP]) {
        if (t >= 2) ws_wait<8>(c.sync, kSyncOutP, t - 1);  // kSyncOutP and kSyncOutC
        lds_t* const sq = lds_opaque(c.ss0) + (t & 1) * c.slot;
        ws_store<T, NP>(acc, sq, sq + c.LQ * kD * 2, sq + 2 * c.LQ * kD * 2, a.bias, s, p, opaque_s(a.L), m, g);
        ws_post(c.sync, kSyncStore + p, t + 1);
    };
    uint32_t t = 0;  // head number
    uint32_t i = 0;  // sample number
    for (int b = blockIdx.x; b < c.batch; b += grid, ++i) {
        for (int s = 0; s < kWsH - 1; ++s, ++t) {
            const int ln = opaque_v(c.lane);
            const int m = ln & 15, g = ln >> 4;
            if (t >= 2) out_proj(b, s, t, m, g);
            if (s == 0 && i > 0) ws_wait(c.sync, kSyncXready, i);  // every producer's rows of this sample's X
            f32x4 acc[3][NP];
            ws_project<T, NP, PK>(lds_opaque(c.sx0), m, g, rw, wtile_off<kWsE, PK>(s * 4 + p, m, g), acc);
            // (Head t - 1's operands for the next out-projection; at t = 0
            // head 5's, which nothing uses.)
            ws_load_wo<FT, PK>(wo, rw[3], ft0, m, g, s > 0 ? s - 1 : kWsH - 1);
            store(s, t, m, g, acc);
        }
        // The last head, then the next sample's X.
        const int ln = opaque_v(c.lane);
        const int m = ln & 15, g = ln >> 4;
        const bool more = b + grid < c.batch;
        out_proj(b, kWsH - 1, t, m, g);
        u32x4 xv[ws_xu<NP>()];
        {
            f32x4 acc[3][NP];
            ws_project<T, NP, PK>(lds_opaque(c.sx0), m, g, rw, wtile_off<kWsE, PK>((kWsH - 1) * 4 + p, m, g), acc);
            ws_post(c.sync, kSyncXfree + p, i + 1);
            ws_load_wo<FT, PK>(wo, rw[3], ft0, m, g, kWsH - 2);
            // (Part of the loads here; the rest once acc is stored.  After
            // the last sample this re-reads its own X, unused: the issue
            // stays branch-free.)
            __builtin_amdgcn_sched_barrier(0);
            ws_x_issue<T, ws_xu<NP>(), 0, kWsXEarly>(xv, a, more ? b + grid : b, p, ln);
            store(kWsH - 1, t, m, g, acc);
        }
        ++t;
        __builtin_amdgcn_sched_barrier(0);
        ws_x_issue<T, ws_xu<NP>(), kWsXEarly, ws_xu<NP>()>(xv, a, more ? b + grid : b, p, ln);
        __builtin_amdgcn_sched_barrier(0);
        if (more) {
            ws_wait(c.sync, kSyncXfree, i + 1);  // every producer is done with this sample's X
            ws_x_commit<ws_xu<NP>()>(xv, lds_opaque(c.sx0), a.L, p, ln);
            if (a.ln_w) {
                wave_lds_handoff();  // the wave reads back the rows it wrote
                ws_layernorm_rows<T>(lds_opaque(c.sx0), a, p, 4, c.lane);
            }
        }
        ws_post(c.sync, kSyncXready + p, i + 1);
    }
    // Heads T - 2 and T - 1 of the last sample, then its Y.
    const int m = c.lane & 15, g = c.lane >> 4;
    const int last = blockIdx.x + ((c.batch - 1 - (int)blockIdx.x) / grid) * grid;
    ws_wait(c.sync, kSyncAttn, t - 1);
    out_proj_head<T, FT, NP>(yacc, wo, lds_opaque(c.ss0) + ((t - 2) & 1) * c.slot, m, g);
    ws_load_wo<FT, PK>(wo, rw[3], ft0, m, g, kWsH - 1);
    ws_wait(c.sync, kSyncAttn, t);
    out_proj_head<T, FT, NP>(yacc, wo, lds_opaque(c.ss0) + ((t - 1) & 1) * c.slot, m, g);
    ws_store_y<T, FT, NP, RES>(yacc, a, last, ft0, m, g);
}

// Consumer wave 4 + cq, 7 steps per sample: attention of head s - 1 at step
// s = 1 .. 6, out-projection of head s - 2 at step s and of the previous
// sample's last head (then that sample's Y) at step 0.
template <typename T, int NP, bool CAUSAL, bool PK, bool RES>
__device__ __forceinline__ void ws_consumer(const WsCtx& c, const MhaArgs& a, const rsrc_t (&rw)[4], int cq) {
    constexpr int FT = 6 - ws_ftp<RES, PK>();
    const int ft0 = 4 * ws_ftp<RES, PK>() + FT * cq;
    const int grid = gridDim.x;
    f32x4 yacc[FT][NP];
#pragma unroll
    for (int f = 0; f < FT; ++f)
#pragma unroll
        for (int q = 0; q < NP; ++q) yacc[f][q] = f32x4{0.f, 0.f, 0.f, 0.f};
    u32x4 wo[2][FT];
    uint32_t t0 = 0;  // number of this sample's head 0
    for (int b = blockIdx.x; b < c.batch; b += grid, t0 += kWsH) {
        for (int s = 0; s <= kWsH; ++s) {
            const int ln = opaque_v(c.lane);
            const int m = ln & 15, g = ln >> 4;
            if (s >= 2 || (s == 0 && t0 > 0)) {
                const uint32_t h = s >= 2 ? t0 + s - 2 : t0 - 1;  // head to out-project
                ws_wait(c.sync, kSyncAttn, h + 1);
                out_proj_head<T, FT, NP>(yacc, wo, lds_opaque(c.ss0) + (h & 1) * c.slot, m, g);
                ws_post(c.sync, kSyncOutC + cq, h + 1);
                if (s == 0) {
                    ws_store_y<T, FT, NP, RES>(yacc, a, b - grid, ft0, m, g);
#pragma unroll
                    for (int f = 0; f < FT; ++f)
#pragma unroll
                        for (int q = 0; q < NP; ++q) yacc[f][q] = f32x4{0.f, 0.f, 0.f, 0.f};
                }
            }
            if (s >= 1) {
                const uint32_t h = t0 + s - 1;  // head to attend
                ws_wait(c.sync, kSyncStore, h + 1);
                const int L = opaque_s(a.L);
                lds_t* const sq = lds_opaque(c.ss0) + (h & 1) * c.slot;
                lds_t* const sk = sq + c.LQ * kD * 2;
                lds_t* const sv = sk + c.LQ * kD * 2;
                const auto put = [&](int qt, const u32x4 (&out)[2]) {
                    if (qt * 16 + m < L)
#pragma unroll
                        for (int half = 0; half < 2; ++half) lds_st16(sq + xoff<kD>(qt * 16 + m, 2 * g + half), out[half]);
                };
                if (!CAUSAL && cq + 4 < NP) {
                    u32x4 outa[2], outb[2];
                    ws_attend_pair<T, NP>(sq, sk, sv, cq, cq + 4, L, a.c2, m, g, outa, outb);
                    put(cq, outa);
                    put(cq + 4, outb);
                } else {
#pragma unroll
                    for (int r = 0; r < 2; ++r) {
                        const int qt = cq + 4 * r;
                        if (qt < NP) {
                            u32x4 out[2];
                            ws_attend_tile<T, NP, CAUSAL>(sq, sk, sv, qt, L, a.c2, m, g, out);
                            put(qt, out);
                        }
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
                ws_post(c.sync, kSyncAttn + cq, h + 1);
            }
            ws_load_wo<FT, PK>(wo, rw[3], ft0, m, g, s > 0 ? s - 1 : 0);
        }
    }
    const int m = c.lane & 15, g = c.lane >> 4;
    const int last = blockIdx.x + ((c.batch - 1 - (int)blockIdx.x) / grid) * grid;
    ws_wait(c.sync, kSyncAttn, t0);
    out_proj_head<T, FT, NP>(yacc, wo, lds_opaque(c.ss0) + ((t0 - 1) & 1) * c.slot, m, g);
    ws_store_y<T, FT, NP, RES>(yacc, a, last, ft0, m, g);
}

// Y of every sample of this workgroup set to NaN (after a wait gave up).
template <typename T>
__device__ void ws_poison_y(const MhaArgs& a, int batch, int tid) {
    using M = Mfma16<T>;
    constexpr int YC = kWsE / 8;  // 16-byte chunks per row
    const uint32_t nan2 = M::pack2(__builtin_nanf(""), __builtin_nanf(""));
    for (int b = blockIdx.x; b < batch; b += gridDim.x) {
        const rsrc_t ry = make_rsrc(static_cast<const T*>(a.y) + b * a.ysb, (uint32_t)(((a.L - 1) * a.yss + kWsE) * 2));
        for (int idx = tid; idx < a.L * YC; idx += kThreads) {
            const int r = idx / YC, c = idx - (idx / YC) * YC;
            buf_st16_cached(ry, (uint32_t)(r * a.yss + c * 8) * 2, u32x4{nan2, nan2, nan2, nan2});
        }
    }
}

template <typename T, int NP, bool CAUSAL, bool PK, bool RES>
__global__ __launch_bounds__(kThreads) void mha_ws(MhaArgs a, int batch) {
    constexpr int E = kWsE;
    constexpr int LP = NP * 16;
    constexpr int LV = ws_lv(NP);
    static_assert(kWaves == 8, "wave roles assume 8 waves");
    static_assert(E / 16 == 24, "Y tiles split over the waves: 4 producers and 4 consumers, 6 per pair");

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    WsCtx c;
    c.lane = tid & 63;
    c.batch = batch;
    c.LQ = ws_lq(a.L);
    c.slot = (2 * c.LQ + LV) * kD * 2;
    c.sx0 = lds_base();
    c.ss0 = c.sx0 + a.L * E * 2;
    c.sync = c.ss0 + 2 * c.slot;
    if (tid < kSyncWords) lds_st4(c.sync + 4 * tid, tid == kSyncSpin ? (uint32_t)a.ws_spin : 0u);  // (visible after the first barrier)

    rsrc_t rw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) rw[i] = make_rsrc(a.w[i], (uint32_t)(E * E * 2));

    // ---- first sample's X; V rows past 16 NP of both slots zeroed once -------------
    ws_load_x<T, NP, kThreads>(c.sx0, a, blockIdx.x, tid);
    for (int idx = tid; idx < 2 * (LV - LP) * 8; idx += kThreads) {
        const int s = idx / ((LV - LP) * 8), j = idx - s * ((LV - LP) * 8);
        lds_st16(c.ss0 + s * c.slot + 2 * c.LQ * kD * 2 + LP * kD * 2 + j * 16, u32x4{0, 0, 0, 0});
    }
    __syncthreads();
    if (a.ln_w) {  // (uniform: the same for every wave)
        ws_layernorm_rows<T>(c.sx0, a, wave, kWaves, c.lane);
        __syncthreads();
    }

    // The two roles run separate loops (the branch is uniform over each
    // wave), each with its own registers; after the prologue's barriers they
    // meet only through the progress counters.
    if (wave < 4)
        ws_producer<T, NP, PK, RES>(c, a, rw, wave);
    else
        ws_consumer<T, NP, CAUSAL, PK, RES>(c, a, rw, wave - 4);
    // Every wave's Y stores complete before any poison store is issued.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (__builtin_amdgcn_readfirstlane(lds_ld4(c.sync + 4 * kSyncAbort)) != 0) ws_poison_y<T>(a, batch, tid);
}

template <typename K>
int launch_ws(K kernel, int grid, int batch, size_t lds, hipStream_t st, const MhaArgs& a) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) ATX_FAIL(ATX_ERR_LAUNCH, "hipFuncSetAttribute(%zu bytes LDS): %s", lds, hipGetErrorString(e));
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kThreads), lds, st, a, batch);
    ATX_CHECK_LAUNCH("atx_mha_fwd (persistent form) launch");
    return ATX_OK;
}

template <typename T, bool CAUSAL, bool PK, bool RES>
int ws_np_res(int np, int grid, int batch, size_t lds, hipStream_t st, const MhaArgs& a) {
    switch (np) {
        case 5: return launch_ws(mha_ws<T, 5, CAUSAL, PK, RES>, grid, batch, lds, st, a);
        case 6: return launch_ws(mha_ws<T, 6, CAUSAL, PK, RES>, grid, batch, lds, st, a);
        case 7: return launch_ws(mha_ws<T, 7, CAUSAL, PK, RES>, grid, batch, lds, st, a);
        default: ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_mha_fwd (persistent form): %d position tiles", np);
    }
}

// (The residual add is a template parameter: its loads would otherwise take
// registers in the kernels without it.)
template <typename T, bool CAUSAL, bool PK>
int ws_np(int np, int grid, int batch, size_t lds, hipStream_t st, const MhaArgs& a) {
    return a.residual ? ws_np_res<T, CAUSAL, PK, true>(np, grid, batch, lds, st, a)
                      : ws_np_res<T, CAUSAL, PK, false>(np, grid, batch, lds, st, a);
}

constexpr int kMaxDevices = 64;
std::mutex g_cu_mu;
int g_cu_count[kMaxDevices] = {};

// Compute units of the current device (looked up once per device).
int cu_count(int* out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) ATX_FAIL(ATX_ERR_LAUNCH, "atx_mha_fwd: hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_mha_fwd: device %d (at most %d devices)", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_cu_mu);
    if (!g_cu_count[dev]) {
        int n = 0;
        e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess || n < 1)
            ATX_FAIL(ATX_ERR_LAUNCH, "atx_mha_fwd: compute-unit count of device %d: %s", dev, hipGetErrorString(e));
        g_cu_count[dev] = n;
    }
    *out = g_cu_count[dev];
    return ATX_OK;
}

}  // namespace

size_t mha_ws_lds_bytes(int E, int L) {
    if (E != kWsE || L < 65 || L > kWsMaxL) return 0;
    const size_t lds = ws_lds(L);
    return lds <= 160 * 1024 ? lds : 0;
}

int mha_ws_launch(int L, bool causal, bool bf16, bool packed, int batch, size_t lds, hipStream_t st, const MhaArgs& args) {
    MhaArgs a = args;
    a.ws_spin = (int)kWsSpin;
    if (const char* env = getenv("ATX_MHA_WS_SPIN")) {  // tests: force the give-up path
        const long v = strtol(env, nullptr, 10);
        if (v >= 1 && v < (long)kWsSpin) a.ws_spin = (int)v;
    }
    int ncu = 0;
    if (const int rc = cu_count(&ncu)) return rc;
    const int grid = batch < ncu ? batch : ncu;
    const int np = (L + 15) / 16;
    if (packed) {
        if (bf16) return causal ? ws_np<__bf16, true, true>(np, grid, batch, lds, st, a) : ws_np<__bf16, false, true>(np, grid, batch, lds, st, a);
        return causal ? ws_np<_Float16, true, true>(np, grid, batch, lds, st, a) : ws_np<_Float16, false, true>(np, grid, batch, lds, st, a);
    }
    if (bf16) return causal ? ws_np<__bf16, true, false>(np, grid, batch, lds, st, a) : ws_np<__bf16, false, false>(np, grid, batch, lds, st, a);
    return causal ? ws_np<_Float16, true, false>(np, grid, batch, lds, st, a) : ws_np<_Float16, false, false>(np, grid, batch, lds, st, a);
}

}  // namespace atx
