// Policy-head backward (atx_kq_bwd): the arguments and the first phase --
// the gradient of the masked logits, dL -- shared by the 16-bit kernel
// (atx_kq_bwd.hip) and the fp32 one (atx_kq_bwd_fp32.hip).
#pragma once

#include "ataraxos_attn.h"
#include "atx_common.hpp"

namespace atx {

struct KqBwdArgs {
    const void* q;
    const void* k;
    int64_t qsb, ksb;
    int qss, kss;  // row strides (elements)
    const uint8_t* mask;
    int64_t msb;
    int mss;
    const float* grad;
    int64_t gsb;
    const float* probs;
    int64_t psb;
    void* dq;
    void* dk;
    int64_t dqsb, dksb;
    int dqss, dkss;
    int S;
    int Dfull;      // q / k / dq / dk row width
    int nd;         // column slices of D (the template width) in Dfull
    float scale;
    int mask_al4;   // mask base and strides are multiples of 4 bytes
    int grad_vec;   // S % 4 == 0 and every G / P row starts 16-byte aligned
};

constexpr int kKqBwdThreads = 512;
constexpr int kKqBwdWaves = 8;

// dL of sample b, streamed from G (and P) with the legality bytes: for every
// 8-entry piece (row i, columns 8c .. 8c + 7) of the [RP x RP] matrix, zero
// past the sample, calls store(i, c, dl) once.  PROBS: dL = P (G - sum G P),
// the sum reduced per wave and then over the waves in a fixed order through
// `sred` (kKqBwdWaves floats of LDS); otherwise dL = G; illegal entries 0.
//
// Logits with G rows that are not 16-byte aligned (S % 4 != 0, as at the
// reference Move head's 101 squares), S <= 110 and contiguous mask rows:
// the sample's S * S entries are read flat instead, in groups of 4 per lane
// (one 4-byte mask word, one 16-byte or four 4-byte G loads), after every
// piece has been zeroed, and each entry goes to LDS through store1(i, j,
// value).  (The piece path would issue 8 scattered 4-byte G loads and 8
// byte loads of the mask per piece; byte loads are the costly part.)
//
// The probabilities gradient takes the flat path too when `scratch` (LDS
// that is free during this phase, `scratch_bytes` of it) holds the sample's
// S * S products G P as floats: they are written there flat and summed per
// 8-entry piece in the piece path's (row, column) order, so the sum depends
// on the sample's data only, not on where its rows start.
template <int RP, bool PROBS, typename Store, typename Store1>
__device__ __forceinline__ void kq_bwd_dl(const KqBwdArgs& a, int b, lds_t* sred, Store store, Store1 store1,
                                          lds_t* scratch, int scratch_bytes) {
    constexpr int kThreads = kKqBwdThreads, kWaves = kKqBwdWaves;
    constexpr uint32_t kOut = 0xfffffff0u;
    constexpr int GC = RP / 8;  // 8-entry pieces per dL row
    constexpr int PERT = (RP * GC + kThreads - 1) / kThreads;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int S = a.S;
    const rsrc_t rg = make_rsrc(a.grad + b * a.gsb, (uint32_t)(S * S * 4));
    const rsrc_t rp = make_rsrc(PROBS ? a.probs + b * a.psb : a.grad, PROBS ? (uint32_t)(S * S * 4) : 0u);
    const uint8_t* const mrow0 = a.mask ? a.mask + b * a.msb : nullptr;
    const rsrc_t rm = make_rsrc(mrow0 ? mrow0 : a.mask, mrow0 ? (uint32_t)((S - 1) * a.mss + S) : 0u);

    constexpr int FG = 6;  // 4-entry groups per thread of the flat path: S <= 110
    if (!a.grad_vec && S * S + 3 <= FG * 4 * kThreads && (!mrow0 || a.mss == S) &&
        (!PROBS || S * S * 4 <= scratch_bytes)) {
        const int n = S * S;
        // Group k holds entries e = 4k - sh .. 4k - sh + 3 (those in [0, n)),
        // sh the mask's byte misalignment: the group's 4 mask bytes are one
        // 4-byte-aligned word.  Its G entries are one 16-byte-aligned load
        // when the G and mask bases agree (contiguous tensors do), else four
        // 4-byte loads.  The two partial groups at the ends load bytes.
        // (without a mask, sh aligns the G groups instead)
        const uintptr_t gbase = (uintptr_t)(a.grad + b * a.gsb);
        const int sh = mrow0 ? (int)((uintptr_t)mrow0 & 3) : (int)((gbase >> 2) & 3);
        const bool g16 = ((gbase - 4 * sh) & 15) == 0;  // (uniform)
        const bool p16 = PROBS && (((uintptr_t)(a.probs + b * a.psb) - 4 * sh) & 15) == 0;
        f32x4 gv[FG], pv[PROBS ? FG : 1];
        uint32_t mw[FG];
#pragma unroll
        for (int u = 0; u < FG; ++u) {
            const int off = 4 * (tid + u * kThreads) - sh;  // first entry of the group
            const bool full = off >= 0 && off + 4 <= n;
            if (g16) {
                gv[u] = as_f32x4(buf_ld16(rg, full ? (uint32_t)off * 4 : kOut));
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    gv[u][r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rg, full ? (off + r) * 4 : (int)kOut, 0, 0));
            }
            if constexpr (PROBS) {
                if (p16) {
                    pv[u] = as_f32x4(buf_ld16(rp, full ? (uint32_t)off * 4 : kOut));
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        pv[u][r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rp, full ? (off + r) * 4 : (int)kOut, 0, 0));
                }
            }
            mw[u] = !mrow0 ? 0x01010101u : __builtin_amdgcn_raw_buffer_load_b32(rm, full ? off : (int)kOut, 0, 0);
            if (!full && off + 4 > 0 && off < n) {  // a partial group (two lanes of the workgroup)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const bool in = off + r >= 0 && off + r < n;
                    gv[u][r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rg, in ? (off + r) * 4 : (int)kOut, 0, 0));
                    if constexpr (PROBS)
                        pv[u][r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rp, in ? (off + r) * 4 : (int)kOut, 0, 0));
                    if (mrow0) mw[u] |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rm, in ? off + r : (int)kOut, 0, 0) << (8 * r);
                }
            }
        }
        float sigma = 0.f;
        if constexpr (PROBS) {
            // G P of every entry, flat, then summed per piece in row order
#pragma unroll
            for (int u = 0; u < FG; ++u)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int e = 4 * (tid + u * kThreads) - sh + r;
                    if (e >= 0 && e < n) lds_st4(scratch + e * 4, __builtin_bit_cast(uint32_t, gv[u][r] * pv[u][r]));
                }
            __syncthreads();
            float part = 0.f;
#pragma unroll
            for (int u = 0; u < PERT; ++u) {
                const int idx = tid + u * kThreads;
                const int i = idx / GC, j0 = (idx - (idx / GC) * GC) * 8;
                if (idx < RP * GC && i < S && j0 < S)
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (j0 + e < S) part += __builtin_bit_cast(float, lds_ld4(scratch + (i * S + j0 + e) * 4));
            }
#pragma unroll
            for (int x = 32; x >= 1; x >>= 1) part += shfl_xor(part, x);
            if (lane == 0) lds_st4(sred + wave * 4, __builtin_bit_cast(uint32_t, part));
            __syncthreads();  // (also: every wave is done reading the scratch)
#pragma unroll
            for (int w = 0; w < kWaves; ++w) sigma += __builtin_bit_cast(float, lds_ld4(sred + w * 4));
        }
        const float zero8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < PERT; ++u) {
            const int idx = tid + u * kThreads;
            if (idx < RP * GC) store(idx / GC, idx - (idx / GC) * GC, zero8);
        }
        __syncthreads();  // the zeros land before the entries
#pragma unroll
        for (int u = 0; u < FG; ++u) {
            int e = 4 * (tid + u * kThreads) - sh;
            if (e >= n) break;  // (this and every later group of the thread)
            int i = 0, j = e;  // e < 0 (the first group): j reaches 0 at e = 0
            if (e >= 0) {
                i = e / S;
                j = e - i * S;
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (e >= 0 && e < n) {
                    const float x = PROBS ? pv[u][r] * (gv[u][r] - sigma) : gv[u][r];
                    store1(i, j, ((mw[u] >> (8 * r)) & 0xffu) != 0u ? x : 0.f);
                }
                ++e;
                if (++j == S) {
                    j = 0;
                    ++i;
                }
            }
        }
        return;
    }

    // ---- phase 1: dL into LDS -------------------------------------------------
    // Thread t handles dL chunks t, t + 512, ...: row i = idx / GC, columns
    // j = 8 * (idx % GC) .. + 7.
    float gv[PERT][8], pv[PROBS ? PERT : 1][8];
    uint32_t legal[PERT];  // bit e: entry j0 + e is legal and inside the sample
    float part = 0.f;
#pragma unroll
    for (int u = 0; u < PERT; ++u) {
        const int idx = tid + u * kThreads;
        const int i = idx / GC, j0 = (idx - (idx / GC) * GC) * 8;
        const bool live = idx < RP * GC && i < S && j0 < S;
        // G (and P) values
        if (a.grad_vec) {
            const uint32_t off = live ? (uint32_t)(i * S + j0) * 4 : kOut;
            // j0 + 4 < S or the second half starts the next row: not loaded
            const uint32_t off2 = live && j0 + 4 < S ? off + 16 : kOut;
            const f32x4 g0 = as_f32x4(buf_ld16(rg, off)), g1 = as_f32x4(buf_ld16(rg, off2));
#pragma unroll
            for (int e = 0; e < 4; ++e) gv[u][e] = g0[e], gv[u][4 + e] = g1[e];
            if constexpr (PROBS) {
                const f32x4 p0 = as_f32x4(buf_ld16(rp, off)), p1 = as_f32x4(buf_ld16(rp, off2));
#pragma unroll
                for (int e = 0; e < 4; ++e) pv[u][e] = p0[e], pv[u][4 + e] = p1[e];
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t off = live && j0 + e < S ? (uint32_t)(i * S + j0 + e) * 4 : kOut;
                gv[u][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rg, (int)off, 0, 0));
                if constexpr (PROBS)
                    pv[u][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rp, (int)off, 0, 0));
            }
        }
        // legality bits
        uint32_t lb = 0;
        if (live) {
            const int nin = min(S - j0, 8);
            const uint32_t in_bits = (1u << nin) - 1u;
            if (!mrow0) {
                lb = in_bits;
            } else if (a.mask_al4) {
                const uint32_t moff = (uint32_t)(i * a.mss + j0);
                uint32_t w[2];
#pragma unroll
                for (int d = 0; d < 2; ++d) {
                    if (j0 + 4 * d + 4 <= S) {
                        w[d] = __builtin_amdgcn_raw_buffer_load_b32(rm, (int)(moff + 4 * d), 0, 0);
                    } else {
                        w[d] = 0;
                        for (int e = 0; j0 + 4 * d + e < S; ++e)
                            w[d] |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rm, (int)(moff + 4 * d + e), 0, 0) << (8 * e);
                    }
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) lb |= (((w[e >> 2] >> (8 * (e & 3))) & 0xffu) != 0 ? 1u : 0u) << e;
                lb &= in_bits;
            } else {
                for (int e = 0; e < nin; ++e)
                    lb |= (__builtin_amdgcn_raw_buffer_load_b8(rm, (int)(i * a.mss + j0 + e), 0, 0) != 0 ? 1u : 0u) << e;
            }
        }
        legal[u] = lb;
        if constexpr (PROBS) {
#pragma unroll
            for (int e = 0; e < 8; ++e) part = __builtin_fmaf(gv[u][e], pv[u][e], part);
        }
    }
    float sigma = 0.f;
    if constexpr (PROBS) {
        // sum(G * P) over the sample: per wave, then the 8 wave sums in order
#pragma unroll
        for (int x = 32; x >= 1; x >>= 1) part += shfl_xor(part, x);
        if (lane == 0) lds_st4(sred + wave * 4, __builtin_bit_cast(uint32_t, part));
        __syncthreads();
#pragma unroll
        for (int w = 0; w < kWaves; ++w) sigma += __builtin_bit_cast(float, lds_ld4(sred + w * 4));
    }
#pragma unroll
    for (int u = 0; u < PERT; ++u) {
        const int idx = tid + u * kThreads;
        if (idx >= RP * GC) break;
        const int i = idx / GC, c = idx - (idx / GC) * GC;
        float dl[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float x = PROBS ? pv[u][e] * (gv[u][e] - sigma) : gv[u][e];
            dl[e] = ((legal[u] >> e) & 1u) ? x : 0.f;
        }
        store(i, c, dl);
    }
}

// LDS of the fp32 kernel and its launcher (atx_kq_bwd_fp32.hip).
// rp: squares staged (64, 96 or 128; 112 with 16-column slices).
size_t kq_bwd_fp32_lds_bytes(int dslice, int rp);
int dispatch_kq_bwd_fp32(bool probs, int dslice, int rp, int grid, size_t lds, hipStream_t st, const KqBwdArgs& a);

}  // namespace atx
