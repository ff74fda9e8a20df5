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
#include "ataraxos_attn.h"
#include "atx_common.hpp"

namespace atx {

struct BwdArgs {
    const void* q;
    const void* k;
    const void* v;
    const void* o;
    const void* dout;
    void* dq;
    void* dk;
    void* dv;
    int64_t qsb, qsh, ksb, ksh, vsb, vsh, osb, osh, dosb, dosh, dqsb, dqsh, dksb, dksh, dvsb, dvsh;
    int qss, kss, vss, oss, doss, dqss, dkss, dvss;  // sequence strides (elements)
    const uint8_t* kpad;
    int64_t kpsb;
    int H, Sq, Skv;
    float c2, scale;  // c2 = scale * log2(e)
    int causal;
};

namespace {

constexpr int kThreads = 512;
constexpr int kWaves = 8;

// Row layout shared by every staged matrix.  At D = 64 / 128 the 16-byte
// chunk c of row r sits at c ^ ((r >> 1) & 7): the 16 rows of an MFMA operand
// read and the 4 rows x 4 column groups of a transposing read both fall in
// distinct bank groups.  Other D pad rows to an odd number of 16-byte units.
template <int D>
constexpr bool kSwz = (D == 64 || D == 128);
template <int D>
constexpr int row_bytes() {
    return kSwz<D> ? D * 2 : D * 2 + 16;
}
// Row r, 16-byte chunk c.  The swizzle depends on r mod 16 only, so tile
// offsets (multiples of 16 rows) add on.
template <int D>
__device__ inline int chunk_off(int r, int c) {
    return r * row_bytes<D>() + (kSwz<D> ? (c ^ ((r >> 1) & 7)) : c) * 16;
}
// Row r, elements e .. e+3 (e a multiple of 4): one 8-byte unit.
template <int D>
__device__ inline int quad_off(int r, int e) {
    return chunk_off<D>(r, e >> 3) + (e & 7) * 2;
}

}  // namespace

// Bytes of LDS for one workgroup: K, V (rk rows), Q, dO (rq rows), and the
// log-sum-exp and delta of rq queries.
inline size_t bwd_lds_bytes(int D, int rk, int rq) {
    const int rs = (D == 64 || D == 128) ? D * 2 : D * 2 + 16;
    return (size_t)(2 * rk + 2 * rq) * rs + (size_t)rq * 8;
}

// Waves per SIMD the register allocator is asked to fit: 4 lets two
// 8-wave workgroups share a CU (128 VGPRs each), which the C3 shape's LDS
// (66.5 KiB) allows; longer sequences keep more scores per lane.
template <int D, int NKC>
constexpr int bwd_occ() {
    return (NKC <= 4 && D <= 64) ? 4 : 2;
}

// NKC = 32-key chunks (S_kv <= 32 * NKC).
template <typename T, int D, int NKC>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(bwd_occ<D, NKC>(), 8)))
void attn_bwd_16bit(BwdArgs a) {
    using M = Mfma16<T>;
    constexpr int CH = D / 8;          // 16-byte chunks per row
    constexpr int NI = (D + 31) / 32;  // MFMAs per 16x16 score tile
    constexpr int NDT = D / 16;        // head-dim output tiles
    constexpr int QD = D / 4;          // contiguous outputs per lane
    constexpr int NKT = 2 * NKC;       // key tiles
    constexpr int RK = NKT * 16;       // K / V rows staged
    constexpr int RS = row_bytes<D>();
    constexpr uint32_t kOut = 0xfffffff0u;  // a buffer offset past any slice: loads 0

    const int nqt = (a.Sq + 15) >> 4;
    const int nqp = (nqt + 1) >> 1;  // pairs of query tiles
    const int RQ = nqp * 32;         // Q / dO rows staged

    lds_t* const sk = lds_base();
    lds_t* const sv = sk + RK * RS;
    lds_t* const sq = sv + RK * RS;
    lds_t* const sdo = sq + RQ * RS;
    lds_t* const slse = sdo + RQ * RS;    // RQ floats: log-sum-exp in log2 units
    lds_t* const sdelta = slse + RQ * 4;  // RQ floats: -rowsum(O * dO)

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int m = lane & 15, g = lane >> 4;
    const int b = blockIdx.x / a.H, h = blockIdx.x - (blockIdx.x / a.H) * a.H;
    const float kNegInf = -__builtin_inff();

    // One descriptor per tensor slice, ending at its last row: rows past S
    // read as zero, output rows past S are dropped.
    auto slice = [&](const void* base, int64_t sb, int64_t sh, int ss, int rows) {
        return make_rsrc(static_cast<const T*>(base) + b * sb + h * sh, (uint32_t)(((rows - 1) * ss + D) * 2));
    };
    const rsrc_t rq = slice(a.q, a.qsb, a.qsh, a.qss, a.Sq);
    const rsrc_t rk = slice(a.k, a.ksb, a.ksh, a.kss, a.Skv);
    const rsrc_t rv = slice(a.v, a.vsb, a.vsh, a.vss, a.Skv);
    const rsrc_t ro = slice(a.o, a.osb, a.osh, a.oss, a.Sq);
    const rsrc_t rdo = slice(a.dout, a.dosb, a.dosh, a.doss, a.Sq);
    const rsrc_t rdq = slice(a.dq, a.dqsb, a.dqsh, a.dqss, a.Sq);
    const rsrc_t rdk = slice(a.dk, a.dksb, a.dksh, a.dkss, a.Skv);
    const rsrc_t rdv = slice(a.dv, a.dvsb, a.dvsh, a.dvss, a.Skv);

    // O rows of a query tile in the MFMA operand layout (row m, chunks 4i+g),
    // for delta; chunks past the row read 0.
    u32x4 oop[NI];
    auto load_o = [&](int qt) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const bool in = CH % 4 == 0 || 4 * i + g < CH;
            oop[i] = buf_ld16(ro, in ? (uint32_t)((qt * 16 + m) * a.oss + (4 * i + g) * 8) * 2 : kOut);
        }
    };
    if (wave < nqt) load_o(wave);

    // ---- stage K, V (RK rows), Q, dO (RQ rows) ------------------------------
    // Every load of a batch is issued before the first LDS store, so a
    // thread waits for memory once per batch (once in all at C3), not once
    // per row chunk.  Batches cover RK rows of all four tensors; query rows
    // past RK (S_q > S_kv) follow in a loop of their own.
    {
        constexpr int KIT = (RK * CH + kThreads - 1) / kThreads;
        constexpr int UB = KIT < 4 ? KIT : 4;  // chunks per thread per batch
        const int nq = RQ * CH;
        for (int base = 0; base < RK * CH; base += UB * kThreads) {
            u32x4 kx[UB], vx[UB], qx[UB], dx[UB];
#pragma unroll
            for (int u = 0; u < UB; ++u) {
                const int idx = base + u * kThreads + tid;
                const int r = idx / CH, c = idx - (idx / CH) * CH;
                const bool kin = idx < RK * CH, qin = idx < nq;
                kx[u] = buf_ld16(rk, kin ? (uint32_t)(r * a.kss + c * 8) * 2 : kOut);
                vx[u] = buf_ld16(rv, kin ? (uint32_t)(r * a.vss + c * 8) * 2 : kOut);
                qx[u] = buf_ld16(rq, qin ? (uint32_t)(r * a.qss + c * 8) * 2 : kOut);
                dx[u] = buf_ld16(rdo, qin ? (uint32_t)(r * a.doss + c * 8) * 2 : kOut);
            }
#pragma unroll
            for (int u = 0; u < UB; ++u) {
                const int idx = base + u * kThreads + tid;
                const int r = idx / CH, c = idx - (idx / CH) * CH;
                if (idx < RK * CH) {
                    lds_st16(sk + chunk_off<D>(r, c), kx[u]);
                    lds_st16(sv + chunk_off<D>(r, c), vx[u]);
                }
                if (idx < nq) {
                    lds_st16(sq + chunk_off<D>(r, c), qx[u]);
                    lds_st16(sdo + chunk_off<D>(r, c), dx[u]);
                }
            }
        }
        for (int idx = RK * CH + tid; idx < nq; idx += kThreads) {
            const int r = idx / CH, c = idx - (idx / CH) * CH;
            lds_st16(sq + chunk_off<D>(r, c), buf_ld16(rq, (uint32_t)(r * a.qss + c * 8) * 2));
            lds_st16(sdo + chunk_off<D>(r, c), buf_ld16(rdo, (uint32_t)(r * a.doss + c * 8) * 2));
        }
    }
    // Rows of the last pair that no query tile covers: defined lse and delta.
    for (int r = nqt * 16 + tid; r < RQ; r += kThreads) {
        lds_st4(slse + r * 4, 0u);
        lds_st4(sdelta + r * 4, 0u);
    }

    // Usable keys of this lane in phase 1 (bit 4*kt + i <-> key 16*kt + 4g + i).
    uint64_t kbits = 0;
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt) {
        const int n = min(max(a.Skv - (kt * 16 + 4 * g), 0), 4);
        kbits |= (uint64_t)((1u << n) - 1u) << (4 * kt);
    }
    const uint8_t* prow = a.kpad ? a.kpad + (int64_t)b * a.kpsb : nullptr;
    if (prow) {
        for (int kt = 0; kt < NKT; ++kt)
            for (int i = 0; i < 4; ++i) {
                const int key = kt * 16 + 4 * g + i;
                if (key < a.Skv && prow[key]) kbits &= ~((uint64_t)1 << (4 * kt + i));
            }
    }
    __syncthreads();

    // Per-lane LDS offsets.  Operand reads of 16-row tiles: row m, chunks
    // 4i + g.  Transposing reads: input lane a4 + 4t of a 16-lane group points
    // at row 4g + t and elements a4*QD + 4dt .. +3, which hands lane m the
    // four rows 4g .. 4g+3 of head-dim (m/4)*QD + 4dt + m%4.
    int coff[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) coff[i] = chunk_off<D>(m, 4 * i + g);
    int troff[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) troff[dt] = quad_off<D>(4 * g + (m >> 2), (m & 3) * QD + 4 * dt);
    auto ld_op = [&](const lds_t* base, int i) {
        u32x4 v = lds_ld16(base + coff[i]);
        if (CH % 4 != 0 && 4 * i + g >= CH) v = u32x4{0, 0, 0, 0};
        return v;
    };
    // Stores QD contiguous elements d = g*QD .. of row `row` from four-element
    // groups x[dt] (d = g*QD + 4dt + i), scaled.
    auto store_row = [&](rsrc_t r, int ss, int row, const f32x4 (&x)[NDT], float mul) {
        const uint32_t base = (uint32_t)(row * ss + g * QD) * 2;
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
    auto dot8 = [&](u32x4 x, u32x4 y, float acc) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc = M::dot2(x[j], y[j], acc);
        return acc;
    };

    // ---- phase 1: one 16-query tile per wave pass --------------------------
    for (int qt = wave; qt < nqt; qt += kWaves) {
        const int qrow = qt * 16 + m;
        const lds_t* const qbase = sq + qt * 16 * RS;
        const lds_t* const dobase = sdo + qt * 16 * RS;
        u32x4 qop[NI], doop[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            qop[i] = ld_op(qbase, i);
            doop[i] = ld_op(dobase, i);
        }
        // delta = rowsum(O * dO) of this lane's query (the first tile's O
        // was requested before the staging loads)
        if (qt != wave) load_o(qt);
        float part = 0.f;
#pragma unroll
        for (int i = 0; i < NI; ++i) part = dot8(oop[i], doop[i], part);
        const float delta = colgroup_sum(part);
        // usable keys of this query row
        uint64_t ok = kbits;
        if (a.causal) {
            uint64_t cb = 0;
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt) {
                const int n = min(max(qrow - (kt * 16 + 4 * g) + 1, 0), 4);
                cb |= (uint64_t)((1u << n) - 1u) << (4 * kt);
            }
            ok &= cb;
        }
        // Keys at or past kend are unusable for every query of the tile;
        // tiles below kfull need no per-score mask (no padding, every key
        // < S_kv and, causal, <= the tile's first query).
        const int kend = a.causal ? min(a.Skv, qt * 16 + 16) : a.Skv;
        const int kfull = prow ? 0 : (a.causal ? min(a.Skv, qt * 16 + 1) : a.Skv);
        // S^T = K Q^T (raw scores; masked ones -inf)
        f32x4 s[NKT];  // tiles at or past kend are never read
        float mx = kNegInf;
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt) {
            if (kt * 16 < kend) {
                f32x4 acc = M::mma(ld_op(sk + kt * 16 * RS, 0), qop[0], f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                for (int i = 1; i < NI; ++i) acc = M::mma(ld_op(sk + kt * 16 * RS, i), qop[i], acc);
                if (kt * 16 + 16 > kfull) {
                    // keep or -inf by bit masks (whole-vector casts: a bit
                    // cast of one vector element reads element 0)
                    const uint32_t w = (uint32_t)(ok >> (4 * kt));
                    u32x4 ab = __builtin_bit_cast(u32x4, acc);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t keep = (uint32_t)((int32_t)(w << (31 - i)) >> 31);
                        ab[i] = (ab[i] & keep) | (~keep & 0xff800000u);
                    }
                    acc = __builtin_bit_cast(f32x4, ab);
                }
                mx = fmaxf(fmaxf(mx, acc[0]), acc[1]);
                mx = fmaxf(fmaxf(mx, acc[2]), acc[3]);
                s[kt] = acc;
            }
        }
        mx = colgroup_max(mx);
        // no usable key: P = 0 everywhere here (dQ = 0); lse stays -inf
        const bool empty = mx == kNegInf;
        const float nbase = empty ? 0.f : -mx * a.c2;
        float sum = 0.f;
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt) {
            if (kt * 16 < kend) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    s[kt][i] = fast_exp2(__builtin_fmaf(s[kt][i], a.c2, nbase));  // unnormalised P
                    sum += s[kt][i];
                }
            }
        }
        sum = colgroup_sum(sum);
        const float lse = empty ? kNegInf : mx * a.c2 + __builtin_log2f(sum);
        const float rs = empty ? 0.f : a.scale / sum;  // normalisation and dQ's scale
        const float ndelta = empty ? 0.f : -delta;
        if (g == 0) {
            lds_st4(slse + qrow * 4, __builtin_bit_cast(uint32_t, lse));
            lds_st4(sdelta + qrow * 4, __builtin_bit_cast(uint32_t, ndelta));
        }
        const f32x4 ndelta4 = f32x4{ndelta, ndelta, ndelta, ndelta};
        // dP^T - delta = V dO^T - delta (the accumulator starts at -delta),
        // scale * dS^T = P^T (dP^T - delta) * scale, packed per 32-key chunk
        u32x4 dsk[NKC];
#pragma unroll
        for (int c = 0; c < NKC; ++c) {
            float ds[8];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int kt = 2 * c + hh;
                if (kt * 16 < kend) {
                    f32x4 dp = M::mma(ld_op(sv + kt * 16 * RS, 0), doop[0], ndelta4);
#pragma unroll
                    for (int i = 1; i < NI; ++i) dp = M::mma(ld_op(sv + kt * 16 * RS, i), doop[i], dp);
#pragma unroll
                    for (int i = 0; i < 4; ++i) ds[4 * hh + i] = s[kt][i] * (rs * dp[i]);
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) ds[4 * hh + i] = 0.f;
                }
            }
            dsk[c] = u32x4{M::pack2(ds[0], ds[1]), M::pack2(ds[2], ds[3]), M::pack2(ds[4], ds[5]), M::pack2(ds[6], ds[7])};
        }
        // dQ^T = K^T (scale * dS^T)
        f32x4 dq[NDT];
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) dq[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NKC; ++c) {
            if (c * 32 < kend) {
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) {
                    const u32x2 lo = lds_ld8_tr16(sk + 32 * c * RS + troff[dt]);
                    const u32x2 hi = lds_ld8_tr16(sk + (32 * c + 16) * RS + troff[dt]);
                    dq[dt] = M::mma(u32x4{lo[0], lo[1], hi[0], hi[1]}, dsk[c], dq[dt]);
                }
            }
        }
        store_row(rdq, a.dqss, qrow, dq, 1.0f);
    }
    __syncthreads();  // log-sum-exp and delta of every query are in LDS

    // ---- phase 2: one 16-key tile per wave pass ----------------------------
    for (int kt = wave; kt < NKT; kt += kWaves) {
        if (kt * 16 >= a.Skv) break;  // no key here: nothing to compute or store
        const int key = kt * 16 + m;
        const bool kok = key < a.Skv && !(prow && prow[key]);
        const bool kfull = __builtin_amdgcn_ballot_w64(!kok) == 0;
        const lds_t* const kbase = sk + kt * 16 * RS;
        const lds_t* const vbase = sv + kt * 16 * RS;
        u32x4 kop[NI], vop[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            kop[i] = ld_op(kbase, i);
            vop[i] = ld_op(vbase, i);
        }
        f32x4 dvt[NDT], dkt[NDT];
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) dvt[dt] = dkt[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
        // causal: pairs before kt / 2 end before the tile's first key and add
        // nothing, unless a query that sees no key (lse = -inf) makes its P
        // row NaN, which reaches every dV row
        bool skip_early = a.causal;
        if (skip_early) {
            bool e = false;
            for (int r = lane; r < RQ; r += 64) e |= __builtin_bit_cast(float, lds_ld4(slse + r * 4)) == kNegInf;
            skip_early = __builtin_amdgcn_ballot_w64(e) == 0;
        }
        for (int qp = skip_early ? kt / 2 : 0; qp < nqp; ++qp) {
            const int q0 = qp * 32;
            const bool full = kfull && q0 + 31 < a.Sq && (!a.causal || kt * 16 + 15 <= q0);
            float p[8], ds[8];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int qt = 2 * qp + hh;
                // S = Q K^T and dP - delta = dO V^T - delta (accumulated onto
                // -delta): rows = queries
                // qt*16 + 4g + i, column = key
                const f32x4 lse4 = as_f32x4(lds_ld16(slse + (qt * 16 + 4 * g) * 4));
                const f32x4 ndelta4 = as_f32x4(lds_ld16(sdelta + (qt * 16 + 4 * g) * 4));
                f32x4 sacc = M::mma(ld_op(sq + qt * 16 * RS, 0), kop[0], f32x4{0.f, 0.f, 0.f, 0.f});
                f32x4 dpacc = M::mma(ld_op(sdo + qt * 16 * RS, 0), vop[0], ndelta4);
#pragma unroll
                for (int i = 1; i < NI; ++i) {
                    sacc = M::mma(ld_op(sq + qt * 16 * RS, i), kop[i], sacc);
                    dpacc = M::mma(ld_op(sdo + qt * 16 * RS, i), vop[i], dpacc);
                }
                if (full) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float pv = fast_exp2(__builtin_fmaf(sacc[i], a.c2, -lse4[i]));
                        p[4 * hh + i] = pv;
                        ds[4 * hh + i] = pv * dpacc[i];
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int q = qt * 16 + 4 * g + i;
                        const bool ok = kok && q < a.Sq && (!a.causal || key <= q);
                        const float pv = fast_exp2(__builtin_fmaf(sacc[i], a.c2, -lse4[i]));
                        // 0 * lse: NaN only for a query that sees no key (lse = -inf)
                        p[4 * hh + i] = ok ? pv : 0.f * lse4[i];
                        ds[4 * hh + i] = ok ? pv * dpacc[i] : 0.f;
                    }
                }
            }
            const u32x4 pb = {M::pack2(p[0], p[1]), M::pack2(p[2], p[3]), M::pack2(p[4], p[5]), M::pack2(p[6], p[7])};
            const u32x4 db = {M::pack2(ds[0], ds[1]), M::pack2(ds[2], ds[3]), M::pack2(ds[4], ds[5]), M::pack2(ds[6], ds[7])};
            // dV^T += dO^T P,  dK^T += Q^T dS over the 32 queries of the pair
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
                const u32x2 dlo = lds_ld8_tr16(sdo + 32 * qp * RS + troff[dt]);
                const u32x2 dhi = lds_ld8_tr16(sdo + (32 * qp + 16) * RS + troff[dt]);
                dvt[dt] = M::mma(u32x4{dlo[0], dlo[1], dhi[0], dhi[1]}, pb, dvt[dt]);
                const u32x2 qlo = lds_ld8_tr16(sq + 32 * qp * RS + troff[dt]);
                const u32x2 qhi = lds_ld8_tr16(sq + (32 * qp + 16) * RS + troff[dt]);
                dkt[dt] = M::mma(u32x4{qlo[0], qlo[1], qhi[0], qhi[1]}, db, dkt[dt]);
            }
        }
        store_row(rdv, a.dvss, key, dvt, 1.0f);
        store_row(rdk, a.dkss, key, dkt, a.scale);
    }
}

namespace {

template <typename K>
int launch_bwd(K kernel, int grid, size_t lds, hipStream_t st, const BwdArgs& a) {
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) ATX_FAIL(ATX_ERR_LAUNCH, "hipFuncSetAttribute(%zu bytes LDS): %s", lds, hipGetErrorString(e));
    }
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kThreads), lds, st, a);
    ATX_CHECK_LAUNCH("atx_attn_bwd launch");
    return ATX_OK;
}

template <typename T, int D>
int dispatch_bwd_nkc(int nkc, int grid, size_t lds, hipStream_t st, const BwdArgs& a) {
    switch (nkc) {
        case 1: return launch_bwd(attn_bwd_16bit<T, D, 1>, grid, lds, st, a);
        case 2: return launch_bwd(attn_bwd_16bit<T, D, 2>, grid, lds, st, a);
        case 3: return launch_bwd(attn_bwd_16bit<T, D, 3>, grid, lds, st, a);
        case 4: return launch_bwd(attn_bwd_16bit<T, D, 4>, grid, lds, st, a);
        case 5: return launch_bwd(attn_bwd_16bit<T, D, 5>, grid, lds, st, a);
        case 6: return launch_bwd(attn_bwd_16bit<T, D, 6>, grid, lds, st, a);
        case 7: return launch_bwd(attn_bwd_16bit<T, D, 7>, grid, lds, st, a);
        case 8: return launch_bwd(attn_bwd_16bit<T, D, 8>, grid, lds, st, a);
        default: ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: seq_kv needs %d 32-key chunks (<= 8)", nkc);
    }
}

template <typename T>
int dispatch_bwd(int D, int nkc, int grid, size_t lds, hipStream_t st, const BwdArgs& a) {
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

bool rows16(const void* base, int64_t sb, int64_t ss, int64_t sh) {
    return aligned16(base) && ((sb * 2) & 15) == 0 && ((ss * 2) & 15) == 0 && ((sh * 2) & 15) == 0;
}

}  // namespace
}  // namespace atx

extern "C" int atx_attn_bwd(const AtxAttnBwdParams* p, void* stream) {
    using namespace atx;
    clear_error();
    if (!p) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_bwd: params is NULL");
    if (p->abi_version != ATX_ABI_VERSION)
        ATX_FAIL(ATX_ERR_ABI, "atx_attn_bwd: abi_version %d, library is %d", p->abi_version, ATX_ABI_VERSION);
    if (p->dtype != ATX_DTYPE_BF16 && p->dtype != ATX_DTYPE_FP16) {
        if (p->dtype == ATX_DTYPE_FP32) ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: fp32 is not supported");
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_bwd: unknown dtype %d", p->dtype);
    }
    if (p->batch < 1 || p->seq_q < 1 || p->seq_kv < 1 || p->num_heads < 1 || p->num_kv_heads < 1 || p->head_dim < 1)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_bwd: sizes must be >= 1");
    if (p->num_kv_heads != p->num_heads)
        ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: num_kv_heads %d != num_heads %d (GQA) not supported",
                 p->num_kv_heads, p->num_heads);
    if (!p->q || !p->k || !p->v || !p->o || !p->d_o || !p->dq || !p->dk || !p->dv)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_bwd: null tensor pointer");
    if (!(p->scale > 0.f) || p->scale == __builtin_inff())
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_bwd: scale must be finite and > 0 (got %g)", (double)p->scale);
    if (p->head_dim % 16 != 0 || p->head_dim > 128)
        ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: head_dim %d not supported (multiple of 16, <= 128)", p->head_dim);
    if (p->seq_q > 256 || p->seq_kv > 256)
        ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: seq_q %d / seq_kv %d not supported (<= 256)", p->seq_q, p->seq_kv);
    const int64_t grid = (int64_t)p->batch * p->num_heads;
    if (grid > 0x7fffffff) ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: batch*heads too large");
    // Sequence strides of length-1 sequences are never used.
    auto sstride = [](int64_t s, int seq, int d) { return seq == 1 ? (int64_t)d : s; };
    const int D = p->head_dim;
    const int64_t qss = sstride(p->q_stride_s, p->seq_q, D), oss = sstride(p->o_stride_s, p->seq_q, D);
    const int64_t doss = sstride(p->do_stride_s, p->seq_q, D), dqss = sstride(p->dq_stride_s, p->seq_q, D);
    const int64_t kss = sstride(p->k_stride_s, p->seq_kv, D), vss = sstride(p->v_stride_s, p->seq_kv, D);
    const int64_t dkss = sstride(p->dk_stride_s, p->seq_kv, D), dvss = sstride(p->dv_stride_s, p->seq_kv, D);
    if (!rows16(p->q, p->q_stride_b, qss, p->q_stride_h) || !rows16(p->k, p->k_stride_b, kss, p->k_stride_h) ||
        !rows16(p->v, p->v_stride_b, vss, p->v_stride_h) || !rows16(p->o, p->o_stride_b, oss, p->o_stride_h) ||
        !rows16(p->d_o, p->do_stride_b, doss, p->do_stride_h) ||
        !rows16(p->dq, p->dq_stride_b, dqss, p->dq_stride_h) ||
        !rows16(p->dk, p->dk_stride_b, dkss, p->dk_stride_h) || !rows16(p->dv, p->dv_stride_b, dvss, p->dv_stride_h))
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_bwd: every row must start on a 16-byte boundary");
    // one (batch, head) slice per descriptor: 32-bit offsets, rows up to the
    // next multiple of 32 past the end; output rows must not overlap
    const int64_t strides_q[] = {qss, oss, doss, dqss}, strides_k[] = {kss, vss, dkss, dvss};
    for (int64_t s : strides_q)
        if (s < 0 || (p->seq_q + 32) * s * 2 + D * 2 > 0x7fffffffLL)
            ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: sequence strides must be >= 0 and one slice < 2 GiB");
    for (int64_t s : strides_k)
        if (s < 0 || (p->seq_kv + 32) * s * 2 + D * 2 > 0x7fffffffLL)
            ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: sequence strides must be >= 0 and one slice < 2 GiB");
    if (dqss < D || dkss < D || dvss < D)
        ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_attn_bwd: gradient rows overlap");

    const int nkc = (p->seq_kv + 31) / 32;
    const int rk = nkc * 32, rq = ((p->seq_q + 31) / 32) * 32;
    const size_t lds = bwd_lds_bytes(D, rk, rq);
    if (lds > 160 * 1024)
        ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_attn_bwd: seq_q %d, seq_kv %d, head_dim %d need %zu bytes of LDS (> 160 KiB)",
                 p->seq_q, p->seq_kv, D, lds);

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
    a.Sq = p->seq_q;
    a.Skv = p->seq_kv;
    a.c2 = p->scale * kLog2e;
    a.scale = p->scale;
    a.causal = p->causal != 0;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (p->dtype == ATX_DTYPE_BF16) return dispatch_bwd<__bf16>(D, nkc, (int)grid, lds, st, a);
    return dispatch_bwd<_Float16>(D, nkc, (int)grid, lds, st, a);
}
