// Attention backward kernels for gfx950 (see atx_attn_bwd.hip for the
// algorithm): the 16-bit kernel, the fp32 kernel and their launcher, shared by
// the translation units that instantiate them (16-bit, 16-bit LOOP, fp32,
// fp32 LOOP), so
// that the instantiations compile in parallel.
#pragma once
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
    int H, G, Sq, Skv;  // query heads, query heads per KV head
    int QB;             // LOOP variants: query rows staged per block (multiple of 32; fp32: 16)
    float c2, scale;  // c2 = scale * log2(e)
    int causal;
    DropKey drop;  // attention dropout (the DROP instantiations only)
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
template <int D, int NKC, bool LOOP = false>
constexpr int bwd_occ() {
    // LOOP keeps each wave's dK / dV tiles across the blocks: 2 waves per
    // SIMD (256 VGPRs) leave room for them
    return (!LOOP && NKC <= 4 && D <= 64) ? 4 : 2;
}

// NKC = 32-key chunks (S_kv <= 32 * NKC).  LOOP (grouped-query attention, or
// a query sequence whose rows do not all fit in LDS): one workgroup per
// (batch, KV head) runs the G = H / H_kv query heads of the group, each in
// blocks of QB query rows, one block after another; K and V are staged once,
// Q and dO per block, and each wave's dK / dV tiles accumulate over the
// blocks in registers (fp32, in head then block order) before the single
// store -- the sum over the repeat_interleave'd heads of attention.py:210-220
// and over all queries, without atomics.  dQ rows are complete per block
// (every key is resident).
//
// DROP (attention dropout): the forward used P' = P o M,
// M = keep / (1 - p) from drop_hash.  dV = P'^T dO, and with dP' = dO V^T,
// dS = P o (M o dP' - delta); delta = rowsum(P o M o dP') = rowsum(O o dO)
// with O the forward's dropout output, so delta is unchanged.  The dP'
// accumulators then start at 0 and M joins before -delta.
template <typename T, int D, int NKC, bool LOOP, bool DROP = false>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(bwd_occ<D, NKC, LOOP>(), 8)))
void attn_bwd_16bit(BwdArgs a) {
    using M = Mfma16<T>;
    constexpr int CH = D / 8;          // 16-byte chunks per row
    constexpr int NI = (D + 31) / 32;  // MFMAs per 16x16 score tile
    constexpr int NDT = D / 16;        // head-dim output tiles
    constexpr int QD = D / 4;          // contiguous outputs per lane
    constexpr int NKT = 2 * NKC;       // key tiles
    constexpr int RK = NKT * 16;       // K / V rows staged
    constexpr int RS = row_bytes<D>();
    constexpr int NSLOT = (NKT + kWaves - 1) / kWaves;  // key tiles per wave
    constexpr uint32_t kOut = 0xfffffff0u;  // a buffer offset past any slice: loads 0

    // Q / dO rows of the LDS layout: every query (pairs of 16-row tiles), or
    // (LOOP) one block of QB rows
    const int RQ = LOOP ? a.QB : ((((a.Sq + 15) >> 4) + 1) >> 1) * 32;
    const int nblk = LOOP ? (a.Sq + a.QB - 1) / a.QB : 1;

    lds_t* const sk0 = lds_base();

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int m = lane & 15, g = lane >> 4;
    const int G = LOOP ? a.G : 1;
    const int Hkv = a.H / G;
    const int b = blockIdx.x / Hkv, hk = blockIdx.x - (blockIdx.x / Hkv) * Hkv;
    const float kNegInf = -__builtin_inff();

    // One descriptor per tensor slice, ending at its last row: rows past S
    // read as zero, output rows past S are dropped.
    auto slice = [&](const void* base, int64_t sb, int64_t sh, int hh, int ss, int rows, int r0 = 0) {
        return make_rsrc(static_cast<const T*>(base) + b * sb + hh * sh + (int64_t)r0 * ss,
                         (uint32_t)(((rows - 1) * ss + D) * 2));
    };
    const rsrc_t rk = slice(a.k, a.ksb, a.ksh, hk, a.kss, a.Skv);
    const rsrc_t rv = slice(a.v, a.vsb, a.vsh, hk, a.vss, a.Skv);
    const rsrc_t rdk = slice(a.dk, a.dksb, a.dksh, hk, a.dkss, a.Skv);
    const rsrc_t rdv = slice(a.dv, a.dvsb, a.dvsh, hk, a.dvss, a.Skv);

    // Usable keys of this lane in phase 1 (bit 4*kt + i <-> key 16*kt + 4g + i).
    uint64_t kbits = 0;
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt) {
        const int n = min(max(a.Skv - (kt * 16 + 4 * g), 0), 4);
        kbits |= (uint64_t)((1u << n) - 1u) << (4 * kt);
    }
    const uint8_t* prow = a.kpad ? a.kpad + (int64_t)b * a.kpsb : nullptr;

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

    // dK / dV of the wave's key tiles summed over the group's heads and the
    // query blocks (LOOP only)
    f32x4 dvs[LOOP ? NSLOT : 1][NDT], dks[LOOP ? NSLOT : 1][NDT];
    if constexpr (LOOP)
#pragma unroll
        for (int j = 0; j < NSLOT; ++j)
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) dvs[j][dt] = dks[j][dt] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int it = 0; it < G * nblk; ++it) {
        const int hg = it / nblk, qb = it - (it / nblk) * nblk;
        const int h = hk * G + hg;
        const int q0 = qb * (LOOP ? a.QB : 0);    // first query of the block
        const int Sqb = LOOP ? min(a.QB, a.Sq - q0) : a.Sq;  // its queries
        const int nqt = (Sqb + 15) >> 4;
        const int nqp = (nqt + 1) >> 1;  // pairs of query tiles
        const rsrc_t rq = slice(a.q, a.qsb, a.qsh, h, a.qss, Sqb, q0);
        const rsrc_t ro = slice(a.o, a.osb, a.osh, h, a.oss, Sqb, q0);
        const rsrc_t rdo = slice(a.dout, a.dosb, a.dosh, h, a.doss, Sqb, q0);
        const rsrc_t rdq = slice(a.dq, a.dqsb, a.dqsh, h, a.dqss, Sqb, q0);
        if (LOOP && it > 0) __syncthreads();  // the previous block's phase 2 is done with Q, dO, lse, delta
        // LDS bases, re-derived per block through an opaque copy in the LOOP
        // variant: otherwise the K / V operand reads, the same for every
        // block, are hoisted out of the loop and the kernel runs out of
        // registers.
        lds_t* const sk = LOOP ? lds_opaque(sk0) : sk0;
        lds_t* const sv = sk + RK * RS;
        lds_t* const sq = sv + RK * RS;
        lds_t* const sdo = sq + RQ * RS;
        lds_t* const slse = sdo + RQ * RS;    // RQ floats: log-sum-exp in log2 units
        lds_t* const sdelta = slse + RQ * 4;  // RQ floats: -rowsum(O * dO)

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

        // ---- stage K, V (RK rows, first head only), Q, dO (RQ rows) ----------
        // Every load of a batch is issued before the first LDS store, so a
        // thread waits for memory once per batch (once in all at C3), not once
        // per row chunk.  Batches cover RK rows of all four tensors; query rows
        // past RK (S_q > S_kv) follow in a loop of their own.
        {
            constexpr int KIT = (RK * CH + kThreads - 1) / kThreads;
            constexpr int UB = KIT < 4 ? KIT : 4;  // chunks per thread per batch
            const int nq = nqp * 32 * CH;
            const bool kv = it == 0;
            for (int base = 0; base < RK * CH; base += UB * kThreads) {
                u32x4 kx[UB], vx[UB], qx[UB], dx[UB];
#pragma unroll
                for (int u = 0; u < UB; ++u) {
                    const int idx = base + u * kThreads + tid;
                    const int r = idx / CH, c = idx - (idx / CH) * CH;
                    const bool kin = kv && idx < RK * CH, qin = idx < nq;
                    if (!LOOP || kv) {
                        kx[u] = buf_ld16(rk, kin ? (uint32_t)(r * a.kss + c * 8) * 2 : kOut);
                        vx[u] = buf_ld16(rv, kin ? (uint32_t)(r * a.vss + c * 8) * 2 : kOut);
                    }
                    qx[u] = buf_ld16(rq, qin ? (uint32_t)(r * a.qss + c * 8) * 2 : kOut);
                    dx[u] = buf_ld16(rdo, qin ? (uint32_t)(r * a.doss + c * 8) * 2 : kOut);
                }
#pragma unroll
                for (int u = 0; u < UB; ++u) {
                    const int idx = base + u * kThreads + tid;
                    const int r = idx / CH, c = idx - (idx / CH) * CH;
                    if ((!LOOP || kv) && idx < RK * CH) {
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
        if (it == 0 && prow) {
            for (int kt = 0; kt < NKT; ++kt)
                for (int i = 0; i < 4; ++i) {
                    const int key = kt * 16 + 4 * g + i;
                    if (key < a.Skv && prow[key]) kbits &= ~((uint64_t)1 << (4 * kt + i));
                }
        }
        __syncthreads();

        // ---- phase 1: one 16-query tile per wave pass --------------------------
        for (int qt = wave; qt < nqt; qt += kWaves) {
            const int qrow = qt * 16 + m;  // row of the block
            const int qabs = q0 + qrow;    // query index
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
                    const int n = min(max(qabs - (kt * 16 + 4 * g) + 1, 0), 4);
                    cb |= (uint64_t)((1u << n) - 1u) << (4 * kt);
                }
                ok &= cb;
            }
            // Keys at or past kend are unusable for every query of the tile;
            // tiles below kfull need no per-score mask (no padding, every key
            // < S_kv and, causal, <= the tile's first query).
            const int kend = a.causal ? min(a.Skv, q0 + qt * 16 + 16) : a.Skv;
            const int kfull = prow ? 0 : (a.causal ? min(a.Skv, q0 + qt * 16 + 1) : a.Skv);
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
            // dropout row of this query: element index of key 0
            const uint64_t drow = DROP ? (uint64_t)(((int64_t)b * a.H + h) * a.Sq + qabs) * (uint64_t)a.Skv : 0;
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
                        f32x4 dp = M::mma(ld_op(sv + kt * 16 * RS, 0), doop[0], DROP ? f32x4{0.f, 0.f, 0.f, 0.f} : ndelta4);
#pragma unroll
                        for (int i = 1; i < NI; ++i) dp = M::mma(ld_op(sv + kt * 16 * RS, i), doop[i], dp);
                        if constexpr (DROP) {
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                const bool keep = drop_hash(drow + (uint64_t)(kt * 16 + 4 * g + i), a.drop.k0, a.drop.k1) >= a.drop.thresh;
                                dp[i] = __builtin_fmaf(dp[i], keep ? a.drop.scale : 0.f, ndelta);
                            }
                        }
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
        // dV^T += dO^T P and dK^T += Q^T dS of key tile kt over every query
        // pair, into dvt / dkt.
        auto key_tile = [&](int kt, f32x4 (&dvt)[NDT], f32x4 (&dkt)[NDT]) {
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
            // causal: pairs ending before the tile's first key add nothing,
            // unless a query that sees no key (lse = -inf) makes its P row
            // NaN, which reaches every dV row
            bool skip_early = a.causal;
            if (skip_early) {
                bool e = false;
                for (int r = lane; r < RQ; r += 64) e |= __builtin_bit_cast(float, lds_ld4(slse + r * 4)) == kNegInf;
                skip_early = __builtin_amdgcn_ballot_w64(e) == 0;
            }
            for (int qp = skip_early ? max(0, (kt * 16 - q0) / 32) : 0; qp < nqp; ++qp) {
                const int qp0 = qp * 32;  // first row of the pair in the block
                const bool full = kfull && qp0 + 31 < Sqb && (!a.causal || kt * 16 + 15 <= q0 + qp0);
                float p[8], ds[8];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int qt = 2 * qp + hh;
                    // S = Q K^T and dP - delta = dO V^T - delta (accumulated onto
                    // -delta): rows = queries qt*16 + 4g + i, column = key
                    const f32x4 lse4 = as_f32x4(lds_ld16(slse + (qt * 16 + 4 * g) * 4));
                    const f32x4 ndelta4 = as_f32x4(lds_ld16(sdelta + (qt * 16 + 4 * g) * 4));
                    f32x4 sacc = M::mma(ld_op(sq + qt * 16 * RS, 0), kop[0], f32x4{0.f, 0.f, 0.f, 0.f});
                    f32x4 dpacc = M::mma(ld_op(sdo + qt * 16 * RS, 0), vop[0], DROP ? f32x4{0.f, 0.f, 0.f, 0.f} : ndelta4);
#pragma unroll
                    for (int i = 1; i < NI; ++i) {
                        sacc = M::mma(ld_op(sq + qt * 16 * RS, i), kop[i], sacc);
                        dpacc = M::mma(ld_op(sdo + qt * 16 * RS, i), vop[i], dpacc);
                    }
                    f32x4 ms = f32x4{1.f, 1.f, 1.f, 1.f};  // dropout multiplier of each score
                    if constexpr (DROP) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const uint64_t idx =
                                (uint64_t)(((int64_t)b * a.H + h) * a.Sq + q0 + qt * 16 + 4 * g + i) * (uint64_t)a.Skv + key;
                            ms[i] = drop_hash(idx, a.drop.k0, a.drop.k1) >= a.drop.thresh ? a.drop.scale : 0.f;
                            dpacc[i] = __builtin_fmaf(dpacc[i], ms[i], ndelta4[i]);
                        }
                    }
                    if (full) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const float pv = fast_exp2(__builtin_fmaf(sacc[i], a.c2, -lse4[i]));
                            p[4 * hh + i] = DROP ? pv * ms[i] : pv;
                            ds[4 * hh + i] = pv * dpacc[i];
                        }
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int q = qt * 16 + 4 * g + i;
                            const bool ok = kok && q < Sqb && (!a.causal || key <= q0 + q);
                            const float pv = fast_exp2(__builtin_fmaf(sacc[i], a.c2, -lse4[i]));
                            // 0 * lse: NaN only for a query that sees no key (lse = -inf)
                            p[4 * hh + i] = ok ? (DROP ? pv * ms[i] : pv) : 0.f * lse4[i];
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
        };
        if constexpr (LOOP) {
#pragma unroll
            for (int j = 0; j < NSLOT; ++j) {
                const int kt = wave + j * kWaves;
                if (kt < NKT && kt * 16 < a.Skv) key_tile(kt, dvs[j], dks[j]);
            }
        } else {
            for (int kt = wave; kt < NKT; kt += kWaves) {
                if (kt * 16 >= a.Skv) break;  // no key here: nothing to compute or store
                f32x4 dvt[NDT], dkt[NDT];
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) dvt[dt] = dkt[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
                key_tile(kt, dvt, dkt);
                store_row(rdv, a.dvss, kt * 16 + m, dvt, 1.0f);
                store_row(rdk, a.dkss, kt * 16 + m, dkt, a.scale);
            }
        }
    }
    if constexpr (LOOP) {
#pragma unroll
        for (int j = 0; j < NSLOT; ++j) {
            const int kt = wave + j * kWaves;
            if (kt < NKT && kt * 16 < a.Skv) {
                store_row(rdv, a.dvss, kt * 16 + m, dvs[j], 1.0f);
                store_row(rdk, a.dkss, kt * 16 + m, dks[j], a.scale);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// fp32 backward: the same two phases on v_mfma_f32_16x16x4_f32 (full fp32
// products).  K, V, Q and dO of the (batch, head) are staged in LDS as fp32
// rows; a row's 4-float chunk ch sits at ch ^ hsw(r), which keeps both the
// 16-byte row reads (16 rows, one chunk each) and the single-element
// "transposed" reads (4 rows x 16 head-dim columns) on distinct banks at
// D = 64.  An MFMA k-step covers one element of a 4-float chunk per lane
// group, so the dot products over d run in the order (chunk, element); the
// A and B operands always agree on it.
// ---------------------------------------------------------------------------
template <int D>
constexpr int kHswMask = ((D / 4) % 16 == 0) ? 15 : ((D / 4) % 8 == 0) ? 7 : 3;
template <int D>
__device__ inline int hsw(int r) {
    return (((r & 3) << 2) | ((r >> 2) & 3)) & kHswMask<D>;
}
// float offset of row r, 4-float chunk ch
template <int D>
__device__ inline int f32_chunk(int r, int ch) {
    return r * D + ((ch ^ hsw<D>(r)) << 2);
}
// float offset of row r, column c
template <int D>
__device__ inline int f32_elem(int r, int c) {
    return r * D + (((c >> 2) ^ hsw<D>(r)) << 2) + (c & 3);
}

inline size_t bwd_lds_bytes_fp32(int D, int rk, int rq) { return (size_t)(2 * rk + 2 * rq) * D * 4 + (size_t)rq * 8; }

template <int D, int NKC>
constexpr int bwd_occ_fp32() {
    return 2;
}

template <int D, int NKC, bool LOOP, bool DROP = false>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(bwd_occ_fp32<D, NKC>(), 8)))
void attn_bwd_fp32(BwdArgs a) {
    constexpr int CH4 = D / 4;    // 4-float chunks per row
    constexpr int NI = D / 16;    // chunk groups (4 chunks, one per lane group) per row
    constexpr int NDT = D / 16;   // head-dim output tiles
    constexpr int QD = D / 4;     // contiguous outputs per lane
    constexpr int NKT = 2 * NKC;  // key tiles
    constexpr int RK = NKT * 16;
    constexpr int NSLOT = (NKT + kWaves - 1) / kWaves;
    constexpr uint32_t kOut = 0xfffffff0u;

    // Q / dO rows of the LDS layout: every query, or (LOOP) one block of QB
    const int RQ = LOOP ? a.QB : ((a.Sq + 15) >> 4) * 16;
    const int nblk = LOOP ? (a.Sq + a.QB - 1) / a.QB : 1;

    lds_t* const lk0 = lds_base();

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int m = lane & 15, g = lane >> 4;
    const int G = LOOP ? a.G : 1;
    const int Hkv = a.H / G;
    const int b = blockIdx.x / Hkv, hk = blockIdx.x - (blockIdx.x / Hkv) * Hkv;
    const float kNegInf = -__builtin_inff();

    auto slice = [&](const void* base, int64_t sb, int64_t sh, int hh, int ss, int rows, int r0 = 0) {
        return make_rsrc(static_cast<const float*>(base) + b * sb + hh * sh + (int64_t)r0 * ss,
                         (uint32_t)(((rows - 1) * ss + D) * 4));
    };
    const rsrc_t rk = slice(a.k, a.ksb, a.ksh, hk, a.kss, a.Skv);
    const rsrc_t rv = slice(a.v, a.vsb, a.vsh, hk, a.vss, a.Skv);
    const rsrc_t rdk = slice(a.dk, a.dksb, a.dksh, hk, a.dkss, a.Skv);
    const rsrc_t rdv = slice(a.dv, a.dvsb, a.dvsh, hk, a.dvss, a.Skv);

    uint64_t kbits = 0;
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt) {
        const int n = min(max(a.Skv - (kt * 16 + 4 * g), 0), 4);
        kbits |= (uint64_t)((1u << n) - 1u) << (4 * kt);
    }
    const uint8_t* prow = a.kpad ? a.kpad + (int64_t)b * a.kpsb : nullptr;

    auto ld_chunk = [&](const lds_t* base, int r, int ch) { return as_f32x4(lds_ld16(base + f32_chunk<D>(r, ch) * 4)); };
    auto ld_elem = [&](const lds_t* base, int r, int c) { return __builtin_bit_cast(float, lds_ld4(base + f32_elem<D>(r, c) * 4)); };
    // head-dim column that MFMA row m of output tile dt stands for
    auto dcol = [&](int dt) { return (m >> 2) * QD + 4 * dt + (m & 3); };
    // row `row`: QD contiguous floats g*QD .. from x[dt] (d = g*QD + 4dt + i)
    auto store_row = [&](rsrc_t r, int ss, int row, const f32x4 (&x)[NDT], float mul) {
        const uint32_t base = (uint32_t)(row * ss + g * QD) * 4;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
            buf_st16_cached(r, base + dt * 16, __builtin_bit_cast(u32x4, f32x4{x[dt][0] * mul, x[dt][1] * mul,
                                                                              x[dt][2] * mul, x[dt][3] * mul}));
    };

    f32x4 dvs[LOOP ? NSLOT : 1][NDT], dks[LOOP ? NSLOT : 1][NDT];
    if constexpr (LOOP)
#pragma unroll
        for (int j = 0; j < NSLOT; ++j)
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) dvs[j][dt] = dks[j][dt] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int it = 0; it < G * nblk; ++it) {
        const int hg = it / nblk, qb = it - (it / nblk) * nblk;
        const int h = hk * G + hg;
        const int q0 = qb * (LOOP ? a.QB : 0);
        const int Sqb = LOOP ? min(a.QB, a.Sq - q0) : a.Sq;
        const int nqt = (Sqb + 15) >> 4;
        const rsrc_t rq = slice(a.q, a.qsb, a.qsh, h, a.qss, Sqb, q0);
        const rsrc_t ro = slice(a.o, a.osb, a.osh, h, a.oss, Sqb, q0);
        const rsrc_t rdo = slice(a.dout, a.dosb, a.dosh, h, a.doss, Sqb, q0);
        const rsrc_t rdq = slice(a.dq, a.dqsb, a.dqsh, h, a.dqss, Sqb, q0);
        if (LOOP && it > 0) __syncthreads();
        lds_t* const lk = lds_opaque(lk0);  // no LDS read is hoisted out of the block loop
        lds_t* const lv = lk + RK * D * 4;
        lds_t* const lq = lv + RK * D * 4;
        lds_t* const ldo = lq + RQ * D * 4;
        lds_t* const slse = ldo + RQ * D * 4;
        lds_t* const sdelta = slse + RQ * 4;

        // ---- stage K, V (first head), Q, dO: 16-byte chunks -------------------
        {
            const bool kv = it == 0;
            const int nk = kv ? RK * CH4 : 0, nq = nqt * 16 * CH4;
            const int n = nk > nq ? nk : nq;
            for (int base = 0; base < n; base += 2 * kThreads) {
                u32x4 kx[2], vx[2], qx[2], dx[2];
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int idx = base + u * kThreads + tid;
                    const int r = idx / CH4, c = idx - (idx / CH4) * CH4;
                    kx[u] = buf_ld16(rk, idx < nk ? (uint32_t)(r * a.kss + c * 4) * 4 : kOut);
                    vx[u] = buf_ld16(rv, idx < nk ? (uint32_t)(r * a.vss + c * 4) * 4 : kOut);
                    qx[u] = buf_ld16(rq, idx < nq ? (uint32_t)(r * a.qss + c * 4) * 4 : kOut);
                    dx[u] = buf_ld16(rdo, idx < nq ? (uint32_t)(r * a.doss + c * 4) * 4 : kOut);
                }
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int idx = base + u * kThreads + tid;
                    const int r = idx / CH4, c = idx - (idx / CH4) * CH4;
                    if (idx < nk) {
                        lds_st16(lk + f32_chunk<D>(r, c) * 4, kx[u]);
                        lds_st16(lv + f32_chunk<D>(r, c) * 4, vx[u]);
                    }
                    if (idx < nq) {
                        lds_st16(lq + f32_chunk<D>(r, c) * 4, qx[u]);
                        lds_st16(ldo + f32_chunk<D>(r, c) * 4, dx[u]);
                    }
                }
            }
        }
        for (int r = nqt * 16 + tid; r < RQ; r += kThreads) {
            lds_st4(slse + r * 4, 0u);
            lds_st4(sdelta + r * 4, 0u);
        }
        if (it == 0 && prow) {
            for (int kt = 0; kt < NKT; ++kt)
                for (int i = 0; i < 4; ++i) {
                    const int key = kt * 16 + 4 * g + i;
                    if (key < a.Skv && prow[key]) kbits &= ~((uint64_t)1 << (4 * kt + i));
                }
        }
        __syncthreads();

        // ---- phase 1: one 16-query tile per wave pass ---------------------------
        for (int qt = wave; qt < nqt; qt += kWaves) {
            const int qrow = qt * 16 + m;  // row of the block
            const int qabs = q0 + qrow;
            // K / V reads are the same for every query tile: keep them in the loop
            const lds_t* const lkq = lds_opaque(lk);
            const lds_t* const lvq = lkq + RK * D * 4;
            f32x4 qop[NI], doop[NI];
            float part = 0.f;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                qop[i] = ld_chunk(lq, qrow, 4 * i + g);
                doop[i] = ld_chunk(ldo, qrow, 4 * i + g);
                const f32x4 o = as_f32x4(buf_ld16(ro, (uint32_t)(qrow * a.oss + (4 * i + g) * 4) * 4));
#pragma unroll
                for (int e = 0; e < 4; ++e) part = __builtin_fmaf(o[e], doop[i][e], part);
            }
            const float delta = colgroup_sum(part);
            uint64_t ok = kbits;
            if (a.causal) {
                uint64_t cb = 0;
#pragma unroll
                for (int kt = 0; kt < NKT; ++kt) {
                    const int n = min(max(qabs - (kt * 16 + 4 * g) + 1, 0), 4);
                    cb |= (uint64_t)((1u << n) - 1u) << (4 * kt);
                }
                ok &= cb;
            }
            const int kend = a.causal ? min(a.Skv, q0 + qt * 16 + 16) : a.Skv;
            // S^T = K Q^T
            f32x4 s[NKT];
            float mx = kNegInf;
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt) {
                s[kt] = f32x4{kNegInf, kNegInf, kNegInf, kNegInf};
                if (kt * 16 < kend) {
                    __builtin_amdgcn_sched_barrier(0);  // bounds the reads in flight (registers)
                    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int i = 0; i < NI; ++i) {
                        const f32x4 kv4 = ld_chunk(lkq, kt * 16 + m, 4 * i + g);
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc = mma_f32(kv4[e], qop[i][e], acc);
                    }
                    const uint32_t w = (uint32_t)(ok >> (4 * kt));
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[i] = ((w >> i) & 1u) ? acc[i] : kNegInf;
                    mx = fmaxf(fmaxf(mx, acc[0]), acc[1]);
                    mx = fmaxf(fmaxf(mx, acc[2]), acc[3]);
                    s[kt] = acc;
                }
            }
            mx = colgroup_max(mx);
            const bool empty = mx == kNegInf;
            const float nbase = empty ? 0.f : -mx * a.c2;
            float sum = 0.f;
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt) {
                if (kt * 16 < kend) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        s[kt][i] = fast_exp2(__builtin_fmaf(s[kt][i], a.c2, nbase));
                        sum += s[kt][i];
                    }
                }
            }
            sum = colgroup_sum(sum);
            const float lse = empty ? kNegInf : mx * a.c2 + __builtin_log2f(sum);
            const float rs = empty ? 0.f : a.scale / sum;
            const float ndelta = empty ? 0.f : -delta;
            if (g == 0) {
                lds_st4(slse + qrow * 4, __builtin_bit_cast(uint32_t, lse));
                lds_st4(sdelta + qrow * 4, __builtin_bit_cast(uint32_t, ndelta));
            }
            // scale * dS^T = P^T (dP^T - delta) * scale, dP^T = V dO^T
            const uint64_t drow = DROP ? (uint64_t)(((int64_t)b * a.H + h) * a.Sq + qabs) * (uint64_t)a.Skv : 0;
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt) {
                if (kt * 16 < kend) {
                    __builtin_amdgcn_sched_barrier(0);
                    f32x4 dp = DROP ? f32x4{0.f, 0.f, 0.f, 0.f} : f32x4{ndelta, ndelta, ndelta, ndelta};
#pragma unroll
                    for (int i = 0; i < NI; ++i) {
                        const f32x4 vv = ld_chunk(lvq, kt * 16 + m, 4 * i + g);
#pragma unroll
                        for (int e = 0; e < 4; ++e) dp = mma_f32(vv[e], doop[i][e], dp);
                    }
                    if constexpr (DROP) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const bool keep = drop_hash(drow + (uint64_t)(kt * 16 + 4 * g + i), a.drop.k0, a.drop.k1) >= a.drop.thresh;
                            dp[i] = __builtin_fmaf(dp[i], keep ? a.drop.scale : 0.f, ndelta);
                        }
                    }
#pragma unroll
                    for (int i = 0; i < 4; ++i) s[kt][i] = s[kt][i] * (rs * dp[i]);
                }
            }
            // dQ^T = K^T (scale * dS^T): k-step (kt, i) covers keys 16kt + 4g' + i
            f32x4 dq[NDT];
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) dq[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt) {
                if (kt * 16 < kend) {
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            dq[dt] = mma_f32(ld_elem(lkq, kt * 16 + 4 * g + i, dcol(dt)), s[kt][i], dq[dt]);
                }
            }
            store_row(rdq, a.dqss, qrow, dq, 1.0f);
        }
        __syncthreads();

        // ---- phase 2: one 16-key tile per wave pass -----------------------------
        auto key_tile = [&](int kt, f32x4 (&dvt)[NDT], f32x4 (&dkt)[NDT]) {
            const int key = kt * 16 + m;
            const bool kok = key < a.Skv && !(prow && prow[key]);
            f32x4 kop[NI], vop[NI];
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                kop[i] = ld_chunk(lk, key, 4 * i + g);
                vop[i] = ld_chunk(lv, key, 4 * i + g);
            }
            bool skip_early = a.causal;
            if (skip_early) {
                bool e = false;
                for (int r = lane; r < RQ; r += 64) e |= __builtin_bit_cast(float, lds_ld4(slse + r * 4)) == kNegInf;
                skip_early = __builtin_amdgcn_ballot_w64(e) == 0;
            }
            // causal: query tiles ending before the key tile add nothing
            for (int qt = skip_early ? max(0, (kt * 16 - q0) / 16) : 0; qt < nqt; ++qt) {
                const f32x4 lse4 = as_f32x4(lds_ld16(slse + (qt * 16 + 4 * g) * 4));
                const f32x4 ndelta4 = as_f32x4(lds_ld16(sdelta + (qt * 16 + 4 * g) * 4));
                f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
                f32x4 dpacc = DROP ? f32x4{0.f, 0.f, 0.f, 0.f} : ndelta4;
#pragma unroll
                for (int i = 0; i < NI; ++i) {
                    const f32x4 qa = ld_chunk(lq, qt * 16 + m, 4 * i + g);
                    const f32x4 da = ld_chunk(ldo, qt * 16 + m, 4 * i + g);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        sacc = mma_f32(qa[e], kop[i][e], sacc);
                        dpacc = mma_f32(da[e], vop[i][e], dpacc);
                    }
                }
                f32x4 ms = f32x4{1.f, 1.f, 1.f, 1.f};  // dropout multiplier of each score
                if constexpr (DROP) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint64_t idx =
                            (uint64_t)(((int64_t)b * a.H + h) * a.Sq + q0 + qt * 16 + 4 * g + i) * (uint64_t)a.Skv + key;
                        ms[i] = drop_hash(idx, a.drop.k0, a.drop.k1) >= a.drop.thresh ? a.drop.scale : 0.f;
                        dpacc[i] = __builtin_fmaf(dpacc[i], ms[i], ndelta4[i]);
                    }
                }
                float p[4], ds[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int q = qt * 16 + 4 * g + i;
                    const bool okq = kok && q < Sqb && (!a.causal || key <= q0 + q);
                    const float pv = fast_exp2(__builtin_fmaf(sacc[i], a.c2, -lse4[i]));
                    p[i] = okq ? (DROP ? pv * ms[i] : pv) : 0.f * lse4[i];  // NaN only for a query that sees no key
                    ds[i] = okq ? pv * dpacc[i] : 0.f;
                }
                // dV^T += dO^T P, dK^T += Q^T dS: k-step i covers queries 16qt + 4g' + i
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) {
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        dvt[dt] = mma_f32(ld_elem(ldo, qt * 16 + 4 * g + i, dcol(dt)), p[i], dvt[dt]);
                        dkt[dt] = mma_f32(ld_elem(lq, qt * 16 + 4 * g + i, dcol(dt)), ds[i], dkt[dt]);
                    }
                }
            }
        };
        if constexpr (LOOP) {
#pragma unroll
            for (int j = 0; j < NSLOT; ++j) {
                const int kt = wave + j * kWaves;
                if (kt < NKT && kt * 16 < a.Skv) key_tile(kt, dvs[j], dks[j]);
            }
        } else {
            for (int kt = wave; kt < NKT; kt += kWaves) {
                if (kt * 16 >= a.Skv) break;
                f32x4 dvt[NDT], dkt[NDT];
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) dvt[dt] = dkt[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
                key_tile(kt, dvt, dkt);
                store_row(rdv, a.dvss, kt * 16 + m, dvt, 1.0f);
                store_row(rdk, a.dkss, kt * 16 + m, dkt, a.scale);
            }
        }
    }
    if constexpr (LOOP) {
#pragma unroll
        for (int j = 0; j < NSLOT; ++j) {
            const int kt = wave + j * kWaves;
            if (kt < NKT && kt * 16 < a.Skv) {
                store_row(rdv, a.dvss, kt * 16 + m, dvs[j], 1.0f);
                store_row(rdk, a.dkss, kt * 16 + m, dks[j], a.scale);
            }
        }
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

// Key chunks the LOOP and fp32 variants are built for: 1, 2, 4 or 8 (keys
// past seq_kv are masked, so rounding up only stages zero rows).
inline int bwd_nkc_pow2(int nkc) { return nkc <= 1 ? 1 : nkc <= 2 ? 2 : nkc <= 4 ? 4 : 8; }

}  // namespace

// Instantiated in atx_attn_bwd_loop.hip (16-bit LOOP), atx_attn_bwd_fp32.hip
// and atx_attn_bwd_fp32_loop.hip.
int dispatch_bwd16_loop(bool bf16, int D, int nkc, int grid, size_t lds, hipStream_t st, const BwdArgs& a);
int dispatch_bwd_fp32(bool loop, int D, int nkc, int grid, size_t lds, hipStream_t st, const BwdArgs& a);
int dispatch_bwd_fp32_loop(int D, int nkc, int grid, size_t lds, hipStream_t st, const BwdArgs& a);
// atx_attn_bwd_drop.hip / atx_attn_bwd_drop_fp32.hip: both variants with
// dropout, head_dim 48 and 64.
int dispatch_bwd_drop(int dtype, bool loop, int D, int nkc, int grid, size_t lds, hipStream_t st, const BwdArgs& a);
int dispatch_bwd_drop_fp32(bool loop, int D, int nkc, int grid, size_t lds, hipStream_t st, const BwdArgs& a);

}  // namespace atx
