// Kernels of the fused attention forward (atx_attn.hip describes the design):
// shared by atx_attn.hip (every head_dim, no dropout) and atx_attn_drop.hip
// (the dropout instantiations).
#pragma once

#include "atx_common.hpp"

namespace atx {

struct AttnArgs {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    int64_t qsb, qss, qsh;
    int64_t ksb, kss, ksh;
    int64_t vsb, vss, vsh;
    int64_t osb, oss, osh;
    const uint8_t* kpad;
    int64_t kpsb;
    int kpad_w4;  // padding rows 4-byte aligned
    int H, group, Sq, Skv, nkt;
    float c2;  // scale * log2(e)
    int causal;
    int xcd_remap;  // H % 8 == 0: rotate heads by batch so each XCD sees all heads
    DropKey drop;   // attention dropout (the DROP instantiations only)
};

constexpr int kThreads = 256;
constexpr int kWaves = 4;

// Padding bytes of keys 4*lane .. 4*lane + 3 (byte i nonzero: key padded
// out), one word per lane, so a wave covers S_kv <= 256.  A 4-byte load when
// the rows are 4-byte aligned, else byte loads.  Issued before the K/V staging
// loads, so its latency overlaps theirs.
__device__ inline uint32_t key_pad_word(const AttnArgs& a, int b, int lane) {
    const uint8_t* row = a.kpad ? a.kpad + (int64_t)b * a.kpsb : nullptr;
    const int key0 = 4 * lane;
    uint32_t pad = 0;
    if (row && key0 < a.Skv) {
        if (a.kpad_w4 && key0 + 4 <= a.Skv) {
            pad = *reinterpret_cast<const uint32_t*>(row + key0);
        } else {
            for (int i = 0; i < 4; ++i)
                if (key0 + i < a.Skv) pad |= (uint32_t)row[key0 + i] << (8 * i);
        }
    }
    return pad;
}

// Per-lane bitmask of usable keys (bit 4*kt + i <-> key 16*kt + 4*g + i):
// inside the key range and not padded out.  Ballot i has bit l set when key
// 4l + i is usable; key 16kt + 4g + i is bit 4kt + g of ballot i.  Called by
// the whole wave.
template <int NKT>
__device__ inline uint64_t key_valid_bits(const AttnArgs& a, int lane, int g, uint32_t pad) {
    uint64_t bal[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) bal[i] = __ballot(4 * lane + i < a.Skv && ((pad >> (8 * i)) & 0xffu) == 0);
    uint64_t bits = 0;
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) bits |= ((bal[i] >> (4 * kt + g)) & 1ull) << (4 * kt + i);
    return bits;
}

// Waves per SIMD that the register allocator is asked to fit, per kernel
// family (16-bit plain / masked, fp32), head_dim (rows: 16, 32, 48, 64, 80,
// 96, 112, 128) and 32-key chunk count (columns: NKC = 1..8).  Each entry is
// the highest target for which hipcc (ROCm 7.2, gfx950) produced the kernel
// (bf16 and fp16) without register spills; the AMDGPU scheduler
// is not monotonic in this target (a looser budget can make it hoist loads
// far enough to spill), so the values were found by compiling every
// instantiation at every target, not by a formula.
constexpr int kOcc16[4][8][8] = {
    {
        {8, 8, 8, 8, 8, 7, 6, 5},
        {8, 8, 8, 8, 8, 7, 6, 5},
        {8, 8, 8, 8, 7, 6, 5, 5},
        {8, 8, 7, 7, 6, 5, 5, 4},
        {8, 7, 7, 6, 6, 5, 5, 4},
        {7, 7, 6, 6, 5, 5, 5, 4},
        {6, 5, 5, 5, 5, 5, 4, 4},
        {5, 5, 4, 4, 4, 4, 4, 4},
    },
    {
        {8, 8, 8, 8, 8, 7, 6, 5},
        {8, 8, 8, 8, 8, 7, 6, 5},
        {8, 8, 8, 8, 7, 6, 5, 5},
        {8, 8, 8, 7, 6, 5, 5, 4},
        {8, 7, 6, 6, 5, 5, 4, 4},
        {8, 6, 6, 6, 5, 5, 4, 4},
        {7, 5, 5, 5, 4, 4, 4, 4},
        {5, 5, 4, 4, 4, 4, 4, 4},
    },
    {
        {8, 8, 8, 8, 8, 6, 5, 4},
        {8, 8, 8, 8, 7, 6, 5, 4},
        {8, 8, 8, 8, 7, 6, 5, 4},
        {8, 8, 7, 7, 6, 5, 5, 4},
        {8, 8, 7, 7, 6, 5, 5, 4},
        {7, 7, 6, 6, 5, 4, 4, 4},
        {6, 6, 6, 5, 5, 5, 4, 4},
        {5, 4, 4, 4, 4, 4, 4, 4},
    },
    {
        {8, 8, 8, 8, 7, 6, 5, 4},
        {8, 8, 8, 8, 6, 5, 5, 4},
        {8, 8, 8, 7, 5, 5, 4, 4},
        {8, 8, 8, 6, 5, 5, 4, 4},
        {8, 8, 7, 5, 5, 5, 4, 4},
        {8, 7, 6, 6, 5, 5, 4, 4},
        {7, 5, 5, 5, 5, 4, 4, 4},
        {5, 5, 4, 4, 4, 4, 4, 3},
    },
};
constexpr int kOcc32[8][8] = {
    {8, 8, 7, 5, 4, 4, 3, 3},
    {8, 8, 6, 4, 4, 4, 3, 3},
    {8, 7, 5, 4, 4, 3, 3, 3},
    {8, 7, 5, 4, 4, 3, 3, 2},
    {8, 6, 5, 4, 4, 3, 3, 2},
    {8, 6, 5, 4, 3, 3, 3, 2},
    {7, 5, 4, 4, 3, 3, 3, 2},
    {7, 5, 4, 4, 3, 3, 2, 2},
};
// The dropout instantiations carry the keep-mask hashing on top: a lower
// target (one wave per SIMD fewer, at least 2) keeps them free of spills.
template <int D, int NKC, bool MASKED, bool FULL, bool DROP = false>
constexpr int occ_16bit() {
    return DROP ? (kOcc16[(MASKED ? 2 : 0) + (FULL ? 1 : 0)][D / 16 - 1][NKC - 1] > 3
                       ? kOcc16[(MASKED ? 2 : 0) + (FULL ? 1 : 0)][D / 16 - 1][NKC - 1] - 1 : 2)
                : kOcc16[(MASKED ? 2 : 0) + (FULL ? 1 : 0)][D / 16 - 1][NKC - 1];
}
template <int D, int NKC, bool DROP = false>
constexpr int occ_fp32() {
    return DROP ? (kOcc32[D / 16 - 1][NKC - 1] > 3 ? kOcc32[D / 16 - 1][NKC - 1] - 1 : 2) : kOcc32[D / 16 - 1][NKC - 1];
}

// K rows: XOR-swizzled 16-byte chunks when a row has 8 or 16 of them, else
// padded by one chunk.  Output stores go through LDS for D = 64 and 128
// (rows of whole 128-byte lines).
template <int D>
constexpr bool kKeySwizzle = (D == 64 || D == 128);
template <int D>
constexpr int K_row_bytes() {
    return kKeySwizzle<D> ? D * 2 : D * 2 + 16;
}
template <int D>
constexpr bool kStagedStores = (D == 64 || D == 128);

// ---------------------------------------------------------------------------
// 16-bit inputs (bf16 / fp16).  NKC = number of 32-key chunks (S_kv <= 32*NKC);
// FULL = the last 16-key tile of the last chunk exists (S_kv > 32*NKC - 16),
// so the number of key tiles is a compile-time constant; MASKED selects the
// variant with causal / key-padding masks, so the plain kernel carries no
// per-element mask work beyond the key bound of its last tile.
// ---------------------------------------------------------------------------
template <typename T, int D, int NKC, bool MASKED, bool FULL, bool DROP = false>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(occ_16bit<D, NKC, MASKED, FULL, DROP>(), 8)))
void attn_fwd_16bit(AttnArgs a) {
    using M = Mfma16<T>;
    constexpr int CH = D / 8;          // 16-byte chunks per row
    constexpr int NI = (D + 31) / 32;  // QK^T MFMAs per 16x16 tile
    constexpr int NDT = D / 16;        // PV output tiles
    constexpr int QD = D / 4;          // contiguous outputs per lane
    constexpr int NKT = FULL ? 2 * NKC : 2 * NKC - 1;  // key tiles
    constexpr int ROWS = NKT * 16;     // K / V rows staged
    constexpr bool KSWZ = kKeySwizzle<D>;   // K rows XOR-swizzled instead of padded
    constexpr int RSK = K_row_bytes<D>();   // K row stride in LDS (bytes)
    constexpr int RSV = D * 2;              // V row stride in LDS (bytes, 8-byte units swizzled)
    constexpr bool STAGE_OUT = kStagedStores<D>;  // whole-line output stores through LDS
    constexpr int OROWS = 8;                // output rows staged per round
    constexpr int KIT = (ROWS * CH + kThreads - 1) / kThreads;

    lds_t* const sk = lds_base();
    lds_t* const sv = sk + ROWS * RSK;
    lds_t* const so = sv + ROWS * RSV;  // per-wave output staging (STAGE_OUT)

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int m = lane & 15, g = lane >> 4;
    // Workgroups are dispatched round-robin over the 8 XCDs, so with H a
    // multiple of 8 workgroup b*H + h would always land on XCD h % 8 (one
    // head slice per XCD: measured 10-15 % slower).  Rotating the head by the
    // batch index gives every XCD every head.
    const int bh = blockIdx.x;
    const int b = bh / a.H;
    int h = bh - b * a.H;
    if (a.xcd_remap) {
        h += b & 7;
        if (h >= a.H) h -= a.H;
    }
    const int hk = h / a.group;
    const int qss = (int)a.qss, kss = (int)a.kss, vss = (int)a.vss, oss = (int)a.oss;

    // One buffer descriptor per tensor slice of this (batch, head); each ends
    // at the last valid row, so rows past S_q / S_kv read as zero and output
    // rows past S_q are not written.
    const rsrc_t rk = make_rsrc(static_cast<const T*>(a.k) + b * a.ksb + hk * a.ksh, ((a.Skv - 1) * kss + D) * 2);
    const rsrc_t rv = make_rsrc(static_cast<const T*>(a.v) + b * a.vsb + hk * a.vsh, ((a.Skv - 1) * vss + D) * 2);
    const rsrc_t rq = make_rsrc(static_cast<const T*>(a.q) + b * a.qsb + h * a.qsh, ((a.Sq - 1) * qss + D) * 2);
    const rsrc_t ro = make_rsrc(static_cast<T*>(a.o) + b * a.osb + h * a.osh, ((a.Sq - 1) * oss + D) * 2);
    T* ob = static_cast<T*>(a.o) + b * a.osb + h * a.osh;

    const int nqt = (a.Sq + 15) >> 4;

    // Q operand (B of S^T = K Q^T): lane (m, g) holds chunk 4i+g of query row m.
    auto load_q = [&](int qt, u32x4 (&qop)[NI]) {
        const uint32_t qrow = qt * 16 + m;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int c = 4 * i + g;
            qop[i] = (CH % 4 == 0 || c < CH) ? buf_ld16(rq, (qrow * qss + c * 8) * 2) : u32x4{0, 0, 0, 0};
        }
    };
    u32x4 qop[NI];
    if (wave < nqt) load_q(wave, qop);

    const uint32_t padw = MASKED ? key_pad_word(a, b, lane) : 0u;

    // ---- stage K and V rows 0 .. ROWS-1 (rows past S_kv read as zero:
    //      padded keys are masked by the -inf bias, padded values meet P = 0)
    u32x4 kreg[KIT], vreg[KIT];
#pragma unroll
    for (int it = 0; it < KIT; ++it) {
        const int idx = tid + it * kThreads;
        const uint32_t r = idx / CH, c = idx - r * CH;
        kreg[it] = buf_ld16(rk, (r * kss + c * 8) * 2);
        vreg[it] = buf_ld16(rv, (r * vss + c * 8) * 2);
    }
    // K: with 8 or 16 chunks per row the 16-byte chunk c of row r sits at
    // c ^ ((r >> 1) & 7); otherwise rows are padded to an odd number of 16-byte
    // units.  Either way the 16 rows of one MFMA operand read fall in distinct
    // bank groups.  V: the 8-byte units of row r sit at unit ^ s(r),
    // s(r) = ((r >> 1) ^ r) & 3, so the transposing reads below touch distinct
    // bank pairs.
#pragma unroll
    for (int it = 0; it < KIT; ++it) {
        const int idx = tid + it * kThreads;
        if ((ROWS * CH) % kThreads == 0 || idx < ROWS * CH) {
            const int r = idx / CH, c = idx - r * CH;
            const int pc = KSWZ ? (c ^ ((r >> 1) & 7)) : c;
            lds_st16(sk + r * RSK + pc * 16, kreg[it]);
            const int sw = ((r >> 1) ^ r) & 3;
            lds_t* row = sv + r * RSV;
            lds_st8(row + (((2 * c) ^ sw) << 3), u32x2{vreg[it][0], vreg[it][1]});
            lds_st8(row + (((2 * c + 1) ^ sw) << 3), u32x2{vreg[it][2], vreg[it][3]});
        }
    }

    uint64_t kbits = 0;
    if constexpr (MASKED) kbits = key_valid_bits<NKT>(a, lane, g, padw);
    const float c2 = a.c2;
    const float kNegInf = -__builtin_inff();
    // Keys at or past S_kv can only sit in the last tile (S_kv > 16*(NKT-1)):
    // an additive 0 / -inf bias per lane masks them with one add per score.
    float kbias[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) kbias[i] = ((NKT - 1) * 16 + 4 * g + i < a.Skv) ? 0.f : kNegInf;

    // Per-lane LDS addresses, fixed for the whole workgroup; tile, chunk and
    // half offsets are compile-time and fold into the instructions' offsets.
    //  K operand: row m of each 16-key tile, chunk 4i+g (swizzled).
    //  V^T operand (ds_read_b64_tr_b16): input lane i = a4 + 4t of a 16-lane
    //  group points at row 4g + t (+32c + 16h) and columns a4*QD + 4dt..+3;
    //  the read hands lane m the four keys of its group for head-dim
    //  (m/4)*QD + 4dt + m%4.
    lds_t* k_lane[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int c = 4 * i + g;
        k_lane[i] = sk + m * RSK + (KSWZ ? (c ^ ((m >> 1) & 7)) : c) * 16;
    }
    const int tr_row = 4 * g + (m >> 2);
    const int tr_sw = ((tr_row >> 1) ^ tr_row) & 3;
    lds_t* v_lane[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) v_lane[dt] = sv + tr_row * RSV + ((((m & 3) * NDT + dt) ^ tr_sw) << 3);
    lds_t* const o_wave = so + wave * (OROWS * 2 * D);
    lds_t* o_put = o_wave + (m & 7) * (2 * D) + g * (QD * 2);
    const uint32_t ones = M::kOnes2;
    __syncthreads();

    for (int qt = wave; qt < nqt; qt += kWaves) {
        const int qrow = qt * 16 + m;
        // The asm barrier below makes every LDS address look new on each
        // pass, so the compiler cannot hoist the (loop-invariant) operand reads
        // of all tiles out of the loop, which would need far more registers.
        lds_t* kl[NI];
        lds_t* vl[NDT];
#pragma unroll
        for (int i = 0; i < NI; ++i) kl[i] = lds_opaque(k_lane[i]);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) vl[dt] = lds_opaque(v_lane[dt]);

        // ---- S^T = K Q^T over the key tiles -------------------------------
        f32x4 s[NKT];
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt) {
            f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                u32x4 kop = lds_ld16(kl[i] + kt * 16 * RSK);
                if (CH % 4 != 0 && 4 * i + g >= CH) kop = u32x4{0, 0, 0, 0};
                acc = M::mma(kop, qop[i], acc);
            }
            s[kt] = acc;
        }
        if (qt + kWaves < nqt) load_q(qt + kWaves, qop);
        // Phase fence: keeps the PV operand reads below the softmax.
        __builtin_amdgcn_sched_barrier(0);

        // ---- mask -----------------------------------------------------------
        if constexpr (MASKED) {
            // Usable-key bits of this query row: padding / range bits, and
            // under causal masking keys 16kt + 4g + i <= qrow, i.e. the low
            // clamp(qrow - 16kt - 4g + 1, 0, 4) bits of nibble kt.  Each score
            // is then kept or replaced by -inf with a bitwise select on its
            // sign-extended bit (no per-element compare masks).
            uint64_t ok = kbits;
            if (a.causal) {
                uint64_t cb = 0;
#pragma unroll
                for (int kt = 0; kt < NKT; ++kt) {
                    const int n = min(max((int)qrow - (kt * 16 + 4 * g) + 1, 0), 4);
                    cb |= (uint64_t)((1u << n) - 1u) << (4 * kt);
                }
                ok &= cb;
            }
            const uint32_t ok_lo = (uint32_t)ok, ok_hi = (uint32_t)(ok >> 32);
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt) {
                u32x4 bits = __builtin_bit_cast(u32x4, s[kt]);  // whole-vector casts only
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int pos = 4 * kt + i;
                    const uint32_t word = pos < 32 ? ok_lo : ok_hi;
                    const uint32_t keep = (uint32_t)((int32_t)(word << (31 - (pos & 31))) >> 31);
                    bits[i] = (bits[i] & keep) | (0xff800000u & ~keep);
                }
                s[kt] = __builtin_bit_cast(f32x4, bits);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) s[NKT - 1][i] += kbias[i];
        }

        // ---- single-pass softmax over the whole key row ---------------------
        float mx = kNegInf;
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[kt][i]);
        mx = colgroup_max(mx);
        // A fully masked row has mx = -inf; -mb = +inf then makes every
        // exponent NaN, which is what softmax over an all -inf row returns.
        const float mb = mx * c2;
        u32x4 pk[NKC];
#pragma unroll
        for (int c = 0; c < NKC; ++c) {
            float p[8];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    p[4 * hh + i] = (2 * c + hh < NKT) ? fast_exp2(__builtin_fmaf(s[(2 * c + hh) % NKT][i], c2, -mb)) : 0.f;
            pk[c] = u32x4{M::pack2(p[0], p[1]), M::pack2(p[2], p[3]), M::pack2(p[4], p[5]), M::pack2(p[6], p[7])};
        }
        __builtin_amdgcn_sched_barrier(0);

        // ---- O^T = V^T P^T, and the row sums as ones^T P^T ------------------
        f32x4 lsum4 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NKC; ++c) lsum4 = M::mma(u32x4{ones, ones, ones, ones}, pk[c], lsum4);
        if constexpr (DROP) {
            // Dropout after the softmax (its sums above are over every
            // weight): zero the dropped 16-bit weights; 1 / (1 - p) joins the
            // normalisation.  Lane (m, g) holds query qrow against keys
            // 16 kt + 4g + i, kt = 2c + hh, packed two per word.
            const uint64_t rowbase = (uint64_t)(((int64_t)b * a.H + h) * a.Sq + qrow) * (uint64_t)a.Skv;
#pragma unroll
            for (int c = 0; c < NKC; ++c)
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const uint64_t key = (uint64_t)(16 * (2 * c + (w >> 1)) + 4 * g + 2 * (w & 1));
                    const uint32_t lo = drop_hash(rowbase + key, a.drop.k0, a.drop.k1) >= a.drop.thresh ? 0xFFFFu : 0u;
                    const uint32_t hi = drop_hash(rowbase + key + 1, a.drop.k0, a.drop.k1) >= a.drop.thresh ? 0xFFFF0000u : 0u;
                    pk[c][w] &= lo | hi;
                }
        }
        f32x4 oacc[NDT];
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
            oacc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < NKC; ++c) {
                const u32x2 lo = lds_ld8_tr16(vl[dt] + (32 * c) * RSV);
                // A missing last tile has P = 0 and no V rows.
                const u32x2 hi = (2 * c + 1 < NKT) ? lds_ld8_tr16(vl[dt] + (32 * c + 16) * RSV) : u32x2{0u, 0u};
                oacc[dt] = M::mma(u32x4{lo[0], lo[1], hi[0], hi[1]}, pk[c], oacc[dt]);
            }
        }

        // ---- normalise; store D/4 contiguous outputs per lane, or (D = 64,
        //      128) through a per-wave LDS tile so every store instruction
        //      writes whole 128-byte rows with the streaming hint ------------
        const float inv = DROP ? fast_rcp(lsum4[0]) * a.drop.scale : fast_rcp(lsum4[0]);
        if constexpr (STAGE_OUT) {
            lds_t* const put = lds_opaque(o_put);
            lds_t* const tile = lds_opaque(o_wave);
            u32x4 w[NDT / 2];
#pragma unroll
            for (int dt = 0; dt < NDT; dt += 2)
                w[dt / 2] = u32x4{M::pack2(oacc[dt][0] * inv, oacc[dt][1] * inv),
                                  M::pack2(oacc[dt][2] * inv, oacc[dt][3] * inv),
                                  M::pack2(oacc[dt + 1][0] * inv, oacc[dt + 1][1] * inv),
                                  M::pack2(oacc[dt + 1][2] * inv, oacc[dt + 1][3] * inv)};
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                if ((m >> 3) == j) {
#pragma unroll
                    for (int dt = 0; dt < NDT; dt += 2) lds_st16(put + dt * 8, w[dt / 2]);
                }
                wave_lds_handoff();  // the reads below see the writes above
#pragma unroll
                for (int k = 0; k < CH / 8; ++k) {
                    const int idx = lane + 64 * k;
                    const uint32_t row = idx / CH, c = idx - row * CH;
                    const u32x4 v = lds_ld16(tile + row * (2 * D) + c * 16);
                    buf_st16(ro, ((qt * 16 + OROWS * j + row) * oss + c * 8) * 2, v);
                }
                wave_lds_handoff();  // the next round's writes follow these reads
            }
        } else if (qrow < a.Sq) {
            T* orow = ob + qrow * oss + g * QD;
            if constexpr (QD % 8 == 0) {
#pragma unroll
                for (int dt = 0; dt < NDT; dt += 2) {
                    const u32x4 w = {M::pack2(oacc[dt][0] * inv, oacc[dt][1] * inv),
                                     M::pack2(oacc[dt][2] * inv, oacc[dt][3] * inv),
                                     M::pack2(oacc[dt + 1][0] * inv, oacc[dt + 1][1] * inv),
                                     M::pack2(oacc[dt + 1][2] * inv, oacc[dt + 1][3] * inv)};
                    st16(orow + dt * 4, w);
                }
            } else {
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) {
                    const u32x2 w = {M::pack2(oacc[dt][0] * inv, oacc[dt][1] * inv),
                                     M::pack2(oacc[dt][2] * inv, oacc[dt][3] * inv)};
                    st8(orow + dt * 4, w);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// fp32 inputs: v_mfma_f32_16x16x4_f32 keeps full fp32 products.  K operands
// come straight from global memory (L1/L2); only V^T is staged in LDS.
// ---------------------------------------------------------------------------
template <int D, int NKC, bool DROP = false>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(occ_fp32<D, NKC, DROP>(), 8)))
void attn_fwd_fp32(AttnArgs a) {
    constexpr int CH = D / 4;    // 16-byte chunks (4 floats) per row
    constexpr int NI = D / 16;   // chunk groups per 16x16 tile
    constexpr int NDT = D / 16;
    constexpr int QD = D / 4;
    constexpr int NKT = 2 * NKC;
    constexpr int NB = (8 * NKC <= 16) ? 16 : (8 * NKC <= 32 ? 32 : 64);  // 4-key blocks per V^T row
    constexpr int RSV = NB * 16;

    lds_t* const svt = lds_base();

    const int nkt = a.nkt;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int m = lane & 15, g = lane >> 4;
    const int bh = blockIdx.x;
    const int b = bh / a.H, h = bh - b * a.H;
    const uint32_t padw = key_pad_word(a, b, lane);  // loaded ahead of the staging (0 without a mask)
    const int hk = h / a.group;

    const float* kb = static_cast<const float*>(a.k) + b * a.ksb + hk * a.ksh;
    const float* vb = static_cast<const float*>(a.v) + b * a.vsb + hk * a.vsh;
    const float* qb = static_cast<const float*>(a.q) + b * a.qsb + h * a.qsh;
    float* ob = static_cast<float*>(a.o) + b * a.osb + h * a.osh;

    // ---- stage V^T: task = (4-key quad, 4-wide d chunk) ------------------
    constexpr int VT = 8 * NKC * CH;
    const int nkq = 4 * nkt;  // quads that the PV loop reads
    for (int t = tid; t < VT; t += kThreads) {
        const int dc = t % CH, kq = t / CH;
        if (kq >= nkq) continue;
        u32x4 x[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int key = 4 * kq + j;
            x[j] = key < a.Skv ? ld16(vb + key * a.vss + dc * 4) : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int d = dc * 4 + e;
            const int hd = ((d / QD) << 2) | (d & 3);
            const u32x4 col = {x[0][e], x[1][e], x[2][e], x[3][e]};
            lds_st16(svt + d * RSV + ((kq ^ hd) << 4), col);
        }
    }
    const bool masked_path = a.causal || a.kpad != nullptr;
    uint64_t kbits = 0;
    if (masked_path) kbits = key_valid_bits<NKT>(a, lane, g, padw);
    __syncthreads();

    const float c2 = a.c2;
    const float kNegInf = -__builtin_inff();
    const int nqt = (a.Sq + 15) >> 4;

    for (int qt = wave; qt < nqt; qt += kWaves) {
        const int qrow = qt * 16 + m;
        lds_t* const svq = lds_opaque(svt);
        u32x4 qop[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i)
            qop[i] = qrow < a.Sq ? ld16(qb + qrow * a.qss + (4 * i + g) * 4) : u32x4{0, 0, 0, 0};

        f32x4 s[NKT];
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt) {
            s[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (kt < nkt) {
                int krow = kt * 16 + m;
                krow = krow < a.Skv ? krow : a.Skv - 1;  // rows past the end are masked below
#pragma unroll
                for (int i = 0; i < NI; ++i) {
                    const f32x4 kop = as_f32x4(ld16(kb + krow * a.kss + (4 * i + g) * 4));
                    const f32x4 qv = as_f32x4(qop[i]);
#pragma unroll
                    for (int j = 0; j < 4; ++j) s[kt] = mma_f32(kop[j], qv[j], s[kt]);
                }
            }
        }

#pragma unroll
        for (int kt = 0; kt < NKT; ++kt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = kt * 16 + 4 * g + i;
                bool ok = key < a.Skv;
                if (masked_path) {
                    ok = (kbits >> (4 * kt + i)) & 1;
                    if (a.causal) ok = ok && key <= qrow;
                }
                s[kt][i] = ok ? s[kt][i] : kNegInf;
            }
        }

        float mx = kNegInf;
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[kt][i]);
        mx = colgroup_max(mx);
        const float mb = mx * c2;
        float lsum = 0.f;
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float e = fast_exp2(__builtin_fmaf(s[kt][i], c2, -mb));
                if (kt >= nkt) e = 0.f;
                s[kt][i] = e;
                lsum += e;
            }
        lsum = colgroup_sum(lsum);
        if constexpr (DROP) {
            // Dropout after the softmax: zero the dropped weights (the sum
            // above covers every weight); 1 / (1 - p) joins the division.
            const uint64_t rowbase = (uint64_t)(((int64_t)b * a.H + h) * a.Sq + qrow) * (uint64_t)a.Skv;
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (drop_hash(rowbase + (uint64_t)(kt * 16 + 4 * g + i), a.drop.k0, a.drop.k1) < a.drop.thresh) s[kt][i] = 0.f;
        }
        __builtin_amdgcn_sched_barrier(0);

        f32x4 oacc[NDT];
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
            oacc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
            const int d = (m >> 2) * QD + dt * 4 + (m & 3);
            const lds_t* vrow = svq + d * RSV;
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt) {
                if (kt < nkt) {
                    const f32x4 vop = as_f32x4(lds_ld16(vrow + (((4 * kt + g) ^ m) << 4)));
#pragma unroll
                    for (int i = 0; i < 4; ++i) oacc[dt] = mma_f32(vop[i], s[kt][i], oacc[dt]);
                }
            }
        }

        if (qrow < a.Sq) {
            // Exact division keeps the fp32 path within a few ulp of the
            // reference's softmax normalisation.
            float* orow = ob + qrow * a.oss + g * QD;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
                f32x4 r = {oacc[dt][0] / lsum, oacc[dt][1] / lsum, oacc[dt][2] / lsum, oacc[dt][3] / lsum};
                if constexpr (DROP) r *= a.drop.scale;
                st16(orow + dt * 4, __builtin_bit_cast(u32x4, r));
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Launch and per-head_dim dispatch templates
// ---------------------------------------------------------------------------
template <typename Kernel>
int launch(Kernel kernel, int grid, size_t lds, hipStream_t stream, const AttnArgs& args) {
    if (lds > 64 * 1024) {
        // Above the 64 KiB default the dynamic LDS size must be raised per kernel.
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) ATX_FAIL(ATX_ERR_LAUNCH, "hipFuncSetAttribute(%zu bytes LDS): %s", lds, hipGetErrorString(e));
    }
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kThreads), lds, stream, args);
    ATX_CHECK_LAUNCH("atx_attn_fwd launch");
    return ATX_OK;
}

template <typename T, int D, bool MASKED, bool FULL, bool DROP = false>
int dispatch_16bit_mode(int nkc, int grid, size_t lds, hipStream_t st, const AttnArgs& a) {
    switch (nkc) {
        case 1: return launch(attn_fwd_16bit<T, D, 1, MASKED, FULL, DROP>, grid, lds, st, a);
        case 2: return launch(attn_fwd_16bit<T, D, 2, MASKED, FULL, DROP>, grid, lds, st, a);
        case 3: return launch(attn_fwd_16bit<T, D, 3, MASKED, FULL, DROP>, grid, lds, st, a);
        case 4: return launch(attn_fwd_16bit<T, D, 4, MASKED, FULL, DROP>, grid, lds, st, a);
        case 5: return launch(attn_fwd_16bit<T, D, 5, MASKED, FULL, DROP>, grid, lds, st, a);
        case 6: return launch(attn_fwd_16bit<T, D, 6, MASKED, FULL, DROP>, grid, lds, st, a);
        case 7: return launch(attn_fwd_16bit<T, D, 7, MASKED, FULL, DROP>, grid, lds, st, a);
        case 8: return launch(attn_fwd_16bit<T, D, 8, MASKED, FULL, DROP>, grid, lds, st, a);
    }
    ATX_FAIL(ATX_ERR_UNSUPPORTED, "seq_kv chunk count %d", nkc);
}

template <typename T, int D, bool DROP = false>
int dispatch_16bit(int nkc, int grid, hipStream_t st, const AttnArgs& a) {
    const size_t k_lds = (size_t)a.nkt * 16 * K_row_bytes<D>();
    const size_t v_lds = (size_t)a.nkt * 16 * D * 2;
    const size_t o_lds = kStagedStores<D> ? (size_t)kWaves * 8 * D * 2 : 0;
    const size_t lds = k_lds + v_lds + o_lds;
    const bool masked = a.causal || a.kpad;
    const bool full = a.nkt == 2 * nkc;
    if (masked) {
        return full ? dispatch_16bit_mode<T, D, true, true, DROP>(nkc, grid, lds, st, a)
                    : dispatch_16bit_mode<T, D, true, false, DROP>(nkc, grid, lds, st, a);
    }
    return full ? dispatch_16bit_mode<T, D, false, true, DROP>(nkc, grid, lds, st, a)
                : dispatch_16bit_mode<T, D, false, false, DROP>(nkc, grid, lds, st, a);
}

template <int D, bool DROP = false>
int dispatch_fp32(int nkc, int grid, hipStream_t st, const AttnArgs& a) {
    const int nb = (8 * nkc <= 16) ? 16 : (8 * nkc <= 32 ? 32 : 64);
    const size_t lds = (size_t)D * nb * 16;
    switch (nkc) {
        case 1: return launch(attn_fwd_fp32<D, 1, DROP>, grid, lds, st, a);
        case 2: return launch(attn_fwd_fp32<D, 2, DROP>, grid, lds, st, a);
        case 3: return launch(attn_fwd_fp32<D, 3, DROP>, grid, lds, st, a);
        case 4: return launch(attn_fwd_fp32<D, 4, DROP>, grid, lds, st, a);
        case 5: return launch(attn_fwd_fp32<D, 5, DROP>, grid, lds, st, a);
        case 6: return launch(attn_fwd_fp32<D, 6, DROP>, grid, lds, st, a);
        case 7: return launch(attn_fwd_fp32<D, 7, DROP>, grid, lds, st, a);
        case 8: return launch(attn_fwd_fp32<D, 8, DROP>, grid, lds, st, a);
    }
    ATX_FAIL(ATX_ERR_UNSUPPORTED, "seq_kv chunk count %d", nkc);
}

// atx_attn_drop.hip: the dropout instantiations (head_dim 48 and 64).
int dispatch_fwd_drop(int dtype, int D, int nkc, int grid, hipStream_t st, const AttnArgs& a);

}  // namespace atx
