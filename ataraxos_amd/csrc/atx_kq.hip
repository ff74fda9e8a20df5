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
// the four consecutive to-squares 16*jt + 4g .. +3.  The four waves of a
// workgroup split the tile rows and keep their logits in registers across
// the two block reductions (max, sum), so the logits are never written to
// memory.  LDS holds first the K and Q rows of a 128-byte feature slice and
// the sample's legality bytes, then the finished S*S fp32 row, which leaves
// as one contiguous run of 16-byte stores.
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
    int B, S, nchunks;  // nchunks: 16-byte chunks per q/k row
    float scale, c2;
    int probs;
    int mask_lin;  // a sample's legality bytes are S*S contiguous bytes, 16-byte aligned, S % 4 == 0
    int out_vec;   // a sample's output starts 16-byte aligned and S*S % 4 == 0
};

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kSliceChunks = 8;  // 16-byte chunks per staged slice = one 128-byte LDS row

// One 128-byte feature slice of a 16x16 tile: two 16-byte operand chunks per
// lane for each of A (K rows) and B (Q rows).
template <typename T>
struct KqMma {
    __device__ static inline f32x4 slice(const u32x4 (&a)[2], const u32x4 (&b)[2], f32x4 acc) {
        acc = Mfma16<T>::mma(a[0], b[0], acc);
        return Mfma16<T>::mma(a[1], b[1], acc);
    }
};

template <>
struct KqMma<float> {
    __device__ static inline f32x4 slice(const u32x4 (&a)[2], const u32x4 (&b)[2], f32x4 acc) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const f32x4 fa = as_f32x4(a[i]), fb = as_f32x4(b[i]);
#pragma unroll
            for (int j = 0; j < 4; ++j) acc = mma_f32(fa[j], fb[j], acc);
        }
        return acc;
    }
};

}  // namespace

// LDS bytes for one workgroup: the K and Q rows of one 128-byte feature slice
// plus the legality bytes [S][SP] (SP = S rounded up to 4), or the finished
// values [S][SP] fp32, whichever is larger (they reuse one region).
inline int kq_lds_bytes(int nt, int S) {
    const int SP = (S + 3) & ~3;
    const int staged = 2 * nt * 16 * 128 + ((S * SP + 15) & ~15);
    const int out = S * SP * 4;
    return staged > out ? staged : out;
}

// One workgroup per sample; NT = number of 16-square tiles per side
// (S <= 16*NT); MULTI = features wider than one 128-byte slice; PROBS =
// softmax output (else masked logits).
//
// Wave w owns the tile rows it = w, w + 4, ... (R of them) and every tile
// column jt, and keeps their logits in registers (tile (r, jt) of the wave
// in acc[r][jt]).  The max and the sum of the softmax are reduced as trees
// in registers, then across the waves; the finished values go through LDS
// so that the sample's S*S row leaves as contiguous 16-byte stores.
template <typename T, int NT, bool MULTI, bool PROBS>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(MULTI ? 2 : 4, 8)))
void kq_policy(KqArgs a) {
    constexpr int R = (NT + kWaves - 1) / kWaves;
    constexpr int ROWS = NT * 16;
    constexpr int QKC = ROWS * kSliceChunks;               // chunks per tensor and slice
    constexpr int QIT = (QKC + kThreads - 1) / kThreads;   // per thread
    constexpr int MIT = (ROWS * ROWS / 16 + kThreads - 1) / kThreads;  // legality chunks per thread
    constexpr int MG = (ROWS * ROWS / 4 + 1 + kThreads - 1) / kThreads;  // legality words per thread (grouped)
    constexpr int NLB = (R * NT * 4 + 31) / 32;

    lds_t* const sk = lds_base();
    lds_t* const sq = sk + ROWS * 128;
    lds_t* const smask = sq + ROWS * 128;
    lds_t* const sout = sk;  // after the products and the legality reads
    __shared__ float red[kWaves];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: tile rows stay scalar
    const int m = lane & 15, g = lane >> 4;
    const int b = blockIdx.x;
    const int S = a.S;
    const int SP = (S + 3) & ~3;
    const int nslices = (a.nchunks + kSliceChunks - 1) / kSliceChunks;
    constexpr int es = sizeof(T);
    const uint32_t row_bytes = (uint32_t)a.nchunks * 16;
    const uint32_t qrs = (uint32_t)(a.qss * es), krs = (uint32_t)(a.kss * es);
    // rows past S read as zero: the descriptors end at the last row
    const rsrc_t rq = make_rsrc(static_cast<const T*>(a.q) + b * a.qsb, (uint32_t)((S - 1) * a.qss * es) + row_bytes);
    const rsrc_t rk = make_rsrc(static_cast<const T*>(a.k) + b * a.ksb, (uint32_t)((S - 1) * a.kss * es) + row_bytes);
    const float kNegInf = -__builtin_inff();

    // ---- slice sc of Q and K (and, with the first, the legality bytes) ->
    //      LDS.  Chunk c of row r sits at c ^ ((r >> 1) & 7): the 16 rows one
    //      MFMA operand read touches fall in distinct bank groups. ----------
    // Legality with contiguous rows that are not 16-byte aligned (S % 4 != 0,
    // as at the reference's 101 squares): the sample's S*S bytes in groups of
    // 4, group k = bytes 4k - sh .. 4k - sh + 3 with sh the base's
    // misalignment, so that each group is one aligned 4-byte load (the two
    // partial groups at the ends load bytes); the bytes are then placed in
    // the [S][SP] LDS rows.  (One byte load per square was the cost.)
    const uint8_t* const mbase = a.mask ? a.mask + b * a.msb : nullptr;
    const bool grouped = mbase && !a.mask_lin && a.mss == S;  // (uniform)
    const int msh = (int)((uintptr_t)mbase & 3);
    auto stage = [&](int sc) {
        u32x4 qv[QIT], kv[QIT], mv[MIT];
#pragma unroll
        for (int it = 0; it < QIT; ++it) {
            const uint32_t idx = tid + it * kThreads;
            const uint32_t r = idx >> 3, c = sc * kSliceChunks + (idx & 7);
            const bool in = (int)c < a.nchunks;
            qv[it] = in ? buf_ld16(rq, r * qrs + c * 16) : u32x4{0, 0, 0, 0};
            kv[it] = in ? buf_ld16(rk, r * krs + c * 16) : u32x4{0, 0, 0, 0};
        }
        const bool lin = sc == 0 && a.mask && a.mask_lin;
        if (lin) {
            const rsrc_t rm = make_rsrc(a.mask + b * a.msb, (uint32_t)(S * S));
#pragma unroll
            for (int it = 0; it < MIT; ++it) mv[it] = buf_ld16(rm, (tid + it * kThreads) * 16);  // past S*S: zero
        }
        if (sc) __syncthreads();  // the previous slice's operand reads are done
#pragma unroll
        for (int it = 0; it < QIT; ++it) {
            const uint32_t idx = tid + it * kThreads;
            if (QKC % kThreads == 0 || idx < QKC) {
                const uint32_t r = idx >> 3, c = idx & 7;
                const uint32_t pc = (c ^ ((r >> 1) & 7)) << 4;
                lds_st16(sq + r * 128 + pc, qv[it]);
                lds_st16(sk + r * 128 + pc, kv[it]);
            }
        }
        if (lin) {  // SP == S: one contiguous run
#pragma unroll
            for (int it = 0; it < MIT; ++it) {
                const int idx = tid + it * kThreads;
                if (idx * 16 < S * S) lds_st16(smask + idx * 16, mv[it]);
            }
        } else if (sc == 0 && !grouped) {  // any layout, or no mask (= every square legal)
            const uint8_t* mb = a.mask ? a.mask + b * a.msb : nullptr;
            for (int idx = tid; idx < S * SP; idx += kThreads) {
                const int i = idx / SP, j = idx - i * SP;
                uint32_t v = j < S;
                if (mb && j < S) v = mb[i * a.mss + j] != 0;
                lds_st1(smask + idx, v);
            }
        }
        __syncthreads();
    };

    // ---- logits of the wave's tiles.  Lane (m, g) supplies chunks g and
    //      4 + g of row 16*t + m (the swizzle of those rows depends on m
    //      only).  Rows past the board (it >= NT) repeat the last tile row;
    //      their legality is zero. ---------------------------------------
    const int sw = (m >> 1) & 7;
    const int c0 = (g ^ sw) * 16, c1 = ((4 + g) ^ sw) * 16;
    f32x4 acc[R][NT];
    auto products = [&](bool first) {
        u32x4 qop[R][2];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const lds_t* qrow = sq + (min(wave + kWaves * r, NT - 1) * 16 + m) * 128;
            qop[r][0] = lds_ld16(qrow + c0);
            qop[r][1] = lds_ld16(qrow + c1);
        }
        const lds_t* krow = lds_opaque(sk + m * 128);
#pragma unroll
        for (int jt = 0; jt < NT; ++jt) {
            const u32x4 kop[2] = {lds_ld16(krow + jt * 2048 + c0), lds_ld16(krow + jt * 2048 + c1)};
#pragma unroll
            for (int r = 0; r < R; ++r)
                acc[r][jt] = KqMma<T>::slice(kop, qop[r], first ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[r][jt]);
            // one tile column at a time: the scheduler may not hoist the
            // operand reads of every column (their registers would spill)
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    const int n2 = S * S;
    auto mask_issue = [&](uint32_t (&mw)[MG]) {
        const rsrc_t rm = make_rsrc(mbase, (uint32_t)n2);
#pragma unroll
        for (int it = 0; it < MG; ++it) {
            const int off = 4 * (tid + it * kThreads) - msh;
            const bool full = off >= 0 && off + 4 <= n2;
            mw[it] = __builtin_amdgcn_raw_buffer_load_b32(rm, full ? off : (int)0xfffffff0u, 0, 0);
            if (!full && off + 4 > 0 && off < n2) {  // a partial group (two threads of the workgroup)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const bool in = off + r >= 0 && off + r < n2;
                    mw[it] |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rm, in ? off + r : (int)0xfffffff0u, 0, 0) << (8 * r);
                }
            }
        }
    };
    auto mask_place = [&](const uint32_t (&mw)[MG]) {
#pragma unroll
        for (int it = 0; it < MG; ++it) {
            int e = 4 * (tid + it * kThreads) - msh;
            if (e >= n2) break;  // (this and every later group of the thread)
            int i = 0, j = e;    // e < 0 (the first group): j reaches 0 at e = 0
            if (e >= 0) {
                i = e / S;
                j = e - i * S;
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (e >= 0 && e < n2) lds_st1(smask + i * SP + j, ((mw[it] >> (8 * r)) & 0xffu) != 0u ? 1u : 0u);
                ++e;
                if (++j == S) {
                    j = 0;
                    ++i;
                }
            }
        }
        // the rows' padding columns S .. SP - 1: illegal
        for (int idx = tid; idx < S * (SP - S); idx += kThreads) {
            const int i = idx / (SP - S);
            lds_st1(smask + i * SP + S + (idx - i * (SP - S)), 0u);
        }
    };
    if constexpr (!MULTI) {
        if (grouped) {  // (before the slice: nothing else is live yet; its barrier publishes the bytes)
            uint32_t mw[MG];
            mask_issue(mw);
            mask_place(mw);
        }
        stage(0);
        products(true);
    } else if constexpr (sizeof(T) == 4) {  // fp32: the same order (measured 6 % faster here than the one below)
        if (grouped) {
            uint32_t mw[MG];
            mask_issue(mw);
            mask_place(mw);
        }
        for (int sc = 0; sc < nslices; ++sc) {
            stage(sc);
            products(sc == 0);
        }
    } else {
        // 16-bit: the mask words are requested before the first slice and
        // placed after it, so both loads wait together (2-3 % faster at the
        // reference head); the next slice's barriers (there are at least two
        // slices) publish the bytes before the legality is read.
        {
            uint32_t mw[MG];
            if (grouped) mask_issue(mw);
            stage(0);
            if (grouped) mask_place(mw);
        }
        products(true);
        for (int sc = 1; sc < nslices; ++sc) {
            stage(sc);
            products(false);
        }
    }

    // ---- legality, 4 bits per tile (bit 4u + e = to-square 4g + e of tile
    //      u = r*NT + jt), from a word of 4 bytes read at a clamped address;
    //      cleared off the board --------------------------------------------
    uint32_t lbits[NLB] = {};
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int i = (wave + kWaves * r) * 16 + m;  // >= S also covers it >= NT
#pragma unroll
        for (int jt = 0; jt < NT; ++jt) {
            const int j0 = jt * 16 + 4 * g;
            uint32_t w = lds_ld4(smask + min(i, S - 1) * SP + min(j0, SP - 4));
            w |= w >> 4;  // fold each byte onto its bit 0
            w |= w >> 2;
            w |= w >> 1;
            uint32_t nib = (w & 1u) | ((w >> 7) & 2u) | ((w >> 14) & 4u) | ((w >> 21) & 8u);
            if (!(i < S && j0 < S)) nib = 0;
            const int u = r * NT + jt;
            lbits[u / 8] |= nib << (4 * (u % 8));
        }
    }

    // ---- values.  Softmax: logits scaled by scale*log2(e), illegal -> -inf;
    //      exp2(x - max) makes the maximum exactly 1 (a single legal move gets
    //      probability exactly 1).  Logits: scaled, illegal -> -1e10. --------
    const float mul = PROBS ? a.c2 : a.scale;
    const float fill = PROBS ? kNegInf : -1e10f;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int jt = 0; jt < NT; ++jt) {
            const int u = r * NT + jt;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                acc[r][jt][e] = ((lbits[u / 8] >> (4 * (u % 8) + e)) & 1u) ? acc[r][jt][e] * mul : fill;
        }

    if constexpr (PROBS) {
        // per-lane trees, then the wave, then the workgroup
        float t[R * NT];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int jt = 0; jt < NT; ++jt)
                t[r * NT + jt] = fmaxf(fmaxf(acc[r][jt][0], acc[r][jt][1]), fmaxf(acc[r][jt][2], acc[r][jt][3]));
#pragma unroll
        for (int n = R * NT; n > 1; n = (n + 1) / 2)
#pragma unroll
            for (int i = 0; i < n / 2; ++i) t[i] = fmaxf(t[i], t[n - 1 - i]);
        float mx = t[0];
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) mx = fmaxf(mx, shfl_xor(mx, off));
        if (lane == 0) red[wave] = mx;
        __syncthreads();
        mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        __syncthreads();
        const bool none_legal = mx == kNegInf;
        const float base = none_legal ? 0.f : mx;
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int jt = 0; jt < NT; ++jt) {
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[r][jt][e] = fast_exp2(acc[r][jt][e] - base);
                t[r * NT + jt] = (acc[r][jt][0] + acc[r][jt][1]) + (acc[r][jt][2] + acc[r][jt][3]);
            }
#pragma unroll
        for (int n = R * NT; n > 1; n = (n + 1) / 2)
#pragma unroll
            for (int i = 0; i < n / 2; ++i) t[i] += t[n - 1 - i];
        float sm = t[0];
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) sm += shfl_xor(sm, off);
        if (lane == 0) red[wave] = sm;
        __syncthreads();
        sm = (red[0] + red[1]) + (red[2] + red[3]);
        const float inv = 1.0f / sm;
        const float uniform = 1.0f / (float)(S * S);
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int jt = 0; jt < NT; ++jt)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[r][jt][e] = none_legal ? uniform : acc[r][jt][e] * inv;
    } else {
        __syncthreads();  // every wave is done with the operand and legality LDS
    }

    // ---- registers -> LDS [S][SP] -> the sample's contiguous S*S row ------
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int i = (wave + kWaves * r) * 16 + m;
        if (i < S) {
            lds_t* orow = sout + (i * SP + 4 * g) * 4;
#pragma unroll
            for (int jt = 0; jt < NT; ++jt)
                if (jt * 16 + 4 * g < S) lds_st16(orow + jt * 64, __builtin_bit_cast(u32x4, acc[r][jt]));
        }
    }
    __syncthreads();
    const rsrc_t ro = make_rsrc(a.out + b * a.osb, (uint32_t)(S * S * 4));
    if (a.out_vec && SP == S) {  // plain (L2-cached) stores: measured faster here than streaming ones
        for (int idx = tid; idx * 4 < S * S; idx += kThreads) buf_st16_cached(ro, idx * 16, lds_ld16(sout + idx * 16));
    } else {
        // Groups of 4 entries, group k = entries 4k - sh .. 4k - sh + 3 with
        // sh the output's misalignment in floats: one aligned 16-byte store
        // each (the two partial groups at the ends store single floats).
        const int n = S * S;
        const int osh = (int)(((uintptr_t)(a.out + b * a.osb) >> 2) & 3);
        const int ng = (n + osh + 3) >> 2;
        for (int k = tid; k < ng; k += kThreads) {
            const int off = 4 * k - osh;
            int e = off, i = 0, j = off;  // off < 0 (the first group): j reaches 0 at e = 0
            if (e >= 0) {
                i = e / S;
                j = e - i * S;
            }
            uint32_t v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                v[r] = (e >= 0 && e < n) ? lds_ld4(sout + (i * SP + j) * 4) : 0u;
                ++e;
                if (++j == S) {
                    j = 0;
                    ++i;
                }
            }
            if (off >= 0 && off + 4 <= n) {
                buf_st16_cached(ro, (uint32_t)off * 4, u32x4{v[0], v[1], v[2], v[3]});
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (off + r >= 0 && off + r < n) buf_st4_cached(ro, (uint32_t)(off + r) * 4, v[r]);
            }
        }
    }
}

namespace {

template <typename T, int NT, bool MULTI>
int launch_kq(hipStream_t st, const KqArgs& a) {
    if (a.probs)
        hipLaunchKernelGGL((kq_policy<T, NT, MULTI, true>), dim3(a.B), dim3(kThreads), kq_lds_bytes(NT, a.S), st, a);
    else
        hipLaunchKernelGGL((kq_policy<T, NT, MULTI, false>), dim3(a.B), dim3(kThreads), kq_lds_bytes(NT, a.S), st, a);
    ATX_CHECK_LAUNCH("atx_kq_masked_softmax_fwd launch");
    return ATX_OK;
}

template <typename T, bool MULTI>
int dispatch_kq_nt(int nt, hipStream_t st, const KqArgs& a) {
    switch (nt) {
        case 1: return launch_kq<T, 1, MULTI>(st, a);
        case 2: return launch_kq<T, 2, MULTI>(st, a);
        case 3: return launch_kq<T, 3, MULTI>(st, a);
        case 4: return launch_kq<T, 4, MULTI>(st, a);
        case 5: return launch_kq<T, 5, MULTI>(st, a);
        case 6: return launch_kq<T, 6, MULTI>(st, a);
        case 7: return launch_kq<T, 7, MULTI>(st, a);
        case 8: return launch_kq<T, 8, MULTI>(st, a);
        default: ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_kq_masked_softmax_fwd: %d tiles", nt);
    }
}

template <typename T>
int dispatch_kq(int nt, hipStream_t st, const KqArgs& a) {
    return a.nchunks > kSliceChunks ? dispatch_kq_nt<T, true>(nt, st, a) : dispatch_kq_nt<T, false>(nt, st, a);
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

    if (p->mask && (p->mask_stride_s < 0 || p->mask_stride_b < 0 ||
                    (int64_t)(p->seq + 16) * p->mask_stride_s + 256 > 0x7fffffffLL))
        ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_kq_masked_softmax_fwd: mask strides must be >= 0 and one sample < 2 GiB");
    // One sample's q / k rows are addressed with 32-bit byte offsets.
    const int64_t row_bytes = (int64_t)p->dim * es;
    if (p->q_stride_s < 0 || p->k_stride_s < 0 ||
        (int64_t)(p->seq + 16) * p->q_stride_s * es + row_bytes > 0x7fffffffLL ||
        (int64_t)(p->seq + 16) * p->k_stride_s * es + row_bytes > 0x7fffffffLL)
        ATX_FAIL(ATX_ERR_UNSUPPORTED, "atx_kq_masked_softmax_fwd: row strides must be >= 0 and one sample < 2 GiB");

    KqArgs a;
    a.q = p->q;
    a.k = p->k;
    a.qsb = p->q_stride_b; a.qss = p->q_stride_s;
    a.ksb = p->k_stride_b; a.kss = p->k_stride_s;
    a.mask = p->mask;
    a.msb = p->mask_stride_b; a.mss = p->mask_stride_s;
    a.out = p->out;
    a.osb = p->out_stride_b;
    a.B = p->batch;
    a.S = p->seq;
    a.nchunks = p->dim * es / 16;
    a.scale = p->scale;
    a.c2 = p->scale * kLog2e;
    a.probs = p->out_mode == ATX_KQ_OUT_PROBS;
    a.mask_lin = p->mask && aligned16(p->mask) && (p->mask_stride_b % 16 == 0) && (p->mask_stride_s == p->seq) &&
                 (p->seq % 4 == 0);
    a.out_vec = aligned16(p->out) && (p->out_stride_b % 4 == 0) && ((p->seq * p->seq) % 4 == 0);
    const int nt = (p->seq + 15) / 16;
    hipStream_t st = static_cast<hipStream_t>(stream);
    switch (p->dtype) {
        case ATX_DTYPE_BF16: return dispatch_kq<__bf16>(nt, st, a);
        case ATX_DTYPE_FP16: return dispatch_kq<_Float16>(nt, st, a);
        default: return dispatch_kq<float>(nt, st, a);
    }
}
