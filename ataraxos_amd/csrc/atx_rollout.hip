// Batched Stratego simulator for gfx950: the producer of the legal-move masks
// and infostates of self-play (the reference's StrategoRolloutBuffer,
// csrc/stratego_buffer.cu / .cpp).
//
// Layout: N games as a structure of arrays (include/ataraxos_rollout.h), the
// reference buffer's tensors unchanged.
//
// Kernels:
//   rollout_apply      one wave per game.  The move is validated and resolved
//                      with wave-uniform scalars; the scans over the board
//                      (Zobrist hash, chase-ring search, "side to move has a
//                      move") are spread over the 64 lanes and reduced with a
//                      ballot or an XOR butterfly; lane 0 writes the game's
//                      scalars.  The reference runs one thread per game with
//                      serial 100-square loops.
//   rollout_legal_mask one workgroup per game.  Each of 100 threads turns its
//                      square's piece into a 100-bit set of reachable squares
//                      in LDS; then every 16-byte chunk of the game's 10,000
//                      mask bytes is formed from 16 bits of those sets and
//                      written once (the reference clears the mask with a
//                      separate torch::zeros pass and then sets entries).
//   rollout_infostate  one thread per 16-byte chunk of the output, no LDS,
//                      no barrier: every output float written once with
//                      16-byte streaming stores (the reference: a zeroing
//                      pass plus one thread per float).
//   rollout_reset      one wave per game, lanes over squares and ring slots.
//   rollout_hash       one wave per game, XOR butterfly.
//
// Indices derived from the state (ring heads, lengths, the side to move,
// owners and pieces used as table indices) are masked or range-checked, so a
// corrupted state cannot make a kernel touch memory outside its arrays; for
// a valid state every such guard is the identity.
#include "atx_common.hpp"
#include "ataraxos_rollout.h"

namespace atx {
namespace {

constexpr int kSq = 100;
constexpr int kActions = kSq * kSq;
constexpr int kHist = 32;
constexpr int kChase = 64;
constexpr int kZobristPieces = 13;
constexpr int kChannels = 488;
constexpr int kNoAttackLimit = 100;   // TRAINING_NO_ATTACK_LIMIT
constexpr int kMaxGameLength = 4000;  // MAX_GAME_LENGTH
constexpr int kTwoSquareLimit = 3;
constexpr int kEmpty = -1;
constexpr int kOngoing = -1, kRedWin = 0, kBlueWin = 1, kDraw = 2;
constexpr int kSpy = 1, kScout = 2, kMiner = 3, kMarshal = 10, kFlag = 11, kBomb = 12;

constexpr int kWaveGames = 4;  // games per 256-thread workgroup in the wave-per-game kernels

__device__ inline bool lake(int r, int c) {
    return (r == 4 || r == 5) && ((unsigned)(c - 2) < 2u || (unsigned)(c - 6) < 2u);
}
__device__ inline bool movable(int p) { return p >= kSpy && p <= kMarshal; }
__device__ inline int rank_of(int p) { return movable(p) ? p : 0; }
__device__ inline bool on_board(int r, int c) { return (unsigned)r < 10u && (unsigned)c < 10u; }

__device__ inline int64_t zobrist_term(const int64_t* z, int sq, int ow, int pc) {
    // ow in {0, 1} and pc in 0..12 for every occupied square of a valid board
    if (ow < 0 || ow > 1 || (unsigned)pc > 12u) return 0;
    return z[(sq * 2 + ow) * kZobristPieces + pc];
}

__device__ inline int64_t wave_xor(int64_t v) {
    uint32_t lo = (uint32_t)v, hi = (uint32_t)((uint64_t)v >> 32);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        lo ^= (uint32_t)__shfl_xor((int)lo, m);
        hi ^= (uint32_t)__shfl_xor((int)hi, m);
    }
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

// ---------------------------------------------------------------------------
// apply
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rollout_apply(AtxRolloutState st, const int64_t* __restrict__ actions) {
    __shared__ int8_t s_own[kWaveGames][128];
    __shared__ int8_t s_pc[kWaveGames][128];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int g = blockIdx.x * kWaveGames + w;
    const bool live = g < st.n_games;
    const int64_t gs = (int64_t)g * kSq;
    const int s1 = 64 + lane;  // second square of this lane (valid if < 100)

    int o0 = kEmpty, p0 = 0, o1 = kEmpty, p1 = 0;
    if (live) {
        o0 = st.board_owner[gs + lane];
        p0 = st.board_piece[gs + lane];
        if (s1 < kSq) {
            o1 = st.board_owner[gs + s1];
            p1 = st.board_piece[gs + s1];
        }
    }
    s_own[w][lane] = (int8_t)o0;
    s_pc[w][lane] = (int8_t)p0;
    if (s1 < kSq) {
        s_own[w][s1] = (int8_t)o1;
        s_pc[w][s1] = (int8_t)p1;
    }
    __syncthreads();

    // ---- validation (wave-uniform), stratego_buffer.cu:107-162 ----
    const int64_t act = live ? actions[g] : -1;
    const int me = live ? st.current_player[g] : 0;
    bool ok = live && !st.terminated[g] && act >= 0 && act < kActions;
    const int src = ok ? (int)(act / kSq) : 0, dst = ok ? (int)(act % kSq) : 1;
    ok = ok && src != dst;
    const int sr = src / 10, sc = src % 10, tr = dst / 10, tc = dst % 10;
    const int a_ow = s_own[w][src], a_pc = s_pc[w][src], d_ow = s_own[w][dst], d_pc = s_pc[w][dst];
    ok = ok && a_ow == me && movable(a_pc) && d_ow != me && !lake(tr, tc);
    const int dr = tr - sr, dc = tc - sc;
    ok = ok && (dr == 0 || dc == 0);
    const int dist = dr != 0 ? (dr > 0 ? dr : -dr) : (dc > 0 ? dc : -dc);
    if (a_pc != kScout) {
        ok = ok && dist == 1;
    } else if (ok) {
        const int ur = (dr > 0) - (dr < 0), uc = (dc > 0) - (dc < 0);
        for (int k = 1; k < dist; ++k) {
            const int r = sr + k * ur, c = sc + k * uc;
            ok = ok && !lake(r, c) && s_own[w][r * 10 + c] == kEmpty;
        }
    }

    // ---- resolution (wave-uniform), :164-244 ----
    const bool attack = d_ow != kEmpty && d_ow != me;
    int win = 1;  // 1 attacker takes dst, 0 attacker dies, -1 both die
    if (attack) {
        if (d_pc == kFlag) win = 1;
        else if (d_pc == kBomb) win = a_pc == kMiner ? 1 : 0;
        else if (a_pc == kSpy && d_pc == kMarshal) win = 1;
        else {
            const int ra = rank_of(a_pc), rd = rank_of(d_pc);
            win = ra > rd ? 1 : (ra < rd ? 0 : -1);
        }
    }
    const int n_ow = win == 1 ? me : (win == 0 ? d_ow : kEmpty);
    const int n_pc = win == 1 ? a_pc : (win == 0 ? d_pc : 0);
    const bool flag_taken = ok && attack && d_pc == kFlag;

    // board after the move, in LDS for the neighbour scans
    if (ok && lane == 0) {
        s_own[w][src] = (int8_t)kEmpty;
        s_pc[w][src] = 0;
        s_own[w][dst] = (int8_t)n_ow;
        s_pc[w][dst] = (int8_t)n_pc;
    }
    __syncthreads();

    if (ok) {
        const int next = me == 0 ? 1 : 0;
        const int mi = me & 1;
        // chasing: does the piece now on dst's square stand next to an
        // opponent piece (:316-330)
        bool threat = false;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const int r = tr + (d == 0 ? -1 : d == 1 ? 1 : 0), c = tc + (d == 2 ? -1 : d == 3 ? 1 : 0);
            threat = threat || (on_board(r, c) && !lake(r, c) && s_own[w][r * 10 + c] == next);
        }
        // Zobrist hash of the board after the move (:333-344)
        int64_t h = 0;
        if (threat) {
            h = zobrist_term(st.zobrist_table, lane, s_own[w][lane], s_pc[w][lane]);
            if (s1 < kSq) h ^= zobrist_term(st.zobrist_table, s1, s_own[w][s1], s_pc[w][s1]);
            h = wave_xor(h);
        }
        const int64_t pi = (int64_t)g * 2 + mi;
        int chase_len = 0;
        bool seen = false;
        if (threat) {
            chase_len = st.chase_hash_len[pi];
            const bool mine = lane < chase_len && st.chase_hashes[pi * kChase + lane] == h;
            seen = __ballot(mine) != 0;
        }
        // side to move next has a movable piece with a free neighbour (:32-56)
        bool has_move = false;
        for (int s = lane; s < kSq; s += 64) {
            if (s_own[w][s] != next || !movable(s_pc[w][s])) continue;
            const int r0 = s / 10, c0 = s % 10;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const int r = r0 + (d == 0 ? -1 : d == 1 ? 1 : 0), c = c0 + (d == 2 ? -1 : d == 3 ? 1 : 0);
                has_move = has_move || (on_board(r, c) && !lake(r, c) && s_own[w][r * 10 + c] != next);
            }
        }
        has_move = __ballot(has_move) != 0;

        if (lane == 0) {
            st.board_owner[gs + src] = (int8_t)kEmpty;
            st.board_piece[gs + src] = 0;
            st.board_owner[gs + dst] = (int8_t)n_ow;
            st.board_piece[gs + dst] = (int8_t)n_pc;
            int outcome = st.outcome[g];
            if (flag_taken) outcome = me == 0 ? kRedWin : kBlueWin;
            int since = attack ? 0 : st.moves_since_attack[g] + 1;
            st.moves_since_attack[g] = since;
            // revealed / moved squares (:247-256)
            uint8_t* rv = st.revealed_squares + gs;
            uint8_t* mv = st.moved_squares + gs;
            if (attack) {
                rv[src] = 1;
                rv[dst] = 1;
            } else {
                mv[src] = 1;
                mv[dst] = 1;
                const uint8_t r_src = rv[src];
                rv[dst] = r_src;
                rv[src] = 0;
            }
            // move-history ring (:258-263)
            const int head = st.move_history_head[g] & (kHist - 1);
            st.move_history[(int64_t)g * kHist + head] = (int32_t)act;
            st.move_history_head[g] = (head + 1) & (kHist - 1);
            if (st.move_history_len[g] < kHist) st.move_history_len[g] += 1;
            const int moves = st.move_number[g] + 1;
            st.move_number[g] = moves;
            st.current_player[g] = (int8_t)next;
            // two-square tracker of the mover (:272-299)
            if (attack) {
                st.two_square_count[pi] = 0;
                st.two_square_pair_lo[pi] = -1;
                st.two_square_pair_hi[pi] = -1;
            } else {
                const int lo = src < dst ? src : dst, hi = src < dst ? dst : src;
                int cnt = 1;
                if (st.two_square_pair_lo[pi] == lo && st.two_square_pair_hi[pi] == hi) {
                    cnt = st.two_square_count[pi] + 1;
                } else {
                    st.two_square_pair_lo[pi] = lo;
                    st.two_square_pair_hi[pi] = hi;
                }
                st.two_square_count[pi] = cnt;
                if (cnt > kTwoSquareLimit) st.two_square_violation[g] = 1;
            }
            // chasing tracker of the mover (:346-381)
            if (threat) {
                const int last = st.chase_last_src[pi];
                if (seen && !(last >= 0 && dst == last)) st.chasing_violation[g] = 1;
                int64_t* ring = st.chase_hashes + pi * kChase;
                if (chase_len >= 0 && chase_len < kChase) {
                    ring[chase_len] = h;
                    st.chase_hash_len[pi] = chase_len + 1;
                } else {
                    const int ch = st.chase_hash_head[pi] & (kChase - 1);
                    ring[ch] = h;
                    st.chase_hash_head[pi] = (ch + 1) & (kChase - 1);
                }
                st.chase_last_src[pi] = src;
            } else {
                st.chase_hash_len[pi] = 0;
                st.chase_hash_head[pi] = 0;
                st.chase_last_src[pi] = -1;
            }
            // terminal checks (:447-458)
            if (outcome == kOngoing) {
                if (moves >= kMaxGameLength || since >= kNoAttackLimit) outcome = kDraw;
                else if (!has_move) outcome = next == 0 ? kBlueWin : kRedWin;
            }
            st.outcome[g] = (int8_t)outcome;
            if (outcome != kOngoing) st.terminated[g] = 1;
        }
    }
    // host-side bookkeeping of apply_actions (stratego_buffer.cpp:94-120): a
    // colour's flag count drops exactly when a flag is attacked, since flags
    // never move and always lose
    if (live && lane == 0) {
        if (flag_taken) st.flag_captured[g] = 1;
        st.terminated_since[g] += st.terminated[g] ? 1 : 0;
    }
}

// ---------------------------------------------------------------------------
// legal-move mask
// ---------------------------------------------------------------------------
constexpr int kMaskThreads = 128;
constexpr int kMaskChunks = kActions / 16;  // 625 chunks of 16 bytes per game

__global__ __launch_bounds__(kMaskThreads) void rollout_legal_mask(AtxRolloutState st, uint8_t* __restrict__ mask) {
    __shared__ int8_t s_own[128];
    __shared__ int8_t s_pc[128];
    __shared__ uint32_t s_reach[kSq][4];  // bit d of word w: square 32w + d reachable
    const int t = threadIdx.x;
    const int g = blockIdx.x;
    const int me = st.current_player[g];
    if (t < kSq) {
        s_own[t] = st.board_owner[(int64_t)g * kSq + t];
        s_pc[t] = st.board_piece[(int64_t)g * kSq + t];
    }
    __syncthreads();
    if (t < kSq) {
        uint32_t m[4] = {0, 0, 0, 0};
        if (s_own[t] == me && movable(s_pc[t])) {
            const int reach = s_pc[t] == kScout ? 9 : 1;
            const int r0 = t / 10, c0 = t % 10;
            for (int d = 0; d < 4; ++d) {
                const int ur = d == 0 ? -1 : d == 1 ? 1 : 0, uc = d == 2 ? -1 : d == 3 ? 1 : 0;
                for (int k = 1; k <= reach; ++k) {
                    const int r = r0 + k * ur, c = c0 + k * uc;
                    if (!on_board(r, c) || lake(r, c)) break;
                    const int s = r * 10 + c, o = s_own[s];
                    if (o == me) break;
                    m[s >> 5] |= 1u << (s & 31);
                    if (o != kEmpty) break;
                }
            }
        }
        s_reach[t][0] = m[0];
        s_reach[t][1] = m[1];
        s_reach[t][2] = m[2];
        s_reach[t][3] = m[3];
    }
    __syncthreads();
    uint8_t* out = mask + (int64_t)g * kActions;
    for (int c = t; c < kMaskChunks; c += kMaskThreads) {
        // entries 16c .. 16c+15: from-square src, to-squares dst0 .. (wrapping
        // into src + 1); dst0 is a multiple of 4 and the sets have no bits
        // past 99, so the two pieces can be OR-ed
        const int e0 = c * 16, src = e0 / kSq, dst0 = e0 - src * kSq;
        auto bits16 = [&](int s, int off) -> uint32_t {
            const int wi = off >> 5, sh = off & 31;
            uint32_t v = s_reach[s][wi] >> sh;
            if (sh > 16 && wi < 3) v |= s_reach[s][wi + 1] << (32 - sh);
            return v & 0xffffu;
        };
        uint32_t bits = bits16(src, dst0);
        if (dst0 + 16 > kSq) bits |= (bits16(src + 1, 0) << (kSq - dst0)) & 0xffffu;
        u32x4 v;
        v.x = ((bits & 15u) * 0x204081u) & 0x01010101u;
        v.y = (((bits >> 4) & 15u) * 0x204081u) & 0x01010101u;
        v.z = (((bits >> 8) & 15u) * 0x204081u) & 0x01010101u;
        v.w = (((bits >> 12) & 15u) * 0x204081u) & 0x01010101u;
        st16_stream(out + e0, v);
    }
}

// ---------------------------------------------------------------------------
// infostate
// ---------------------------------------------------------------------------
constexpr int kInfoChunks = kChannels * kSq / 4;  // 12,200 chunks of 4 floats per game

// One 16-byte chunk (4 squares of one channel) per thread, every thread of
// the grid independent: 85 % of the chunks are the all-zero channels 43-455
// and cost a store; a board channel reads its 4 squares' owner, piece,
// revealed and moved bytes as one aligned 4-byte word each (mostly L2 hits,
// a game's board is shared by its 1,075 board-channel chunks).
__global__ __launch_bounds__(256) void rollout_infostate(AtxRolloutState st, float* __restrict__ out, int64_t total) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= total) return;
    const int g = (int)(c / kInfoChunks);
    const int cl = (int)(c - (int64_t)g * kInfoChunks);
    const int ch = cl / 25, s0 = (cl - ch * 25) * 4;
    u32x4 u = {0u, 0u, 0u, 0u};
    if (ch < 43) {
        const int64_t b = (int64_t)g * kSq + s0;
        const uint32_t ow4 = *reinterpret_cast<const uint32_t*>(st.board_owner + b);
        const uint32_t pc4 = *reinterpret_cast<const uint32_t*>(st.board_piece + b);
        const uint32_t rv4 = *reinterpret_cast<const uint32_t*>(st.revealed_squares + b);
        const uint32_t mv4 = *reinterpret_cast<const uint32_t*>(st.moved_squares + b);
        const int me = st.current_player[g];
        const float turn = (float)st.move_number[g] / (float)kMaxGameLength;
        const float quiet = (float)st.moves_since_attack[g] / (float)kNoAttackLimit;
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int o = (int)(int8_t)(ow4 >> (8 * j)), p = (int)(int8_t)(pc4 >> (8 * j));
            const bool rev = (rv4 >> (8 * j)) & 0xffu, mov = (mv4 >> (8 * j)) & 0xffu;
            const bool own = o == me, opp = o != me && o != kEmpty;
            float x;
            if (ch < 12) x = own && p == ch + 1 ? 1.0f : 0.0f;                                   // own piece types
            else if (ch < 24) x = opp ? (rev ? (p == ch - 11 ? 1.0f : 0.0f) : 1.0f / 12.0f) : 0.0f;  // opponent's
            else if (ch < 36) x = own ? (rev ? (p == ch - 23 ? 1.0f : 0.0f) : 1.0f / 12.0f) : 0.0f;  // own, as seen
            else if (ch == 36) x = own && !rev ? 1.0f : 0.0f;
            else if (ch == 37) x = opp && !rev ? 1.0f : 0.0f;
            else if (ch == 38) x = o == kEmpty ? 1.0f : 0.0f;
            else if (ch == 39) x = own && mov ? 1.0f : 0.0f;
            else if (ch == 40) x = opp && mov ? 1.0f : 0.0f;
            else if (ch == 41) x = turn;
            else x = quiet;
            v[j] = x;
        }
        u.x = __builtin_bit_cast(uint32_t, v[0]);
        u.y = __builtin_bit_cast(uint32_t, v[1]);
        u.z = __builtin_bit_cast(uint32_t, v[2]);
        u.w = __builtin_bit_cast(uint32_t, v[3]);
    } else if (ch >= 456) {
        // the k-th most recent move: +1 at its destination, -1 at its source
        const int k = ch - 456;
        if (k < st.move_history_len[g]) {
            const int head = st.move_history_head[g];
            const int32_t a = st.move_history[(int64_t)g * kHist + ((head - 1 - k + 2 * kHist) & (kHist - 1))];
            const int hs = a / kSq, hd = a % kSq;
            float v[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = s0 + j == hd ? 1.0f : (s0 + j == hs ? -1.0f : 0.0f);
            u.x = __builtin_bit_cast(uint32_t, v[0]);
            u.y = __builtin_bit_cast(uint32_t, v[1]);
            u.z = __builtin_bit_cast(uint32_t, v[2]);
            u.w = __builtin_bit_cast(uint32_t, v[3]);
        }
    }
    st16_stream(out + c * 4, u);
}

// ---------------------------------------------------------------------------
// reset
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rollout_reset(AtxRolloutState st, const int8_t* __restrict__ red,
                                                     const int8_t* __restrict__ blue, int force_all) {
    const int lane = threadIdx.x & 63;
    const int g = blockIdx.x * kWaveGames + (threadIdx.x >> 6);
    if (g >= st.n_games) return;
    if (!force_all && !st.terminated[g]) return;
    const int64_t gs = (int64_t)g * kSq;
    for (int s = lane; s < kSq; s += 64) {
        const int r = red[gs + s], b = blue[gs + s];
        st.board_owner[gs + s] = (int8_t)(r != 0 ? 0 : (b != 0 ? 1 : kEmpty));
        st.board_piece[gs + s] = (int8_t)(r != 0 ? r : b);
        st.moved_squares[gs + s] = 0;
        st.revealed_squares[gs + s] = 0;
    }
    if (lane < kHist) st.move_history[(int64_t)g * kHist + lane] = 0;
    st.chase_hashes[(int64_t)g * 2 * kChase + lane] = 0;
    st.chase_hashes[(int64_t)g * 2 * kChase + kChase + lane] = 0;
    if (lane < 2) {
        const int64_t pi = (int64_t)g * 2 + lane;
        st.two_square_count[pi] = 0;
        st.two_square_pair_lo[pi] = -1;
        st.two_square_pair_hi[pi] = -1;
        st.chase_hash_head[pi] = 0;
        st.chase_hash_len[pi] = 0;
        st.chase_last_src[pi] = -1;
    }
    if (lane == 0) {
        st.current_player[g] = 0;
        st.move_number[g] = 0;
        st.moves_since_attack[g] = 0;
        st.outcome[g] = (int8_t)kOngoing;
        st.terminated[g] = 0;
        st.move_history_head[g] = 0;
        st.move_history_len[g] = 0;
        st.two_square_violation[g] = 0;
        st.chasing_violation[g] = 0;
        st.flag_captured[g] = 0;
        st.terminated_since[g] = 0;
    }
}

// ---------------------------------------------------------------------------
// hash
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rollout_hash(AtxRolloutState st, int64_t* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int g = blockIdx.x * kWaveGames + (threadIdx.x >> 6);
    if (g >= st.n_games) return;  // wave-uniform
    const int64_t gs = (int64_t)g * kSq;
    int64_t h = zobrist_term(st.zobrist_table, lane, st.board_owner[gs + lane], st.board_piece[gs + lane]);
    if (lane + 64 < kSq)
        h ^= zobrist_term(st.zobrist_table, lane + 64, st.board_owner[gs + lane + 64], st.board_piece[gs + lane + 64]);
    h = wave_xor(h);
    if (lane == 0) out[g] = h;
}

__global__ void rollout_hello(int32_t* out, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = 42;
}

int check_state(const AtxRolloutState* st, const char* what) {
    if (!st) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "%s: null state", what);
    if (st->abi_version != ATX_ABI_VERSION)
        ATX_FAIL(ATX_ERR_ABI, "%s: abi_version %d, library %d", what, st->abi_version, ATX_ABI_VERSION);
    if (st->n_games < 0) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "%s: n_games %d < 0", what, st->n_games);
    if (st->n_games == 0) return ATX_OK;
    const void* ptrs[] = {st->board_owner, st->board_piece, st->current_player, st->move_number,
                          st->moves_since_attack, st->outcome, st->terminated, st->flag_captured,
                          st->terminated_since, st->moved_squares, st->revealed_squares, st->move_history,
                          st->move_history_head, st->move_history_len, st->two_square_count,
                          st->two_square_pair_lo, st->two_square_pair_hi, st->two_square_violation,
                          st->zobrist_table, st->chase_hashes, st->chase_hash_head, st->chase_hash_len,
                          st->chase_last_src, st->chasing_violation};
    for (size_t i = 0; i < sizeof(ptrs) / sizeof(ptrs[0]); ++i)
        if (!ptrs[i]) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "%s: state array %zu is null", what, i);
    return ATX_OK;
}

}  // namespace
}  // namespace atx

using namespace atx;

extern "C" int atx_rollout_apply(const AtxRolloutState* st, const int64_t* actions, void* stream) {
    clear_error();
    if (int rc = check_state(st, "atx_rollout_apply")) return rc;
    if (st->n_games == 0) return ATX_OK;
    if (!actions) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_rollout_apply: null actions");
    const int grid = (st->n_games + kWaveGames - 1) / kWaveGames;
    hipLaunchKernelGGL(rollout_apply, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream), *st, actions);
    ATX_CHECK_LAUNCH("atx_rollout_apply");
    return ATX_OK;
}

extern "C" int atx_rollout_legal_mask(const AtxRolloutState* st, uint8_t* mask, void* stream) {
    clear_error();
    if (int rc = check_state(st, "atx_rollout_legal_mask")) return rc;
    if (st->n_games == 0) return ATX_OK;
    if (!mask) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_rollout_legal_mask: null mask");
    if (!aligned16(mask)) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_rollout_legal_mask: mask must be 16-byte aligned");
    hipLaunchKernelGGL(rollout_legal_mask, dim3(st->n_games), dim3(kMaskThreads), 0, static_cast<hipStream_t>(stream), *st,
                       mask);
    ATX_CHECK_LAUNCH("atx_rollout_legal_mask");
    return ATX_OK;
}

extern "C" int atx_rollout_infostate(const AtxRolloutState* st, float* out, void* stream) {
    clear_error();
    if (int rc = check_state(st, "atx_rollout_infostate")) return rc;
    if (st->n_games == 0) return ATX_OK;
    if (!out) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_rollout_infostate: null output");
    if (!aligned16(out)) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_rollout_infostate: output must be 16-byte aligned");
    const void* words[] = {st->board_owner, st->board_piece, st->revealed_squares, st->moved_squares};
    for (const void* p : words)
        if (reinterpret_cast<uintptr_t>(p) & 3u)
            ATX_FAIL(ATX_ERR_INVALID_ARGUMENT,
                     "atx_rollout_infostate: board_owner, board_piece, revealed_squares and moved_squares must be "
                     "4-byte aligned");
    const int64_t total = (int64_t)st->n_games * kInfoChunks;
    hipLaunchKernelGGL(rollout_infostate, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), *st, out, total);
    ATX_CHECK_LAUNCH("atx_rollout_infostate");
    return ATX_OK;
}

extern "C" int atx_rollout_reset(const AtxRolloutState* st, const int8_t* setup_red, const int8_t* setup_blue,
                                 int32_t force_all, void* stream) {
    clear_error();
    if (int rc = check_state(st, "atx_rollout_reset")) return rc;
    if (st->n_games == 0) return ATX_OK;
    if (!setup_red || !setup_blue) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_rollout_reset: null setup");
    const int grid = (st->n_games + kWaveGames - 1) / kWaveGames;
    hipLaunchKernelGGL(rollout_reset, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream), *st, setup_red,
                       setup_blue, force_all != 0 ? 1 : 0);
    ATX_CHECK_LAUNCH("atx_rollout_reset");
    return ATX_OK;
}

extern "C" int atx_rollout_hash(const AtxRolloutState* st, int64_t* out, void* stream) {
    clear_error();
    if (int rc = check_state(st, "atx_rollout_hash")) return rc;
    if (st->n_games == 0) return ATX_OK;
    if (!out) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_rollout_hash: null output");
    const int grid = (st->n_games + kWaveGames - 1) / kWaveGames;
    hipLaunchKernelGGL(rollout_hash, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream), *st, out);
    ATX_CHECK_LAUNCH("atx_rollout_hash");
    return ATX_OK;
}

extern "C" int atx_rollout_hello(int32_t* out, int32_t n, void* stream) {
    clear_error();
    if (n < 0 || (n > 0 && !out)) ATX_FAIL(ATX_ERR_INVALID_ARGUMENT, "atx_rollout_hello: bad output");
    if (n == 0) return ATX_OK;
    hipLaunchKernelGGL(rollout_hello, dim3((n + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream), out, n);
    ATX_CHECK_LAUNCH("atx_rollout_hello");
    return ATX_OK;
}
