/* CPU restatement of the reference's batched Stratego simulator (oracle).
 *
 * Test infrastructure only: the tests and bench's CPU leg load this through
 * oracle/rollout.py as the checker of the HIP rollout kernels; nothing in the
 * product path links or calls it.
 *
 * One plain loop per game over the same structure-of-arrays state the
 * reference's StrategoRolloutBuffer keeps (csrc/stratego_buffer.cpp:20-54).
 * Each function follows the reference kernel cited beside it, statement for
 * statement in meaning: the rules (movement, Scout paths, combat, flag
 * capture, no-move loss, draw limits), the move-history ring, the two-square
 * and chasing trackers, the reset, the 488-channel infostate and the Zobrist
 * hash.  Floats are IEEE single precision with correctly rounded division.
 */
#include <stdint.h>
#include <string.h>

enum {
    SQ = 100,
    ACTIONS = 10000,
    HIST = 32,
    CHASE = 64,
    ZP = 13,
    CH = 488,
    NO_ATTACK_LIMIT = 100,
    MAX_LEN = 4000,
    TWO_SQ_LIMIT = 3,
};
enum { RED = 0, BLUE = 1, EMPTY = -1 };
enum { ONGOING = -1, RED_WIN = 0, BLUE_WIN = 1, DRAW = 2 };
enum { SPY = 1, SCOUT = 2, MINER = 3, MARSHAL = 10, FLAG = 11, BOMB = 12 };

typedef struct {
    int8_t* owner;             /* [N, 100] */
    int8_t* piece;             /* [N, 100] */
    int8_t* player;            /* [N] */
    int32_t* move_number;      /* [N] */
    int32_t* since_attack;     /* [N] */
    int8_t* outcome;           /* [N] */
    uint8_t* terminated;       /* [N] */
    uint8_t* flag_captured;    /* [N] */
    int32_t* terminated_since; /* [N] */
    uint8_t* moved;            /* [N, 100] */
    uint8_t* revealed;         /* [N, 100] */
    int32_t* history;          /* [N, 32] */
    int32_t* history_head;     /* [N] */
    int32_t* history_len;      /* [N] */
    int32_t* two_sq_count;     /* [N, 2] */
    int32_t* two_sq_lo;        /* [N, 2] */
    int32_t* two_sq_hi;        /* [N, 2] */
    uint8_t* two_sq_violation; /* [N] */
    const int64_t* zobrist;    /* [10, 10, 2, 13] */
    int64_t* chase_hashes;     /* [N, 2, 64] */
    int32_t* chase_head;       /* [N, 2] */
    int32_t* chase_len;        /* [N, 2] */
    int32_t* chase_last_src;   /* [N, 2] */
    uint8_t* chasing_violation; /* [N] */
    int32_t n;
} OrcState;

/* stratego_buffer.cu:10-16 */
static int lake(int r, int c) { return (r == 4 || r == 5) && ((c == 2 || c == 3) || (c == 6 || c == 7)); }
/* :25-27 (Spy..Marshal move; Flag, Bomb, empty do not) */
static int movable(int p) { return p >= SPY && p <= MARSHAL; }
/* :18-23 */
static int rank_of(int p) { return movable(p) ? p : 0; }

static const int DR[4] = {-1, 1, 0, 0};
static const int DC[4] = {0, 0, -1, 1};

/* :32-56: a movable piece of `who` with an in-bounds, non-lake, non-own
 * neighbour. */
static int any_move(const int8_t* ow, const int8_t* pc, int who) {
    for (int s = 0; s < SQ; ++s) {
        if (ow[s] != who || !movable(pc[s])) continue;
        for (int d = 0; d < 4; ++d) {
            int r = s / 10 + DR[d], c = s % 10 + DC[d];
            if (r < 0 || r > 9 || c < 0 || c > 9 || lake(r, c)) continue;
            if (ow[r * 10 + c] != who) return 1;
        }
    }
    return 0;
}

/* hash of one board: :789-798 (and :406-416 inside apply) */
static int64_t board_hash(const int8_t* ow, const int8_t* pc, const int64_t* z) {
    int64_t h = 0;
    for (int s = 0; s < SQ; ++s)
        if (ow[s] >= 0) h ^= z[(s * 2 + ow[s]) * ZP + pc[s]];
    return h;
}

static int count_flags(const int8_t* ow, const int8_t* pc, int who) {
    int k = 0;
    for (int s = 0; s < SQ; ++s) k += ow[s] == who && pc[s] == FLAG;
    return k;
}

/* One game of apply_actions_kernel (stratego_buffer.cu:78-459). */
static void apply_one(OrcState* st, int g, int64_t action) {
    if (st->terminated[g]) return;
    const int me = st->player[g];
    int8_t* ow = st->owner + (int64_t)g * SQ;
    int8_t* pc = st->piece + (int64_t)g * SQ;
    uint8_t* mv = st->moved + (int64_t)g * SQ;
    uint8_t* rv = st->revealed + (int64_t)g * SQ;
    if (action < 0 || action >= ACTIONS) return;
    const int src = (int)(action / SQ), dst = (int)(action % SQ);
    if (src == dst) return;
    const int sr = src / 10, sc = src % 10, tr = dst / 10, tc = dst % 10;
    const int a_ow = ow[src], a_pc = pc[src], d_ow = ow[dst], d_pc = pc[dst];
    /* :125-133 */
    if (a_ow != me || !movable(a_pc) || d_ow == me || lake(tr, tc)) return;
    const int dr = tr - sr, dc = tc - sc;
    if (dr != 0 && dc != 0) return;
    const int dist = dr != 0 ? (dr > 0 ? dr : -dr) : (dc > 0 ? dc : -dc);
    if (a_pc != SCOUT) {
        if (dist != 1) return;
    } else {
        /* :148-161: every square strictly between src and dst empty, no lake */
        const int ur = (dr > 0) - (dr < 0), uc = (dc > 0) - (dc < 0);
        for (int k = 1; k < dist; ++k) {
            const int r = sr + k * ur, c = sc + k * uc;
            if (lake(r, c) || ow[r * 10 + c] != EMPTY) return;
        }
    }
    const int attack = d_ow != EMPTY && d_ow != me;
    /* :165-244: combat, or a plain move */
    if (attack) {
        int win; /* 1 attacker takes dst, 0 attacker dies, -1 both die */
        if (d_pc == FLAG) {
            win = 1;
            st->outcome[g] = me == RED ? RED_WIN : BLUE_WIN;
        } else if (d_pc == BOMB) {
            win = a_pc == MINER ? 1 : 0;
        } else if (a_pc == SPY && d_pc == MARSHAL) {
            win = 1;
        } else {
            const int ra = rank_of(a_pc), rd = rank_of(d_pc);
            win = ra > rd ? 1 : (ra < rd ? 0 : -1);
        }
        if (win == 1) {
            ow[dst] = (int8_t)me;
            pc[dst] = (int8_t)a_pc;
        } else if (win == -1) {
            ow[dst] = EMPTY;
            pc[dst] = 0;
        }
        ow[src] = EMPTY;
        pc[src] = 0;
        st->since_attack[g] = 0;
    } else {
        ow[dst] = (int8_t)me;
        pc[dst] = (int8_t)a_pc;
        ow[src] = EMPTY;
        pc[src] = 0;
        st->since_attack[g] += 1;
    }
    /* :247-256: revealed / moved squares */
    if (attack) {
        rv[src] = 1;
        rv[dst] = 1;
    } else {
        mv[src] = 1;
        mv[dst] = 1;
        rv[dst] = rv[src];
        rv[src] = 0;
    }
    /* :258-263: move-history ring */
    {
        const int h = st->history_head[g];
        st->history[(int64_t)g * HIST + h] = (int32_t)action;
        st->history_head[g] = (h + 1) % HIST;
        if (st->history_len[g] < HIST) st->history_len[g] += 1;
    }
    st->move_number[g] += 1;
    st->player[g] = (int8_t)(me == RED ? BLUE : RED);
    /* :272-299: two-square tracker of the mover */
    {
        const int64_t i = (int64_t)g * 2 + me;
        if (attack) {
            st->two_sq_count[i] = 0;
            st->two_sq_lo[i] = -1;
            st->two_sq_hi[i] = -1;
        } else {
            const int lo = src < dst ? src : dst, hi = src < dst ? dst : src;
            if (st->two_sq_lo[i] == lo && st->two_sq_hi[i] == hi) {
                st->two_sq_count[i] += 1;
            } else {
                st->two_sq_count[i] = 1;
                st->two_sq_lo[i] = lo;
                st->two_sq_hi[i] = hi;
            }
            if (st->two_sq_count[i] > TWO_SQ_LIMIT) st->two_sq_violation[g] = 1;
        }
    }
    /* :301-445: chasing tracker of the mover, on the board after the move */
    {
        const int opp = me == RED ? BLUE : RED;
        const int64_t i = (int64_t)g * 2 + me;
        int threat = 0;
        for (int d = 0; d < 4 && !threat; ++d) {
            const int r = tr + DR[d], c = tc + DC[d];
            if (r < 0 || r > 9 || c < 0 || c > 9 || lake(r, c)) continue;
            threat = ow[r * 10 + c] == opp;
        }
        if (threat) {
            int64_t* ring = st->chase_hashes + i * CHASE;
            const int64_t h = board_hash(ow, pc, st->zobrist);
            const int len = st->chase_len[i];
            int seen = 0;
            for (int k = 0; k < len; ++k) seen |= ring[k] == h;
            const int last = st->chase_last_src[i];
            if (seen && !(last >= 0 && dst == last)) st->chasing_violation[g] = 1;
            if (len < CHASE) {
                ring[len] = h;
                st->chase_len[i] = len + 1;
            } else {
                ring[st->chase_head[i]] = h;
                st->chase_head[i] = (st->chase_head[i] + 1) % CHASE;
            }
            st->chase_last_src[i] = src;
        } else {
            st->chase_len[i] = 0;
            st->chase_head[i] = 0;
            st->chase_last_src[i] = -1;
        }
    }
    /* :447-458: draw limits, then the side to move with no move loses */
    if (st->outcome[g] == ONGOING) {
        if (st->move_number[g] >= MAX_LEN || st->since_attack[g] >= NO_ATTACK_LIMIT) {
            st->outcome[g] = DRAW;
        } else {
            const int next = st->player[g];
            if (!any_move(ow, pc, next)) st->outcome[g] = next == RED ? BLUE_WIN : RED_WIN;
        }
    }
    if (st->outcome[g] != ONGOING) st->terminated[g] = 1;
}

/* StrategoRolloutBuffer::apply_actions (stratego_buffer.cpp:64-121): the
 * kernel over every game, flag_captured |= a colour's flag count dropped
 * (counted over the whole board before and after), terminated_since +=
 * terminated. */
void orc_apply(OrcState* st, const int64_t* actions) {
    for (int g = 0; g < st->n; ++g) {
        const int8_t* ow = st->owner + (int64_t)g * SQ;
        const int8_t* pc = st->piece + (int64_t)g * SQ;
        const int rb = count_flags(ow, pc, RED), bb = count_flags(ow, pc, BLUE);
        apply_one(st, g, actions[g]);
        const int ra = count_flags(ow, pc, RED), ba = count_flags(ow, pc, BLUE);
        if (rb > ra || bb > ba) st->flag_captured[g] = 1;
        st->terminated_since[g] += st->terminated[g] ? 1 : 0;
    }
}

/* legal_action_mask_kernel (stratego_buffer.cu:511-565) over a zeroed mask
 * (compute_legal_action_mask allocates it with torch::zeros, cpp:124-131):
 * every [N, 100, 100] byte is written here. */
void orc_legal_mask(const OrcState* st, uint8_t* mask) {
    memset(mask, 0, (size_t)st->n * ACTIONS);
    for (int g = 0; g < st->n; ++g) {
        const int8_t* ow = st->owner + (int64_t)g * SQ;
        const int8_t* pc = st->piece + (int64_t)g * SQ;
        const int me = st->player[g];
        uint8_t* m = mask + (int64_t)g * ACTIONS;
        for (int s = 0; s < SQ; ++s) {
            if (ow[s] != me || !movable(pc[s])) continue;
            const int reach = pc[s] == SCOUT ? 9 : 1;
            for (int d = 0; d < 4; ++d) {
                for (int k = 1; k <= reach; ++k) {
                    const int r = s / 10 + k * DR[d], c = s % 10 + k * DC[d];
                    if (r < 0 || r > 9 || c < 0 || c > 9 || lake(r, c)) break;
                    const int o = ow[r * 10 + c];
                    if (o == me) break;
                    m[s * SQ + r * 10 + c] = 1;
                    if (o != EMPTY) break;
                }
            }
        }
    }
}

/* reset_kernel (stratego_buffer.cu:575-655) plus the host side of
 * reset_terminated (cpp:246-301): every terminated game restarts from its
 * setups; flag_captured and terminated_since are cleared where a game was
 * reset.  `force_all` is reset_all (cpp:304-307). */
void orc_reset(OrcState* st, const int8_t* setup_red, const int8_t* setup_blue, int force_all) {
    for (int g = 0; g < st->n; ++g) {
        if (force_all) st->terminated[g] = 1;
        if (!st->terminated[g]) continue;
        const int8_t* sr = setup_red + (int64_t)g * SQ;
        const int8_t* sb = setup_blue + (int64_t)g * SQ;
        for (int s = 0; s < SQ; ++s) {
            const int64_t i = (int64_t)g * SQ + s;
            if (sr[s] != 0) {
                st->owner[i] = RED;
                st->piece[i] = sr[s];
            } else if (sb[s] != 0) {
                st->owner[i] = BLUE;
                st->piece[i] = sb[s];
            } else {
                st->owner[i] = EMPTY;
                st->piece[i] = 0;
            }
            st->moved[i] = 0;
            st->revealed[i] = 0;
        }
        for (int k = 0; k < HIST; ++k) st->history[(int64_t)g * HIST + k] = 0;
        st->player[g] = RED;
        st->move_number[g] = 0;
        st->since_attack[g] = 0;
        st->outcome[g] = ONGOING;
        st->terminated[g] = 0;
        st->history_head[g] = 0;
        st->history_len[g] = 0;
        for (int p = 0; p < 2; ++p) {
            const int64_t i = (int64_t)g * 2 + p;
            st->two_sq_count[i] = 0;
            st->two_sq_lo[i] = -1;
            st->two_sq_hi[i] = -1;
            st->chase_head[i] = 0;
            st->chase_len[i] = 0;
            st->chase_last_src[i] = -1;
            for (int k = 0; k < CHASE; ++k) st->chase_hashes[i * CHASE + k] = 0;
        }
        st->two_sq_violation[g] = 0;
        st->chasing_violation[g] = 0;
        st->flag_captured[g] = 0;
        st->terminated_since[g] = 0;
    }
}

/* compute_infostate_kernel (stratego_buffer.cu:663-770) into out [N, 488, 100]
 * float32, from the side to move's perspective. */
void orc_infostate(const OrcState* st, float* out) {
    for (int g = 0; g < st->n; ++g) {
        const int8_t* ow = st->owner + (int64_t)g * SQ;
        const int8_t* pc = st->piece + (int64_t)g * SQ;
        const uint8_t* mv = st->moved + (int64_t)g * SQ;
        const uint8_t* rv = st->revealed + (int64_t)g * SQ;
        const int me = st->player[g];
        float* o = out + (int64_t)g * CH * SQ;
        memset(o, 0, sizeof(float) * CH * SQ);
        const float turn = (float)st->move_number[g] / (float)MAX_LEN;
        const float quiet = (float)st->since_attack[g] / (float)NO_ATTACK_LIMIT;
        for (int s = 0; s < SQ; ++s) {
            const int own = ow[s] == me, opp = ow[s] != me && ow[s] != EMPTY;
            const int p = pc[s];
            for (int t = 1; t <= 12; ++t) {
                if (own && p == t) o[(t - 1) * SQ + s] = 1.0f;                    /* 0-11 */
                if (opp) o[(11 + t) * SQ + s] = rv[s] ? (p == t ? 1.0f : 0.0f) : 1.0f / 12.0f; /* 12-23 */
                if (own) o[(23 + t) * SQ + s] = rv[s] ? (p == t ? 1.0f : 0.0f) : 1.0f / 12.0f; /* 24-35 */
            }
            o[36 * SQ + s] = own && !rv[s] ? 1.0f : 0.0f;
            o[37 * SQ + s] = opp && !rv[s] ? 1.0f : 0.0f;
            o[38 * SQ + s] = ow[s] == EMPTY ? 1.0f : 0.0f;
            o[39 * SQ + s] = own && mv[s] ? 1.0f : 0.0f;
            o[40 * SQ + s] = opp && mv[s] ? 1.0f : 0.0f;
            o[41 * SQ + s] = turn;
            o[42 * SQ + s] = quiet;
        }
        /* 456-487: the last moves, newest first: +1 at dst, -1 at src */
        const int len = st->history_len[g], head = st->history_head[g];
        for (int k = 0; k < HIST && k < len; ++k) {
            const int32_t a = st->history[(int64_t)g * HIST + (head - 1 - k + 2 * HIST) % HIST];
            const int src = a / SQ, dst = a % SQ;
            float* row = o + (456 + k) * SQ;
            for (int s = 0; s < SQ; ++s) row[s] = s == dst ? 1.0f : (s == src ? -1.0f : 0.0f);
        }
    }
}

/* hash_board_kernel (stratego_buffer.cu:782-799) */
void orc_hash(const OrcState* st, int64_t* out) {
    for (int g = 0; g < st->n; ++g)
        out[g] = board_hash(st->owner + (int64_t)g * SQ, st->piece + (int64_t)g * SQ, st->zobrist);
}

/* has_any_legal_move (stratego_buffer.cu:32-56) for the side to move, the
 * brute-force check of get_has_legal_movement (cpp:214-217). */
void orc_any_move(const OrcState* st, uint8_t* out) {
    for (int g = 0; g < st->n; ++g)
        out[g] = (uint8_t)any_move(st->owner + (int64_t)g * SQ, st->piece + (int64_t)g * SQ, st->player[g]);
}
