/*
 * ataraxos_rollout.h — C ABI of the batched Stratego simulator in
 * `libataraxos_attn.so`: the producer of the legal-move masks and infostates
 * that the attention hot path consumes during self-play.
 *
 * It replaces the reference's CUDA extension `StrategoRolloutBuffer`
 * (csrc/stratego_buffer.cu, .cuh, .cpp).  Each entry point below names the
 * reference launcher and kernel it replaces.  The conventions of
 * ataraxos_attn.h apply: return codes ATX_OK / ATX_ERR_*, error text from
 * atx_last_error(), asynchronous launch on the caller's stream, no device
 * memory allocated by the library, host-side validation before any HIP call.
 *
 * State.  N games live on the device as a structure of arrays, the same
 * arrays, shapes and element types as the reference buffer's tensors
 * (stratego_buffer.cpp:24-53), every array dense and contiguous in the
 * order of the shapes given below.  torch.bool arrays are one byte per
 * element, 0 or 1 (uint8_t here).  Squares are indexed row * 10 + col; an
 * action is src * 100 + dst.  The caller owns and allocates every array.
 */
#ifndef ATARAXOS_ROLLOUT_H
#define ATARAXOS_ROLLOUT_H

#include <stdint.h>

#include "ataraxos_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct AtxRolloutState {
    int32_t abi_version; /* must equal ATX_ABI_VERSION */
    int32_t n_games;     /* N >= 0 */
    int8_t* board_owner;          /* [N, 100]: 0 red, 1 blue, -1 empty */
    int8_t* board_piece;          /* [N, 100]: PieceType 0..12 */
    int8_t* current_player;       /* [N] */
    int32_t* move_number;         /* [N] */
    int32_t* moves_since_attack;  /* [N] */
    int8_t* outcome;              /* [N]: -1 ongoing, 0 red win, 1 blue win, 2 draw */
    uint8_t* terminated;          /* [N] bool */
    uint8_t* flag_captured;       /* [N] bool */
    int32_t* terminated_since;    /* [N] */
    uint8_t* moved_squares;       /* [N, 100] bool */
    uint8_t* revealed_squares;    /* [N, 100] bool */
    int32_t* move_history;        /* [N, 32] ring of actions */
    int32_t* move_history_head;   /* [N] */
    int32_t* move_history_len;    /* [N] */
    int32_t* two_square_count;    /* [N, 2] per player */
    int32_t* two_square_pair_lo;  /* [N, 2] */
    int32_t* two_square_pair_hi;  /* [N, 2] */
    uint8_t* two_square_violation; /* [N] bool */
    const int64_t* zobrist_table; /* [10, 10, 2, 13] */
    int64_t* chase_hashes;        /* [N, 2, 64] per player ring */
    int32_t* chase_hash_head;     /* [N, 2] */
    int32_t* chase_hash_len;      /* [N, 2] */
    int32_t* chase_last_src;      /* [N, 2] */
    uint8_t* chasing_violation;   /* [N] bool */
} AtxRolloutState;

/*
 * Applies actions[g] (int64 [N], device) to every game g in one launch:
 * validation, movement, Scout paths, combat, flag capture, move history,
 * the two-square and chasing trackers, and the draw / no-move terminal
 * checks.  A terminated game or an illegal action leaves the game as it is.
 * Also does the host-side bookkeeping of the reference's apply_actions:
 * flag_captured |= a flag was captured, terminated_since += terminated.
 * Replaces StrategoRolloutBuffer::apply_actions (stratego_buffer.cpp:64-121)
 * and apply_actions_kernel (stratego_buffer.cu:78-459).
 */
int atx_rollout_apply(const AtxRolloutState* st, const int64_t* actions, void* stream);

/*
 * mask (bool [N, 100, 100], device, 16-byte aligned): mask[g, src, dst] = 1 where moving the
 * side to move's piece from src to dst is legal, 0 elsewhere.  Every byte is
 * written; the caller need not clear the buffer.
 * Replaces compute_legal_action_mask (stratego_buffer.cpp:124-139) and
 * legal_action_mask_kernel (stratego_buffer.cu:511-565).
 */
int atx_rollout_legal_mask(const AtxRolloutState* st, uint8_t* mask, void* stream);

/*
 * out (float32 [N, 488, 10, 10], device, 16-byte aligned): the infostate
 * from the side to move's perspective; channels 43-455 are 0.  Every element
 * is written.  board_owner, board_piece, revealed_squares and moved_squares
 * must be 4-byte aligned (they are read four squares at a time).
 * Replaces compute_infostate_tensor (stratego_buffer.cpp:154-178) and
 * compute_infostate_kernel (stratego_buffer.cu:663-770).
 */
int atx_rollout_infostate(const AtxRolloutState* st, float* out, void* stream);

/*
 * Restarts every terminated game (every game if force_all != 0) from its
 * setups: setup_red / setup_blue (int8 [N, 10, 10], device) hold piece types,
 * 0 = none; a square takes Red's piece if any, else Blue's.  Clears the
 * trackers, flag_captured and terminated_since of the restarted games.
 * Replaces reset_terminated / reset_all (stratego_buffer.cpp:246-307) and
 * reset_kernel (stratego_buffer.cu:575-655).
 */
int atx_rollout_reset(const AtxRolloutState* st, const int8_t* setup_red, const int8_t* setup_blue,
                      int32_t force_all, void* stream);

/*
 * out (int64 [N], device): Zobrist hash of every board, the XOR of
 * zobrist_table[row, col, owner, piece] over the occupied squares.
 * Replaces hash_board (stratego_buffer.cpp:192-206) and hash_board_kernel
 * (stratego_buffer.cu:782-799).
 */
int atx_rollout_hash(const AtxRolloutState* st, int64_t* out, void* stream);

/*
 * out (int32 [n], device) = 42: the build check.
 * Replaces hello_world (stratego_buffer.cpp:56-62, stratego_buffer.cu:64-75).
 */
int atx_rollout_hello(int32_t* out, int32_t n, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ATARAXOS_ROLLOUT_H */
