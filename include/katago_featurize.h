/*
 * katago_featurize.h - C ABI of the position featurizer in libkatago_host.so:
 * the neural-net input rows of KataGo's NNInputs::fillRowV7
 * (/root/reference/cpp/neuralnet/nninputs.cpp:2273-2720), the inputs of
 * every model of versions 8 to 17 (22 spatial planes, 19 global features).
 *
 * The caller describes each position with what KataGo's Board and
 * BoardHistory hold (the colours of the current board and of the boards one
 * and two moves back, their simple-ko points, the ko-ban arrays, the last
 * moves, the phase and rules flags, the side to move's komi); the featurizer
 * computes the board analysis itself: chains and liberties, the ladder
 * searches of the current and two previous boards (Board::searchIsLadderCaptured,
 * board.cpp:1520-1790, through nninputs.cpp:815-870) and the pass-alive area
 * (Board::calculateArea / calculateIndependentLifeArea, board.cpp:1792-2250).
 * katago_amd/host/neuralnet/featurizeadapter.cpp fills a kgn_position from
 * KataGo's own Board/BoardHistory.
 *
 * Points are indexed y * x_size + x on the board (not the nn tensor).
 * Colours: 0 empty, 1 black, 2 white (KataGo's C_EMPTY, C_BLACK, C_WHITE).
 */
#ifndef KATAGO_FEATURIZE_H
#define KATAGO_FEATURIZE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KGN_FEATURES_SPATIAL_V7 22
#define KGN_FEATURES_GLOBAL_V7 19
#define KGN_MOVE_PASS (-1)
#define KGN_MOVE_NULL (-2)

typedef struct kgn_position {
  int32_t x_size, y_size;       /* at most 19 each, and at most the tensor's nn_x, nn_y */
  int32_t next_player;          /* 1 black, 2 white */
  /* Colours of the current board and of hist.getRecentBoard(1) and (2),
   * x_size * y_size each; a null pointer repeats the previous board. */
  const int8_t* colors[3];
  int32_t ko_point[3];          /* each board's Board::ko_loc as y * x_size + x, or -1 */
  /* Optional, per board: for each stone its chain's head and the next stone
   * of its chain's circular list (Board::chain_head, Board::next_in_chain),
   * as points; other entries are ignored. KataGo's ladder search walks chains
   * in this order and one of its early exits depends on it; without these
   * arrays (null) each chain is linked breadth-first from its first stone in
   * scan order, which can change a ladder feature in rare positions. */
  const int16_t* chain_head[3];
  const int16_t* chain_next[3];
  const uint8_t* super_ko_banned;            /* hist.superKoBanned per point, or null (none) */
  const uint8_t* ko_recap_blocked;           /* hist.koRecapBlocked per point, or null */
  const int8_t* second_encore_start_colors;  /* hist.secondEncoreStartColors per point, or null */
  /* The last num_moves (at most 5) entries of hist.moveHistory, oldest first:
   * point, KGN_MOVE_PASS or KGN_MOVE_NULL, and the player who moved. */
  int32_t num_moves;
  int32_t move_point[5];
  int32_t move_player[5];
  int32_t num_approx_valid_turns_this_phase;
  int32_t encore_phase;
  /* Rules (Rules::koRule, scoringRule, taxRule, multiStoneSuicideLegal) and hist.hasButton. */
  int32_t ko_rule, scoring_rule, tax_rule, multi_stone_suicide_legal, has_button;
  /* hist.currentSelfKomi(next_player, drawEquivalentWinsForWhite). */
  float self_komi;
  /* BoardHistory state for the position and the player to move:
   * passWouldEndGame, passWouldEndPhase, shouldSuppressEndGameFromFriendlyPass,
   * isGameFinished, isPastNormalPhaseEnd. */
  uint8_t pass_would_end_game, pass_would_end_phase, suppress_end_game_from_friendly_pass;
  uint8_t is_game_finished, is_past_normal_phase_end;
  /* MiscNNInputParams (nninputs.h:52-63). */
  uint8_t conservative_pass_and_is_root, enable_passing_hacks;
  double playout_doubling_advantage;
  int32_t max_history;          /* MiscNNInputParams::maxHistory (1000 by default) */
} kgn_position;

/* Featurizes n positions into nn_x by nn_y tensors exactly as
 * NNInputs::fillRowV7 does: spatial receives n * nn_x * nn_y * 22 floats
 * (NHWC if use_nhwc, else NCHW), global n * 19. num_threads worker threads
 * take the positions in runs of consecutive ones (0 = one per available
 * core). Returns 0, or -1 with a message in err on an invalid position. */
int32_t kgn_featurize(const kgn_position* positions, int32_t n, int32_t nn_x, int32_t nn_y, int32_t use_nhwc,
                      float* spatial, float* global_out, int32_t num_threads, char* err, int32_t errlen);

/* The boards' ladder searches are the featurizer's main cost, and KataGo's
 * fillRowV7 repeats them for the two previous boards of every position
 * (nninputs.cpp:2546-2566). Each thread keeps the ladder stones of the last
 * `entries` boards it searched (8 by default, KGN_FEATURIZE_MAX_CACHE at
 * most), keyed by everything the search reads (size, ko point, colours,
 * chain order), so a board that comes again (the board one move back is
 * usually the current board of the position featurized before; siblings of a
 * search share their parent) is not searched again. The rows are the same
 * with or without it. 0 turns it off. Returns the previous setting, or -1 for
 * an out-of-range value. No counterpart in the reference. */
#define KGN_FEATURIZE_MAX_CACHE 64
int32_t kgn_featurize_set_cache(int32_t entries);

#ifdef __cplusplus
}
#endif

#endif
