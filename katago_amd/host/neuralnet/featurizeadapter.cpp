// See featurizeadapter.h. Reads only public members and methods of KataGo's
// Board (board.h) and BoardHistory (boardhistory.h).
#include "../neuralnet/featurizeadapter.h"

#include <algorithm>

namespace {

int pointOf(Loc loc, const Board& board) {
  if(loc == Board::PASS_LOC) return KGN_MOVE_PASS;
  if(loc == Board::NULL_LOC) return KGN_MOVE_NULL;
  return Location::getY(loc, board.x_size) * board.x_size + Location::getX(loc, board.x_size);
}

void copyBoard(const Board& b, int8_t* colors, int16_t* chainHead, int16_t* chainNext) {
  for(int y = 0; y < b.y_size; y++)
    for(int x = 0; x < b.x_size; x++) {
      const Loc loc = Location::getLoc(x, y, b.x_size);
      const int i = y * b.x_size + x;
      colors[i] = (int8_t)b.colors[loc];
      const bool stone = b.colors[loc] == C_BLACK || b.colors[loc] == C_WHITE;
      chainHead[i] = (int16_t)(stone ? pointOf(b.chain_head[loc], b) : -1);
      chainNext[i] = (int16_t)(stone ? pointOf(b.next_in_chain[loc], b) : -1);
    }
}

}  // namespace

void HipBackend::positionFromHistory(const Board& board, const BoardHistory& hist, Player nextPlayer,
                                     const MiscNNInputParams& params, kgn_position& pos, PositionStorage& st) {
  pos = kgn_position();
  const int xs = board.x_size, ys = board.y_size;
  pos.x_size = xs;
  pos.y_size = ys;
  pos.next_player = nextPlayer;
  const Board* boards[3] = {&board, &hist.getRecentBoard(1), &hist.getRecentBoard(2)};
  for(int k = 0; k < 3; k++) {
    copyBoard(*boards[k], st.colors[k], st.chainHead[k], st.chainNext[k]);
    pos.colors[k] = st.colors[k];
    pos.chain_head[k] = st.chainHead[k];
    pos.chain_next[k] = st.chainNext[k];
    pos.ko_point[k] = boards[k]->ko_loc == Board::NULL_LOC ? -1 : pointOf(boards[k]->ko_loc, *boards[k]);
  }
  for(int y = 0; y < ys; y++)
    for(int x = 0; x < xs; x++) {
      const Loc loc = Location::getLoc(x, y, xs);
      st.superKoBanned[y * xs + x] = hist.superKoBanned[loc] ? 1 : 0;
      st.koRecapBlocked[y * xs + x] = hist.koRecapBlocked[loc] ? 1 : 0;
      st.secondEncoreStartColors[y * xs + x] = (int8_t)hist.secondEncoreStartColors[loc];
    }
  pos.super_ko_banned = st.superKoBanned;
  pos.ko_recap_blocked = st.koRecapBlocked;
  pos.second_encore_start_colors = st.secondEncoreStartColors;
  const size_t len = hist.moveHistory.size();
  pos.num_moves = (int32_t)std::min<size_t>(5, len);
  for(int i = 0; i < pos.num_moves; i++) {
    const Move& m = hist.moveHistory[len - pos.num_moves + i];
    pos.move_point[i] = pointOf(m.loc, board);
    pos.move_player[i] = m.pla;
  }
  pos.num_approx_valid_turns_this_phase = hist.numApproxValidTurnsThisPhase;
  pos.encore_phase = hist.encorePhase;
  pos.ko_rule = hist.rules.koRule;
  pos.scoring_rule = hist.rules.scoringRule;
  pos.tax_rule = hist.rules.taxRule;
  pos.multi_stone_suicide_legal = hist.rules.multiStoneSuicideLegal ? 1 : 0;
  pos.has_button = hist.hasButton ? 1 : 0;
  pos.self_komi = hist.currentSelfKomi(nextPlayer, params.drawEquivalentWinsForWhite);
  pos.pass_would_end_game = hist.passWouldEndGame(board, nextPlayer) ? 1 : 0;
  pos.pass_would_end_phase = hist.passWouldEndPhase(board, nextPlayer) ? 1 : 0;
  pos.suppress_end_game_from_friendly_pass = hist.shouldSuppressEndGameFromFriendlyPass(board, nextPlayer) ? 1 : 0;
  pos.is_game_finished = hist.isGameFinished ? 1 : 0;
  pos.is_past_normal_phase_end = hist.isPastNormalPhaseEnd ? 1 : 0;
  pos.conservative_pass_and_is_root = params.conservativePassAndIsRoot ? 1 : 0;
  pos.enable_passing_hacks = params.enablePassingHacks ? 1 : 0;
  pos.playout_doubling_advantage = params.playoutDoublingAdvantage;
  pos.max_history = params.maxHistory;
}
