// TEST INFRASTRUCTURE ONLY. A driver, linked against KataGo's own game and
// featurizer sources compiled where they lie under /root/reference (recipe:
// oracle/Makefile.ref, output oracle/_ref/ref_featurize), that writes the
// neural-net input rows KataGo's NNEvaluator::evaluate would build
// (nneval.cpp:441-456: NNInputs::fillRowV3..V7) for given positions, plus
// what the evaluator's post-processing reads (history.isLegal per move,
// nneval.cpp:954-968). It is the checker for fixtures under tests/golden/
// and never part of the product.
//
// Input on stdin, one case per block:
//   case <name> <xSize> <ySize> <nnXLen> <nnYLen> <b|w> <inputsVersion> <rules>
//   <ySize lines of the board as Board::parseBoard reads it>
// and, for random positions reached by play:
//   game <name> <seed> <xSize> <ySize> <nnXLen> <nnYLen> <numMoves> <inputsVersion> <rules>
// and, to check this repository's featurizer (include/katago_featurize.h,
// linked in through katago_amd/host/neuralnet/featurizeadapter.cpp) against
// KataGo's own fillRowV7 on every position of a random game:
//   compare <name> <seed> <xSize> <ySize> <nnXLen> <nnYLen> <numMoves> <rules> <fixtureEvery>
// which prints a summary line and, every fixtureEvery positions, the
// position with KataGo's rows as a fixture line; and, to time both
// featurizers on the same positions (each on one thread):
//   time <name> <seed> <xSize> <ySize> <nnXLen> <nnYLen> <numMoves> <rules> <reps>
// which plays one random game, keeps every position, and prints the
// microseconds per position of KataGo's fillRowV7, of kgn_featurize over the
// prebuilt positions in one single-threaded call with its ladder cache off
// and on, and of positionFromHistory + kgn_featurize one position per call.
// and, for a position reached by a given move sequence (the canary
// positions of testnnevalcanary.cpp):
//   moves <name> <xSize> <ySize> <nnXLen> <nnYLen> <rules> <komi> <numMoves> {<b|w> <x> <y>}
// (x = y = -1 for a pass) which plays the moves with KataGo's BoardHistory,
// sets the komi (as BoardHistory::setKomi after the setup), checks this
// repository's featurizer against fillRowV7 on the position (a "compare"
// line) and emits the position as a "case" would.
// Output on stdout: one JSON object per position and line.
#include <chrono>
#include <cstdio>
#include <iostream>
#include <sstream>
#include <string>
#include <vector>

#include "../core/global.h"
#include "../core/rand.h"
#include "../game/board.h"
#include "../game/boardhistory.h"
#include "../game/rules.h"
#include "../neuralnet/nninputs.h"
#include "featurizeadapter.h"

using std::string;
using std::vector;

namespace {

int numSpatial(int version) {
  switch(version) {
    case 3: return NNInputs::NUM_FEATURES_SPATIAL_V3;
    case 4: return NNInputs::NUM_FEATURES_SPATIAL_V4;
    case 5: return NNInputs::NUM_FEATURES_SPATIAL_V5;
    case 6: return NNInputs::NUM_FEATURES_SPATIAL_V6;
    case 7: return NNInputs::NUM_FEATURES_SPATIAL_V7;
  }
  throw StringError("unknown inputs version");
}
int numGlobal(int version) {
  switch(version) {
    case 3: return NNInputs::NUM_FEATURES_GLOBAL_V3;
    case 4: return NNInputs::NUM_FEATURES_GLOBAL_V4;
    case 5: return NNInputs::NUM_FEATURES_GLOBAL_V5;
    case 6: return NNInputs::NUM_FEATURES_GLOBAL_V6;
    case 7: return NNInputs::NUM_FEATURES_GLOBAL_V7;
  }
  throw StringError("unknown inputs version");
}

Rules rulesNamed(const string& name) {
  if(name == "tromp-taylor") return Rules::getTrompTaylorish();
  return Rules::parseRules(name);
}

void floats(std::ostream& out, const vector<float>& v) {
  out << "[";
  for(size_t i = 0; i < v.size(); i++) {
    if(i) out << ",";
    char buf[32];
    snprintf(buf, sizeof(buf), "%.9g", v[i]);
    out << buf;
  }
  out << "]";
}

void emit(const string& name, const Board& board, const BoardHistory& hist, Player pla, int nnX, int nnY, int version) {
  MiscNNInputParams params;
  const int C = numSpatial(version), G = numGlobal(version);
  vector<float> spatial((size_t)C * nnX * nnY), global(G);
  const bool nhwc = true;
  switch(version) {
    case 3: NNInputs::fillRowV3(board, hist, pla, params, nnX, nnY, nhwc, spatial.data(), global.data()); break;
    case 4: NNInputs::fillRowV4(board, hist, pla, params, nnX, nnY, nhwc, spatial.data(), global.data()); break;
    case 5: NNInputs::fillRowV5(board, hist, pla, params, nnX, nnY, nhwc, spatial.data(), global.data()); break;
    case 6: NNInputs::fillRowV6(board, hist, pla, params, nnX, nnY, nhwc, spatial.data(), global.data()); break;
    default: NNInputs::fillRowV7(board, hist, pla, params, nnX, nnY, nhwc, spatial.data(), global.data()); break;
  }
  // Legal moves as the evaluator's post-processing sees them, pass last.
  vector<int> legal((size_t)nnX * nnY + 1, 0);
  for(int y = 0; y < board.y_size; y++)
    for(int x = 0; x < board.x_size; x++) {
      Loc loc = Location::getLoc(x, y, board.x_size);
      legal[NNPos::locToPos(loc, board.x_size, nnX, nnY)] = hist.isLegal(board, loc, pla) ? 1 : 0;
    }
  legal[NNPos::getPassPos(nnX, nnY)] = hist.isLegal(board, Board::PASS_LOC, pla) ? 1 : 0;
  std::ostringstream out;
  out << "{\"name\":\"" << name << "\",\"x\":" << board.x_size << ",\"y\":" << board.y_size << ",\"nnx\":" << nnX
      << ",\"nny\":" << nnY << ",\"pla\":\"" << (pla == P_WHITE ? "w" : "b") << "\",\"inputs_version\":" << version
      << ",\"no_result_disabled\":"
      << ((hist.rules.koRule != Rules::KO_SIMPLE && hist.rules.scoringRule != Rules::SCORING_TERRITORY) ? "true" : "false")
      << ",\"spatial_nhwc\":";
  floats(out, spatial);
  out << ",\"global\":";
  floats(out, global);
  out << ",\"legal\":[";
  for(size_t i = 0; i < legal.size(); i++) out << (i ? "," : "") << legal[i];
  out << "]}";
  std::cout << out.str() << std::endl;
}

void bits(std::ostream& out, const vector<float>& v) {
  // 0/1 values as a hex string, four values per digit, first value in the
  // high bit.
  static const char* hex = "0123456789abcdef";
  out << "\"";
  for(size_t i = 0; i < v.size(); i += 4) {
    int d = 0;
    for(int k = 0; k < 4; k++) d = d * 2 + (i + k < v.size() && v[i + k] != 0.0f ? 1 : 0);
    out << hex[d];
  }
  out << "\"";
}

template<typename T>
void ints(std::ostream& out, const T* v, int n) {
  out << "[";
  for(int i = 0; i < n; i++) out << (i ? "," : "") << (int)v[i];
  out << "]";
}

void fixture(const string& name, const kgn_position& pos, int nnX, int nnY, const vector<float>& spatial,
             const vector<float>& global) {
  std::ostringstream out;
  const int area = pos.x_size * pos.y_size;
  out << "{\"fixture\":\"" << name << "\",\"nnx\":" << nnX << ",\"nny\":" << nnY << ",\"x_size\":" << pos.x_size
      << ",\"y_size\":" << pos.y_size << ",\"next_player\":" << pos.next_player << ",\"colors\":[";
  for(int k = 0; k < 3; k++) {
    out << (k ? "," : "");
    ints(out, pos.colors[k], area);
  }
  out << "],\"chain_head\":[";
  for(int k = 0; k < 3; k++) {
    out << (k ? "," : "");
    ints(out, pos.chain_head[k], area);
  }
  out << "],\"chain_next\":[";
  for(int k = 0; k < 3; k++) {
    out << (k ? "," : "");
    ints(out, pos.chain_next[k], area);
  }
  out << "],\"ko_point\":";
  ints(out, pos.ko_point, 3);
  out << ",\"super_ko_banned\":";
  ints(out, pos.super_ko_banned, area);
  out << ",\"ko_recap_blocked\":";
  ints(out, pos.ko_recap_blocked, area);
  out << ",\"second_encore_start_colors\":";
  ints(out, pos.second_encore_start_colors, area);
  out << ",\"num_moves\":" << pos.num_moves << ",\"move_point\":";
  ints(out, pos.move_point, 5);
  out << ",\"move_player\":";
  ints(out, pos.move_player, 5);
  char komi[32];
  snprintf(komi, sizeof(komi), "%.9g", pos.self_komi);
  out << ",\"num_approx_valid_turns_this_phase\":" << pos.num_approx_valid_turns_this_phase
      << ",\"encore_phase\":" << pos.encore_phase << ",\"ko_rule\":" << pos.ko_rule << ",\"scoring_rule\":" << pos.scoring_rule
      << ",\"tax_rule\":" << pos.tax_rule << ",\"multi_stone_suicide_legal\":" << pos.multi_stone_suicide_legal
      << ",\"has_button\":" << pos.has_button << ",\"self_komi\":" << komi
      << ",\"pass_would_end_game\":" << (int)pos.pass_would_end_game << ",\"pass_would_end_phase\":" << (int)pos.pass_would_end_phase
      << ",\"suppress_end_game_from_friendly_pass\":" << (int)pos.suppress_end_game_from_friendly_pass
      << ",\"is_game_finished\":" << (int)pos.is_game_finished << ",\"is_past_normal_phase_end\":" << (int)pos.is_past_normal_phase_end
      << ",\"max_history\":" << pos.max_history << ",\"conservative_pass_and_is_root\":" << (int)pos.conservative_pass_and_is_root
      << ",\"enable_passing_hacks\":" << (int)pos.enable_passing_hacks
      << ",\"playout_doubling_advantage\":" << pos.playout_doubling_advantage << ",\"spatial_nhwc_bits\":";
  bits(out, spatial);
  out << ",\"global\":";
  floats(out, global);
  out << "}";
  std::cout << out.str() << std::endl;
}

// KataGo's fillRowV7 and this repository's featurizer on one position:
// the number of differing spatial and global values.
int compareOne(const string& name, const Board& board, const BoardHistory& hist, Player pla, int nnX, int nnY, bool emitFixture,
               string& firstDiff, int variant) {
  // Search-time parameters varied across positions (nninputs.h:52-63).
  MiscNNInputParams params;
  if(variant % 5 == 0) params.playoutDoublingAdvantage = (variant % 3 - 1) * 0.75;
  if(variant % 7 == 0) params.conservativePassAndIsRoot = true;
  if(variant % 11 == 0) params.enablePassingHacks = true;
  if(variant % 13 == 0) params.maxHistory = variant % 4;
  if(variant % 4 == 0) params.drawEquivalentWinsForWhite = 0.3;
  const int C = NNInputs::NUM_FEATURES_SPATIAL_V7, G = NNInputs::NUM_FEATURES_GLOBAL_V7;
  vector<float> refS((size_t)C * nnX * nnY), refG(G), mineS(refS.size()), mineG(G);
  NNInputs::fillRowV7(board, hist, pla, params, nnX, nnY, true, refS.data(), refG.data());
  kgn_position pos;
  HipBackend::PositionStorage storage;
  HipBackend::positionFromHistory(board, hist, pla, params, pos, storage);
  char err[512];
  if(kgn_featurize(&pos, 1, nnX, nnY, 1, mineS.data(), mineG.data(), 1, err, sizeof(err)) != 0)
    throw StringError(string("kgn_featurize failed: ") + err);
  int diffs = 0;
  for(size_t i = 0; i < refS.size(); i++)
    if(refS[i] != mineS[i]) {
      if(diffs++ == 0 && firstDiff.empty()) {
        const int c = (int)(i % C), p = (int)(i / C);
        firstDiff = name + ": spatial feature " + std::to_string(c) + " at (" + std::to_string(p % nnX) + "," +
                    std::to_string(p / nnX) + ") reference " + std::to_string(refS[i]) + " mine " + std::to_string(mineS[i]);
      }
    }
  for(int i = 0; i < G; i++)
    if(refG[i] != mineG[i]) {
      if(diffs++ == 0 && firstDiff.empty())
        firstDiff = name + ": global " + std::to_string(i) + " reference " + std::to_string(refG[i]) + " mine " + std::to_string(mineG[i]);
    }
  if(emitFixture) fixture(name, pos, nnX, nnY, refS, refG);
  return diffs;
}

// Random play as the compare command plays it: mostly legal moves, passes
// now and then, two forced passes at half, seven tenths and nine tenths.
Loc randomMove(const Board& board, const BoardHistory& hist, Player pla, Rand& rand, int m, int moves) {
  vector<Loc> cands;
  for(int y = 0; y < board.y_size; y++)
    for(int x = 0; x < board.x_size; x++) {
      Loc loc = Location::getLoc(x, y, board.x_size);
      if(hist.isLegal(board, loc, pla)) cands.push_back(loc);
    }
  const bool forcedPass = m == moves / 2 || m == moves / 2 + 1 || m == moves * 7 / 10 || m == moves * 7 / 10 + 1 ||
                          m == moves * 9 / 10 || m == moves * 9 / 10 + 1;
  return forcedPass || cands.empty() || rand.nextUInt(30) == 0 ? Board::PASS_LOC : cands[rand.nextUInt((uint32_t)cands.size())];
}

double secondsSince(std::chrono::steady_clock::time_point t0) {
  return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
}

void timeGame(const string& name, uint64_t seed, int xs, int ys, int nnX, int nnY, int moves, const string& rulesS, int reps) {
  Board board(xs, ys);
  Player pla = P_BLACK;
  BoardHistory hist(board, pla, rulesNamed(rulesS), 0);
  Rand rand(seed);
  vector<Board> boards;
  vector<BoardHistory> hists;
  vector<Player> plas;
  for(int m = 0; m <= moves; m++) {
    boards.push_back(board);
    hists.push_back(hist);
    plas.push_back(pla);
    if(m == moves || hist.isGameFinished) break;
    hist.makeBoardMoveAssumeLegal(board, randomMove(board, hist, pla, rand, m, moves), pla, nullptr);
    pla = getOpp(pla);
  }
  const int n = (int)boards.size();
  MiscNNInputParams params;
  const int C = NNInputs::NUM_FEATURES_SPATIAL_V7, G = NNInputs::NUM_FEATURES_GLOBAL_V7;
  const size_t rowS = (size_t)C * nnX * nnY;
  vector<float> spatial(rowS * n), global((size_t)G * n), sink(rowS), gsink(G);
  char err[512];

  auto t0 = std::chrono::steady_clock::now();
  for(int r = 0; r < reps; r++)
    for(int i = 0; i < n; i++)
      NNInputs::fillRowV7(boards[i], hists[i], plas[i], params, nnX, nnY, true, sink.data(), gsink.data());
  const double ref = secondsSince(t0) / ((double)reps * n);

  vector<kgn_position> pos(n);
  vector<HipBackend::PositionStorage> storage(n);
  for(int i = 0; i < n; i++) HipBackend::positionFromHistory(boards[i], hists[i], plas[i], params, pos[i], storage[i]);
  // kgn_featurize over the whole game in one single-threaded call, with the
  // ladder cache off and then on (emptied first: a cache size change clears
  // it, so no board of an earlier pass is found).
  double batch[2];
  for(int cached = 0; cached < 2; cached++) {
    kgn_featurize_set_cache(0);
    if(kgn_featurize(pos.data(), 1, nnX, nnY, 1, spatial.data(), global.data(), 1, err, sizeof(err)) != 0)
      throw StringError(string("kgn_featurize failed: ") + err);
    kgn_featurize_set_cache(cached ? 8 : 0);
    t0 = std::chrono::steady_clock::now();
    for(int r = 0; r < reps; r++) {
      if(r > 0 && cached) {
        kgn_featurize_set_cache(0);
        if(kgn_featurize(pos.data(), 1, nnX, nnY, 1, spatial.data(), global.data(), 1, err, sizeof(err)) != 0)
          throw StringError(string("kgn_featurize failed: ") + err);
        kgn_featurize_set_cache(8);
      }
      if(kgn_featurize(pos.data(), n, nnX, nnY, 1, spatial.data(), global.data(), 1, err, sizeof(err)) != 0)
        throw StringError(string("kgn_featurize failed: ") + err);
    }
    batch[cached] = secondsSince(t0) / ((double)reps * n);
  }
  // One position per call, converting each from KataGo's objects, as
  // NNEvaluator::evaluate would call it (cache on, emptied first).
  kgn_featurize_set_cache(0);
  kgn_featurize_set_cache(8);
  t0 = std::chrono::steady_clock::now();
  for(int i = 0; i < n; i++) {
    HipBackend::positionFromHistory(boards[i], hists[i], plas[i], params, pos[i], storage[i]);
    if(kgn_featurize(&pos[i], 1, nnX, nnY, 1, sink.data(), gsink.data(), 1, err, sizeof(err)) != 0)
      throw StringError(string("kgn_featurize failed: ") + err);
  }
  const double perCall = secondsSince(t0) / n;
  char line[512];
  snprintf(line, sizeof(line),
           "{\"timing\":\"%s\",\"positions\":%d,\"reps\":%d,\"fillRowV7_us\":%.3f,\"featurize_uncached_us\":%.3f,"
           "\"featurize_cached_us\":%.3f,\"adapter_plus_featurize_cached_us\":%.3f}",
           name.c_str(), n, reps, ref * 1e6, batch[0] * 1e6, batch[1] * 1e6, perCall * 1e6);
  std::cout << line << std::endl;
}

}  // namespace

int main() {
  Board::initHash();
  string word;
  while(std::cin >> word) {
    if(word == "case") {
      string name, plaS, rulesS;
      int xs, ys, nnX, nnY, version;
      std::cin >> name >> xs >> ys >> nnX >> nnY >> plaS >> version >> rulesS;
      string line, text;
      std::getline(std::cin, line);
      for(int y = 0; y < ys; y++) {
        std::getline(std::cin, line);
        text += line + "\n";
      }
      Board board = Board::parseBoard(xs, ys, text);
      Player pla = plaS == "w" ? P_WHITE : P_BLACK;
      BoardHistory hist(board, pla, rulesNamed(rulesS), 0);
      emit(name, board, hist, pla, nnX, nnY, version);
    }
    else if(word == "game") {
      string name, rulesS;
      uint64_t seed;
      int xs, ys, nnX, nnY, moves, version;
      std::cin >> name >> seed >> xs >> ys >> nnX >> nnY >> moves >> version >> rulesS;
      Board board(xs, ys);
      Player pla = P_BLACK;
      BoardHistory hist(board, pla, rulesNamed(rulesS), 0);
      Rand rand(seed);
      for(int m = 0; m < moves && !hist.isGameFinished; m++) {
        vector<Loc> cands;
        for(int y = 0; y < ys; y++)
          for(int x = 0; x < xs; x++) {
            Loc loc = Location::getLoc(x, y, xs);
            if(hist.isLegal(board, loc, pla)) cands.push_back(loc);
          }
        Loc loc = cands.empty() || rand.nextUInt(40) == 0 ? Board::PASS_LOC : cands[rand.nextUInt((uint32_t)cands.size())];
        hist.makeBoardMoveAssumeLegal(board, loc, pla, nullptr);
        pla = getOpp(pla);
      }
      emit(name, board, hist, pla, nnX, nnY, version);
    }
    else if(word == "compare") {
      string name, rulesS;
      uint64_t seed;
      int xs, ys, nnX, nnY, moves, every;
      std::cin >> name >> seed >> xs >> ys >> nnX >> nnY >> moves >> rulesS >> every;
      Board board(xs, ys);
      Player pla = P_BLACK;
      BoardHistory hist(board, pla, rulesNamed(rulesS), 0);
      Rand rand(seed);
      int positions = 0, mismatched = 0;
      string firstDiff;
      for(int m = 0; m <= moves; m++) {
        const string posName = name + "-" + std::to_string(m);
        const int d = compareOne(posName, board, hist, pla, nnX, nnY, every > 0 && m % every == 0, firstDiff, (int)(seed + m));
        positions++;
        mismatched += d > 0;
        if(m == moves || hist.isGameFinished) break;
        vector<Loc> cands;
        for(int y = 0; y < ys; y++)
          for(int x = 0; x < xs; x++) {
            Loc loc = Location::getLoc(x, y, xs);
            if(hist.isLegal(board, loc, pla)) cands.push_back(loc);
          }
        // Mostly random legal moves, passes now and then, and two passes in a
        // row at half, seven tenths and nine tenths of the game (which end the
        // game under area rules and start the encore phases under territory
        // rules).
        const bool forcedPass = m == moves / 2 || m == moves / 2 + 1 || m == moves * 7 / 10 || m == moves * 7 / 10 + 1 ||
                                m == moves * 9 / 10 || m == moves * 9 / 10 + 1;
        Loc loc = forcedPass || cands.empty() || rand.nextUInt(30) == 0 ? Board::PASS_LOC : cands[rand.nextUInt((uint32_t)cands.size())];
        hist.makeBoardMoveAssumeLegal(board, loc, pla, nullptr);
        pla = getOpp(pla);
      }
      std::cout << "{\"summary\":\"" << name << "\",\"positions\":" << positions << ",\"mismatched\":" << mismatched
                << ",\"first_diff\":\"" << firstDiff << "\"}" << std::endl;
    }
    else if(word == "moves") {
      string name, rulesS;
      int xs, ys, nnX, nnY, n;
      float komi;
      std::cin >> name >> xs >> ys >> nnX >> nnY >> rulesS >> komi >> n;
      Board board(xs, ys);
      Player pla = P_BLACK;
      BoardHistory hist(board, pla, rulesNamed(rulesS), 0);
      for(int m = 0; m < n; m++) {
        string c;
        int x, y;
        std::cin >> c >> x >> y;
        const Player mover = c == "w" ? P_WHITE : P_BLACK;
        const Loc loc = x < 0 ? Board::PASS_LOC : Location::getLoc(x, y, xs);
        if(!hist.isLegal(board, loc, mover)) throw StringError(name + ": illegal move " + std::to_string(m));
        hist.makeBoardMoveAssumeLegal(board, loc, mover, nullptr);
        pla = getOpp(mover);
      }
      hist.setKomi(komi);
      string firstDiff;
      const int d = compareOne(name, board, hist, pla, nnX, nnY, false, firstDiff, 1);
      std::cout << "{\"compare\":\"" << name << "\",\"differing\":" << d << ",\"first_diff\":\"" << firstDiff << "\"}"
                << std::endl;
      emit(name, board, hist, pla, nnX, nnY, 7);
    }
    else if(word == "time") {
      string name, rulesS;
      uint64_t seed;
      int xs, ys, nnX, nnY, moves, reps;
      std::cin >> name >> seed >> xs >> ys >> nnX >> nnY >> moves >> rulesS >> reps;
      timeGame(name, seed, xs, ys, nnX, nnY, moves, rulesS, reps);
    }
    else {
      std::cerr << "unknown record " << word << std::endl;
      return 1;
    }
  }
  return 0;
}
