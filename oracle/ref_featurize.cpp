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
// Output on stdout: one JSON object per position and line.
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
    else {
      std::cerr << "unknown record " << word << std::endl;
      return 1;
    }
  }
  return 0;
}
