// Drives kgn_featurize (katago_amd/host/neuralnet/featurize.cpp) under the
// host sanitizers: reads positions from a whitespace-separated text file
// (written by tests/test_host_sanitizers.py from the featurizer fixture),
// featurizes each one alone on one thread, then every group of positions
// with the same tensor size in one call on four threads, checks that both
// give the same rows, and writes the single-position rows (NHWC spatial,
// then global, float32) to the output file for the test to compare with the
// fixture's expected bits.
//
// usage: featurize_stress <positions.txt> <out.bin>
#include "../../include/katago_featurize.h"

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <string>
#include <vector>

namespace {

struct Stored {
  int nnx = 0, nny = 0;
  kgn_position p{};
  std::vector<int8_t> colors[3];
  std::vector<int16_t> head[3], next[3];
  std::vector<uint8_t> superKo, koRecap;
  std::vector<int8_t> encoreColors;
  bool hasSuperKo = false, hasKoRecap = false, hasEncore = false;
};

template<typename V>
bool readArray(std::istream& in, int n, std::vector<V>& out) {
  out.resize(n);
  for(int i = 0; i < n; i++) {
    long v;
    if(!(in >> v)) return false;
    out[i] = (V)v;
  }
  return true;
}

bool readPosition(std::istream& in, Stored& s) {
  kgn_position& p = s.p;
  if(!(in >> s.nnx >> s.nny >> p.x_size >> p.y_size >> p.next_player)) return false;
  const int n = p.x_size * p.y_size;
  for(int k = 0; k < 3; k++)
    if(!readArray(in, n, s.colors[k])) return false;
  for(int k = 0; k < 3; k++)
    if(!(in >> p.ko_point[k])) return false;
  for(int k = 0; k < 3; k++)
    if(!readArray(in, n, s.head[k]) || !readArray(in, n, s.next[k])) return false;
  int flag;
  if(!(in >> flag)) return false;
  s.hasSuperKo = flag != 0;
  if(s.hasSuperKo && !readArray(in, n, s.superKo)) return false;
  if(!(in >> flag)) return false;
  s.hasKoRecap = flag != 0;
  if(s.hasKoRecap && !readArray(in, n, s.koRecap)) return false;
  if(!(in >> flag)) return false;
  s.hasEncore = flag != 0;
  if(s.hasEncore && !readArray(in, n, s.encoreColors)) return false;
  if(!(in >> p.num_moves)) return false;
  for(int k = 0; k < 5; k++)
    if(!(in >> p.move_point[k])) return false;
  for(int k = 0; k < 5; k++)
    if(!(in >> p.move_player[k])) return false;
  int u[7];
  std::string komi, doubling;
  if(!(in >> p.num_approx_valid_turns_this_phase >> p.encore_phase >> p.ko_rule >> p.scoring_rule >> p.tax_rule >>
       p.multi_stone_suicide_legal >> p.has_button >> komi))
    return false;
  for(int& v : u)
    if(!(in >> v)) return false;
  if(!(in >> doubling >> p.max_history)) return false;
  p.self_komi = std::strtof(komi.c_str(), nullptr);
  p.pass_would_end_game = (uint8_t)u[0];
  p.pass_would_end_phase = (uint8_t)u[1];
  p.suppress_end_game_from_friendly_pass = (uint8_t)u[2];
  p.is_game_finished = (uint8_t)u[3];
  p.is_past_normal_phase_end = (uint8_t)u[4];
  p.conservative_pass_and_is_root = (uint8_t)u[5];
  p.enable_passing_hacks = (uint8_t)u[6];
  p.playout_doubling_advantage = std::strtod(doubling.c_str(), nullptr);
  return true;
}

// Points the position's pointers at its own arrays (after the vectors
// stopped moving).
void link(Stored& s) {
  for(int k = 0; k < 3; k++) {
    s.p.colors[k] = s.colors[k].data();
    s.p.chain_head[k] = s.head[k].data();
    s.p.chain_next[k] = s.next[k].data();
  }
  s.p.super_ko_banned = s.hasSuperKo ? s.superKo.data() : nullptr;
  s.p.ko_recap_blocked = s.hasKoRecap ? s.koRecap.data() : nullptr;
  s.p.second_encore_start_colors = s.hasEncore ? s.encoreColors.data() : nullptr;
}

}  // namespace

int main(int argc, char** argv) {
  if(argc != 3) {
    std::fprintf(stderr, "usage: %s <positions.txt> <out.bin>\n", argv[0]);
    return 2;
  }
  std::ifstream in(argv[1]);
  std::vector<Stored> pos;
  for(;;) {
    Stored s;
    if(!readPosition(in, s)) break;
    pos.push_back(std::move(s));
  }
  for(Stored& s : pos) link(s);
  std::printf("positions %zu\n", pos.size());
  char err[512];
  std::vector<std::vector<float>> single(pos.size());
  for(size_t i = 0; i < pos.size(); i++) {
    const Stored& s = pos[i];
    std::vector<float> sp((size_t)s.nnx * s.nny * KGN_FEATURES_SPATIAL_V7), gl(KGN_FEATURES_GLOBAL_V7);
    if(kgn_featurize(&s.p, 1, s.nnx, s.nny, 1, sp.data(), gl.data(), 1, err, sizeof(err)) != 0) {
      std::fprintf(stderr, "position %zu: %s\n", i, err);
      return 1;
    }
    single[i] = sp;
    single[i].insert(single[i].end(), gl.begin(), gl.end());
  }
  // Batches of one tensor size on four worker threads.
  std::map<std::pair<int, int>, std::vector<size_t>> groups;
  for(size_t i = 0; i < pos.size(); i++) groups[{pos[i].nnx, pos[i].nny}].push_back(i);
  long mismatches = 0;
  for(const auto& [size, idx] : groups) {
    std::vector<kgn_position> batch;
    for(size_t i : idx) batch.push_back(pos[i].p);
    const size_t rowSp = (size_t)size.first * size.second * KGN_FEATURES_SPATIAL_V7;
    std::vector<float> sp(rowSp * batch.size()), gl((size_t)KGN_FEATURES_GLOBAL_V7 * batch.size());
    if(kgn_featurize(batch.data(), (int32_t)batch.size(), size.first, size.second, 1, sp.data(), gl.data(), 4, err, sizeof(err)) !=
       0) {
      std::fprintf(stderr, "batch %dx%d: %s\n", size.first, size.second, err);
      return 1;
    }
    for(size_t b = 0; b < idx.size(); b++) {
      const std::vector<float>& one = single[idx[b]];
      mismatches += std::memcmp(one.data(), sp.data() + b * rowSp, rowSp * sizeof(float)) != 0;
      mismatches += std::memcmp(one.data() + rowSp, gl.data() + b * KGN_FEATURES_GLOBAL_V7, KGN_FEATURES_GLOBAL_V7 * sizeof(float)) != 0;
    }
  }
  // An invalid position is refused with a message, not a crash.
  {
    kgn_position bad = pos.empty() ? kgn_position{} : pos[0].p;
    bad.x_size = 25;
    std::vector<float> sp(19 * 19 * KGN_FEATURES_SPATIAL_V7), gl(KGN_FEATURES_GLOBAL_V7);
    if(kgn_featurize(&bad, 1, 19, 19, 1, sp.data(), gl.data(), 1, err, sizeof(err)) == 0) {
      std::fprintf(stderr, "a 25-wide board was accepted\n");
      return 1;
    }
  }
  // Off-board ko points on each board, as the last row of a batch whose
  // output arrays end exactly at that row (an overrun is a sanitizer error).
  for(size_t i = 0; i < pos.size() && i < 64; i++) {
    const Stored& s = pos[i];
    for(int k = 0; k < 3; k++)
      for(int ko : {-7, s.p.x_size * s.p.y_size, 399, 100000}) {
        kgn_position bad[2] = {s.p, s.p};
        bad[1].ko_point[k] = ko;
        std::vector<float> sp((size_t)2 * s.nnx * s.nny * KGN_FEATURES_SPATIAL_V7), gl(2 * KGN_FEATURES_GLOBAL_V7);
        if(kgn_featurize(bad, 2, s.nnx, s.nny, 1, sp.data(), gl.data(), 1, err, sizeof(err)) == 0 &&
           (k == 0 || bad[1].colors[k] != nullptr)) {
          std::fprintf(stderr, "position %zu: ko point %d on board %d was accepted\n", i, ko, k);
          return 1;
        }
      }
  }
  std::FILE* f = std::fopen(argv[2], "wb");
  if(f == nullptr) return 1;
  for(const std::vector<float>& r : single) std::fwrite(r.data(), sizeof(float), r.size(), f);
  std::fclose(f);
  std::printf("batch mismatches %ld\n", mismatches);
  return mismatches == 0 ? 0 : 1;
}
