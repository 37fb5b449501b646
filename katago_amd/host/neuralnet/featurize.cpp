// Position featurizer: the input rows of KataGo's NNInputs::fillRowV7
// (/root/reference/cpp/neuralnet/nninputs.cpp:2273-2720) from board-state
// arrays (include/katago_featurize.h).
//
// The board analysis is this file's own: a padded board with incremental
// chains, on which the ladder search and the pass-alive area follow KataGo's
// rules exactly:
//  * ladders: Board::searchIsLadderCaptured and
//    searchIsLadderCapturedAttackerFirst2Libs (board.cpp:1520-1790) as
//    driven by iterLadders (nninputs.cpp:815-870): the same move generation,
//    base cases, ko handling, node budget and depth limit, moves played and
//    undone as KataGo's Board plays and undoes them;
//  * area: Board::calculateArea, calculateIndependentLifeArea and
//    calculateAreaForPla (Benson's algorithm with KataGo's big-territory
//    marking, board.cpp:1792-2250).
// The ladder search's move lists follow the order of each chain's circular
// list, and one of its early exits looks at a list's last entry, so the
// verdict can depend on that order: the board keeps it as KataGo's does, and
// takes the starting order from the caller (kgn_position::chain_head /
// chain_next, which KataGo's Board holds). A caller without it gets each
// chain linked breadth-first from its first stone in scan order, which can
// differ from KataGo in such positions (about one in ten thousand of random
// play's positions).
//
// Each thread keeps the ladder stones of the boards it searched last, keyed
// by the whole board, so the boards one and two moves back, which fillRowV7
// searches again for every position, are usually found instead.
#include "../../../include/katago_featurize.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

namespace {

constexpr int MAX_SIDE = 19;
constexpr int MAX_W = MAX_SIDE + 2;
constexpr int MAX_AREA = MAX_W * MAX_W;
// Every board is laid out on the largest board's padded grid, so the four
// neighbour offsets are constants: up, left, right, down (KataGo's
// adj_offsets order, board.cpp:36-45).
constexpr int STRIDE = MAX_W;
constexpr int ADJ[4] = {-STRIDE, -1, 1, STRIDE};
constexpr int NONE_KEY = -1;
constexpr int8_t EMPTY = 0, BLACK = 1, WHITE = 2, WALL = 3;
constexpr int NONE = -1;
constexpr int LADDER_NODE_BUDGET = 25000;  // board.cpp:1590

inline int8_t opponent(int8_t p) { return (int8_t)(3 - p); }

struct LadderFrame;

// One stone reported by iterLadders: a stone of a chain in inescapable
// atari or that can be put into one, and, for the first stone of a chain
// with two liberties, the attacker's working moves (at most two).
struct LadderHit {
  int16_t point;  // a point of the padded grid
  int8_t numWorking;
  int16_t working[2];
};

// A board's ladder stones, kept for boards that come again: the board one
// move back of a position is usually the current board of the position
// before it, and the siblings of a search share their parent. The key is
// everything the search reads: the size, the ko point, the colours and (when
// the caller gives them) each stone's chain head and successor.
struct LadderCacheEntry {
  bool valid = false;
  int xs = 0, ys = 0, ko = NONE_KEY;
  bool chains = false;
  int8_t colors[MAX_SIDE * MAX_SIDE];
  int16_t head[MAX_SIDE * MAX_SIDE];
  int16_t next[MAX_SIDE * MAX_SIDE];
  std::vector<LadderHit> hits;
};

// Per-thread scratch of the board routines: a stamped mark array for
// duplicate-free walks, the ladder search's stack, and the ladder cache.
struct Scratch {
  uint32_t mark[MAX_AREA] = {};
  uint32_t stamp = 0;
  // The move lists of every level of a ladder search, one after another
  // (a level's list starts where its parent's ends), addressed by index.
  std::vector<int> moves;
  std::vector<LadderFrame> frames;
  std::vector<int> working;
  std::vector<LadderCacheEntry> cache;
  size_t cacheNext = 0;  // the entry the next miss replaces
  uint32_t next() {
    if(++stamp == 0) {
      memset(mark, 0, sizeof(mark));
      stamp = 1;
    }
    return stamp;
  }
};

// A board with a wall border: point (x, y) is (y + 1) * STRIDE + x + 1. Each
// chain is a circular list through next[] whose order, and whose head, follow
// the same rules as KataGo's Board (board.cpp:990-1330): a move merges its
// neighbours by splicing the smaller chain in after the larger one's head,
// and undoing a move either unlinks the stone or rebuilds the split chains by
// depth-first walks. The ladder search walks chains in this order, and one of
// its early exits looks at the last entry of a move list built in it, so the
// order is part of the result. libs[] and size[] are valid at heads.
struct GoBoard {
  int xs = 0, ys = 0;
  int16_t ko = NONE;
  int8_t color[MAX_AREA];
  int16_t head[MAX_AREA];
  int16_t next[MAX_AREA];
  int16_t libs[MAX_AREA];
  int16_t size[MAX_AREA];

  struct Record {
    int16_t loc;
    int8_t pla;
    int16_t ko;
    uint8_t capDirs;  // bit d: the move captured in direction d; 0x10: suicide
  };

  static int at(int x, int y) { return (y + 1) * STRIDE + x + 1; }
  int atPoint(int point) const { return at(point % xs, point / xs); }
  int numLibs(int p) const { return libs[head[p]]; }

  // From colours, and optionally the chains' heads and links as points
  // (y * x_size + x) of KataGo's Board; without them each chain is linked in
  // breadth-first order from its first stone in scan order.
  void init(int xSize, int ySize, const int8_t* colors, int koPoint, const int16_t* chainHead, const int16_t* chainNext,
            Scratch& s) {
    // Board::ko_loc is a point of this board or none (-1); any other value
    // would address a feature plane outside the row.
    if(koPoint < -1 || koPoint >= xSize * ySize) throw std::runtime_error("featurize: ko_point off the board");
    xs = xSize;
    ys = ySize;
    for(int i = 0; i < MAX_AREA; i++) {
      color[i] = WALL;
      head[i] = (int16_t)i;
      next[i] = (int16_t)i;
      libs[i] = 0;
      size[i] = 0;
    }
    const int area = xs * ys;
    int16_t toGrid[MAX_SIDE * MAX_SIDE];
    for(int y = 0, i = 0; y < ys; y++)
      for(int x = 0; x < xs; x++, i++) {
        const int8_t c = colors[i];
        if(c != EMPTY && c != BLACK && c != WHITE) throw std::runtime_error("featurize: colour outside 0..2");
        toGrid[i] = (int16_t)at(x, y);
        color[toGrid[i]] = c;
      }
    if(chainHead != nullptr && chainNext != nullptr) {
      for(int i = 0; i < area; i++) {
        const int p = toGrid[i];
        if(color[p] == EMPTY) continue;
        const int h = chainHead[i], nx = chainNext[i];
        if(h < 0 || h >= area || nx < 0 || nx >= area) throw std::runtime_error("featurize: chain link off the board");
        head[p] = toGrid[h];
        next[p] = toGrid[nx];
      }
      // Each chain once from its head: every stone of the circle has the
      // chain's colour and head, and the circle closes within the board;
      // size and liberties are counted on the way.
      int stones = 0, reached = 0;
      for(int i = 0; i < area; i++) {
        const int p = toGrid[i];
        if(color[p] == EMPTY) continue;
        stones++;
        if(head[p] != p) continue;
        const uint32_t st = s.next();
        int n = 0, l = 0, cur = p;
        do {
          if(color[cur] != color[p] || head[cur] != p || ++n > area) throw std::runtime_error("featurize: inconsistent chain links");
          for(int d = 0; d < 4; d++) {
            const int a = cur + ADJ[d];
            if(color[a] == EMPTY && s.mark[a] != st) {
              s.mark[a] = st;
              l++;
            }
          }
          cur = next[cur];
        } while(cur != p);
        size[p] = (int16_t)n;
        libs[p] = (int16_t)l;
        reached += n;
      }
      // Every stone lies on its head's circle (the circles are disjoint).
      if(reached != stones) throw std::runtime_error("featurize: inconsistent chain links");
    }
    else {
      const uint32_t st = s.next();
      int16_t queue[MAX_AREA];
      for(int i = 0; i < area; i++) {
        const int p = toGrid[i];
        if(color[p] == EMPTY || s.mark[p] == st) continue;
        const int8_t c = color[p];
        int qh = 0, qt = 0;
        queue[qt++] = (int16_t)p;
        s.mark[p] = st;
        int prev = p, n = 0;
        while(qh < qt) {
          const int q = queue[qh++];
          head[q] = (int16_t)p;
          next[prev] = (int16_t)q;
          prev = q;
          n++;
          for(int d = 0; d < 4; d++) {
            const int a = q + ADJ[d];
            if(color[a] == c && s.mark[a] != st) {
              s.mark[a] = st;
              queue[qt++] = (int16_t)a;
            }
          }
        }
        next[prev] = (int16_t)p;
        size[p] = (int16_t)n;
      }
      for(int i = 0; i < area; i++) {
        const int p = toGrid[i];
        if(color[p] != EMPTY && head[p] == p) libs[p] = (int16_t)countLibs(p, s);
      }
    }
    ko = (int16_t)(koPoint < 0 ? NONE : toGrid[koPoint]);
  }

  int countLibs(int h, Scratch& s) const {
    const uint32_t st = s.next();
    int n = 0;
    int cur = h;
    do {
      for(int d = 0; d < 4; d++) {
        const int a = cur + ADJ[d];
        if(color[a] == EMPTY && s.mark[a] != st) {
          s.mark[a] = st;
          n++;
        }
      }
      cur = next[cur];
    } while(cur != h);
    return n;
  }

  // KataGo's mergeChains: the chain of b joins the chain of a unless b's is
  // larger; the smaller chain's circle goes in right after the larger head.
  void merge(int a, int b) {
    int h1 = head[a], h2 = head[b];
    if(size[h1] < size[h2]) std::swap(h1, h2);
    size[h1] = (int16_t)(size[h1] + size[h2]);
    int newLibs = 0;
    int last = h2;
    while(true) {
      for(int d = 0; d < 4; d++) {
        const int q = last + ADJ[d];
        if(color[q] == EMPTY && !isLibertyOf(q, h1)) newLibs++;
      }
      head[last] = (int16_t)h1;
      if(next[last] == h2) break;
      last = next[last];
    }
    libs[h1] = (int16_t)(libs[h1] + newLibs);
    next[last] = next[h1];
    next[h1] = (int16_t)h2;
  }

  bool isSuicide(int p, int8_t pla) const {
    const int8_t opp = opponent(pla);
    for(int d = 0; d < 4; d++) {
      const int a = p + ADJ[d];
      if(color[a] == EMPTY) return false;
      if(color[a] == pla && numLibs(a) > 1) return false;
      if(color[a] == opp && numLibs(a) == 1) return false;
    }
    return true;
  }

  // Whether point q is next to a stone of the chain headed by h.
  bool isLibertyOf(int q, int h) const {
    for(int d = 0; d < 4; d++) {
      const int a = q + ADJ[d];
      if(color[a] == color[h] && head[a] == h) return true;
    }
    return false;
  }

  // Adds delta to the liberties of each distinct chain of colour c next to q.
  void changeSurroundingLiberties(int q, int8_t c, int delta) {
    int seen[4];
    int n = 0;
    for(int d = 0; d < 4; d++) {
      const int a = q + ADJ[d];
      if(color[a] != c) continue;
      const int h = head[a];
      bool dup = false;
      for(int j = 0; j < n; j++) dup = dup || seen[j] == h;
      if(dup) continue;
      seen[n++] = h;
      libs[h] = (int16_t)(libs[h] + delta);
    }
  }

  // Removes a chain; the chains of the other colour next to it gain the
  // freed points as liberties. Returns the stones removed.
  int removeChain(int p) {
    const int8_t other = opponent(color[p]);
    int n = 0;
    int cur = p;
    do {
      color[cur] = EMPTY;
      changeSurroundingLiberties(cur, other, 1);
      n++;
      cur = next[cur];
    } while(cur != p);
    return n;
  }

  // Board::playMoveAssumeLegal (board.cpp:990-1080), liberties kept
  // incrementally.
  void play(int p, int8_t pla, Scratch& s) {
    (void)s;
    const int8_t opp = opponent(pla);
    color[p] = pla;
    head[p] = (int16_t)p;
    next[p] = (int16_t)p;
    size[p] = 1;
    libs[p] = (int16_t)immediateLibs(p);
    int captured = 0;
    int possibleKo = NONE;
    int oppSeen[4];
    int numOppSeen = 0;
    for(int d = 0; d < 4; d++) {
      const int a = p + ADJ[d];
      if(color[a] == pla) {
        if(head[a] == head[p]) continue;
        libs[head[a]]--;
        merge(a, p);
      }
      else if(color[a] == opp) {
        const int h = head[a];
        bool seen = false;
        for(int j = 0; j < numOppSeen; j++) seen = seen || oppSeen[j] == h;
        if(seen) continue;
        oppSeen[numOppSeen++] = h;
        libs[h]--;
        if(libs[h] == 0) {
          captured += removeChain(a);
          possibleKo = a;
        }
      }
    }
    const int hp = head[p];
    ko = (int16_t)((captured == 1 && size[hp] == 1 && libs[hp] == 1) ? possibleKo : NONE);
    if(libs[hp] == 0) removeChain(p);
  }

  // Board::playMoveRecorded (board.cpp:754-787).
  Record playRecorded(int p, int8_t pla, Scratch& s) {
    Record r;
    r.loc = (int16_t)p;
    r.pla = pla;
    r.ko = ko;
    r.capDirs = 0;
    const int8_t opp = opponent(pla);
    for(int d = 0; d < 4; d++) {
      const int a = p + ADJ[d];
      if(color[a] == opp && numLibs(a) == 1) r.capDirs |= (uint8_t)(1 << d);
    }
    if(r.capDirs == 0 && isSuicide(p, pla)) r.capDirs = 0x10;
    play(p, pla, s);
    return r;
  }

  // KataGo's addChainHelper / rebuildChainHelper: depth-first over the
  // neighbours in adjacency order, each stone linked to the tail so far.
  int addChainWalk(int h, int tail, int p, int8_t pla) {
    color[p] = pla;
    head[p] = (int16_t)h;
    size[h]++;
    next[p] = (int16_t)tail;
    changeSurroundingLiberties(p, opponent(pla), -1);
    int nextTail = p;
    for(int d = 0; d < 4; d++)
      if(color[p + ADJ[d]] == EMPTY) nextTail = addChainWalk(h, nextTail, p + ADJ[d], pla);
    return nextTail;
  }
  // A chain refilled by an undo starts with no liberties; the undone move's
  // point gives it its one.
  void addChain(int p, int8_t pla) {
    size[p] = 0;
    libs[p] = 0;
    next[p] = (int16_t)addChainWalk(p, p, p, pla);
  }
  static constexpr int16_t UNLINKED = -2;
  int rebuildWalk(int h, int tail, int p, int8_t pla) {
    int add = 0;
    for(int d = 0; d < 4; d++) {
      const int q = p + ADJ[d];
      if(color[q] == EMPTY && !isLibertyOf(q, h)) add++;
    }
    libs[h] = (int16_t)(libs[h] + add);
    head[p] = (int16_t)h;
    size[h]++;
    next[p] = (int16_t)tail;
    int nextTail = p;
    for(int d = 0; d < 4; d++) {
      const int a = p + ADJ[d];
      if(color[a] == pla && head[a] != h) nextTail = rebuildWalk(h, nextTail, a, pla);
    }
    return nextTail;
  }
  void rebuildChain(int p, int8_t pla) {
    size[p] = 0;
    libs[p] = 0;
    next[p] = (int16_t)rebuildWalk(p, p, p, pla);
  }

  // Board::undo (board.cpp:789-907), liberties kept incrementally.
  void undo(const Record& r, Scratch& s) {
    (void)s;
    ko = r.ko;
    const int p = r.loc;
    const int8_t opp = opponent(r.pla);
    for(int d = 0; d < 4; d++) {
      const int a = p + ADJ[d];
      if((r.capDirs & (1 << d)) && color[a] == EMPTY) addChain(a, opp);
    }
    if(r.capDirs == 0x10) addChain(p, r.pla);
    color[p] = EMPTY;
    changeSurroundingLiberties(p, opp, 1);
    const int h = head[p];
    if(size[h] > 1) {
      int neighbours = 0;
      for(int d = 0; d < 4; d++) neighbours += color[p + ADJ[d]] == r.pla;
      if(neighbours <= 1) {
        int hh = h;
        if(hh == p) {
          const int newHead = next[p];
          int cur = p;
          do {
            head[cur] = (int16_t)newHead;
            cur = next[cur];
          } while(cur != p);
          size[newHead] = size[hh];
          libs[newHead] = libs[hh];
          hh = newHead;
        }
        int cur = hh;
        while(next[cur] != p) cur = next[cur];
        next[cur] = next[p];
        int delta = 1;
        for(int d = 0; d < 4; d++) {
          const int q = p + ADJ[d];
          if(color[q] == EMPTY && !isLibertyOf(q, hh)) delta--;
        }
        libs[hh] = (int16_t)(libs[hh] + delta);
        size[hh]--;
      }
      else {
        int cur = p;
        do {
          head[cur] = UNLINKED;
          cur = next[cur];
        } while(cur != p);
        for(int d = 0; d < 4; d++) {
          const int a = p + ADJ[d];
          if(color[a] == r.pla && head[a] == UNLINKED) rebuildChain(a, r.pla);
        }
      }
    }
  }

  // Board::isLegal with isMultiStoneSuicideLegal false (board.cpp:283-305,441-452).
  bool isLegalNoSuicide(int p, int8_t pla) const {
    if(color[p] != EMPTY || p == ko) return false;
    return !isSuicide(p, pla);
  }

  int immediateLibs(int p) const {
    int n = 0;
    for(int d = 0; d < 4; d++) n += color[p + ADJ[d]] == EMPTY;
    return n;
  }

  bool isAdjacentTo(int p, int8_t pla) const {
    for(int d = 0; d < 4; d++)
      if(color[p + ADJ[d]] == pla) return true;
    return false;
  }

  bool isAdjacentToHead(int8_t pla, int p, int h) const {
    for(int d = 0; d < 4; d++) {
      const int a = p + ADJ[d];
      if(color[a] == pla && head[a] == h) return true;
    }
    return false;
  }
};

// ---------------------------------------------------------------------------
// Ladders (board.cpp:1428-1790).

// One level of a ladder search: its move list (a range of Scratch::moves),
// the next move to try, and the record of the move being searched below it.
struct LadderFrame {
  int start, len, cur;
  bool defender;
  GoBoard::Record rec;
};

struct Ladder {
  Scratch& s;
  explicit Ladder(Scratch& sc) : s(sc) {}

  // Board::findLiberties: the liberties of the chain at p not already in
  // list[0..len), appended in chain order starting from the stone p itself.
  static void findLiberties(const GoBoard& b, int p, int* list, int& len) {
    int cur = p;
    do {
      for(int d = 0; d < 4; d++) {
        const int a = cur + ADJ[d];
        if(b.color[a] == EMPTY && std::find(list, list + len, a) == list + len) list[len++] = a;
      }
      cur = b.next[cur];
    } while(cur != p);
  }

  // Board::findLibertyGainingCaptures: liberties of the opponent chains in
  // atari next to the chain at p, without repeats, appended to the list.
  void libertyGainingCaptures(const GoBoard& b, int p, int* list, int& len) {
    const int8_t opp = opponent(b.color[p]);
    const uint32_t st = s.next();  // marks the opponent heads already looked at
    int cur = p;
    do {
      for(int d = 0; d < 4; d++) {
        const int a = cur + ADJ[d];
        if(b.color[a] != opp) continue;
        const int ah = b.head[a];
        if(b.libs[ah] != 1 || s.mark[ah] == st) continue;
        s.mark[ah] = st;
        findLiberties(b, a, list, len);
      }
      cur = b.next[cur];
    } while(cur != p);
  }

  bool hasLibertyGainingCaptures(const GoBoard& b, int p) const {
    const int8_t opp = opponent(b.color[p]);
    int cur = p;
    do {
      for(int d = 0; d < 4; d++) {
        const int a = cur + ADJ[d];
        if(b.color[a] == opp && b.numLibs(a) == 1) return true;
      }
      cur = b.next[cur];
    } while(cur != p);
    return false;
  }

  // Board::getBoundNumLibertiesAfterPlay (board.cpp:307-342).
  static void boundLibsAfterPlay(const GoBoard& b, int p, int8_t pla, int& lower, int& upper) {
    const int8_t opp = opponent(pla);
    int immediate = 0, caps = 0, capStones = 0, connSum = 0, connMax = 0;
    for(int d = 0; d < 4; d++) {
      const int a = p + ADJ[d];
      if(b.color[a] == EMPTY) {
        immediate++;
      }
      else if(b.color[a] == opp) {
        if(b.numLibs(a) == 1) {
          caps++;
          capStones += b.size[b.head[a]];
        }
      }
      else if(b.color[a] == pla) {
        const int conn = b.numLibs(a) - 1;
        connSum += conn;
        connMax = std::max(connMax, conn);
      }
    }
    lower = caps + std::max(connMax, immediate);
    upper = immediate + capStones + connSum;
  }

  // Board::getNumLibertiesAfterPlay (board.cpp:344-429), capped at max
  // (at most 3 here: the list below holds fewer than max points).
  static int libsAfterPlay(const GoBoard& b, int p, int8_t pla, int max) {
    const int8_t opp = opponent(pla);
    int found[4];
    int n = 0;
    int capHeads[4];
    int numCap = 0;
    for(int d = 0; d < 4; d++) {
      const int a = p + ADJ[d];
      if(b.color[a] == EMPTY) {
        found[n++] = a;
        if(n >= max) return max;
      }
      else if(b.color[a] == opp && b.numLibs(a) == 1) {
        found[n++] = a;
        if(n >= max) return max;
        const int h = b.head[a];
        bool seen = false;
        for(int j = 0; j < numCap; j++) seen = seen || capHeads[j] == h;
        if(!seen) capHeads[numCap++] = h;
      }
    }
    auto wouldBeEmpty = [&](int q) {
      if(b.color[q] == EMPTY) return true;
      if(b.color[q] == opp)
        for(int j = 0; j < numCap; j++)
          if(capHeads[j] == b.head[q]) return true;
      return false;
    };
    int connHeads[4];
    int numConn = 0;
    for(int d = 0; d < 4; d++) {
      const int a = p + ADJ[d];
      if(b.color[a] != pla) continue;
      const int h = b.head[a];
      bool seen = false;
      for(int j = 0; j < numConn; j++) seen = seen || connHeads[j] == h;
      if(seen) continue;
      connHeads[numConn++] = h;
      int cur = a;
      do {
        for(int k = 0; k < 4; k++) {
          const int q = cur + ADJ[k];
          if(q == p || !wouldBeEmpty(q)) continue;
          bool counted = false;
          for(int l = 0; l < n; l++) counted = counted || found[l] == q;
          if(!counted) {
            found[n++] = q;
            if(n >= max) return max;
          }
        }
        cur = b.next[cur];
      } while(cur != a);
    }
    return n;
  }

  // Board::wouldBeKoCapture (board.cpp:518-542).
  static bool wouldBeKoCapture(const GoBoard& b, int p, int8_t pla) {
    if(b.color[p] != EMPTY) return false;
    const int8_t opp = opponent(pla);
    int capturable = NONE;
    for(int d = 0; d < 4; d++) {
      const int a = p + ADJ[d];
      if(b.color[a] != WALL && b.color[a] != opp) return false;
      if(b.color[a] == opp && b.numLibs(a) == 1) {
        if(capturable != NONE) return false;
        capturable = a;
      }
    }
    return capturable != NONE && b.size[b.head[capturable]] == 1;
  }

  // Board::countHeuristicConnectionLibertiesX2 (board.cpp:1095-1109).
  static int connectionLibsX2(const GoBoard& b, int p, int8_t pla) {
    int n = 0;
    for(int d = 0; d < 4; d++) {
      const int a = p + ADJ[d];
      if(b.color[a] == pla) {
        const int l = b.numLibs(a);
        if(l > 1) n += l * 2 - 3;
      }
    }
    return n;
  }

  static bool areAdjacent(const GoBoard& b, int p, int q) {
    const int d = p > q ? p - q : q - p;
    return d == 1 || d == STRIDE;
  }

  // At most this many moves in one level's list: the defender's liberty and
  // one per opponent chain in atari around it.
  static constexpr int MAX_LIST = MAX_SIDE * MAX_SIDE + 1;

  // Entering a level of the search (board.cpp:1630-1720): either the level's
  // verdict (1 captured, 0 escapes) or -1 with its move list in
  // s.moves[start .. start + len).
  int enter(GoBoard& b, int target, int8_t defender, bool isDefender, size_t start, int& len) {
    const int8_t attacker = opponent(defender);
    const int libs = b.numLibs(target);
    if(!isDefender && libs <= 1) return 1;
    if(!isDefender && libs >= 3) return 0;
    if(isDefender && libs >= 2) return 0;
    if(isDefender && b.ko != NONE) return 0;
    if(s.moves.size() < start + MAX_LIST) s.moves.resize(start + MAX_LIST + 4096);
    int* m = s.moves.data() + start;
    len = 0;
    if(isDefender) {
      // Captures first, then the chain's liberty unless it is one of them;
      // the bound below is taken at the list's last entry.
      libertyGainingCaptures(b, target, m, len);
      findLiberties(b, target, m, len);
      int lower, upper;
      boundLibsAfterPlay(b, m[len - 1], defender, lower, upper);
      if(lower >= 3) return 0;
      if(len == 1 && upper <= 1) return 1;
    }
    else {
      findLiberties(b, target, m, len);
      int libs0 = b.immediateLibs(m[0]);
      int libs1 = b.immediateLibs(m[1]);
      if(libs0 == 0 && libs1 == 0 && wouldBeKoCapture(b, m[0], attacker) && wouldBeKoCapture(b, m[1], attacker)) {
        if(libsAfterPlay(b, m[0], defender, 3) <= 2 && libsAfterPlay(b, m[1], defender, 3) <= 2) {
          if(!hasLibertyGainingCaptures(b, target)) return 1;
        }
      }
      if(!areAdjacent(b, m[0], m[1])) {
        if(libs0 >= 3 && libs1 >= 3) return 0;
        else if(libs0 >= 3) len = 1;
        else if(libs1 >= 3) {
          m[0] = m[1];
          len = 1;
        }
      }
      if(len > 1) {
        libs0 = libs0 * 2 + connectionLibsX2(b, m[0], defender);
        libs1 = libs1 * 2 + connectionLibsX2(b, m[1], defender);
        if(libs1 > libs0) std::swap(m[0], m[1]);
      }
    }
    return -1;
  }

  // Board::searchIsLadderCaptured (board.cpp:1567-1790): whether the chain
  // at p is captured with best play, searched depth first over an explicit
  // stack. The defender moves at even depths when defFirst. The search
  // gives up (the chain escapes) after LADDER_NODE_BUDGET moves, undoing
  // every move but leaving the root's ko point cleared, as the reference's
  // budget exit does.
  bool captured(GoBoard& b, int p, bool defFirst) {
    if(b.color[p] != BLACK && b.color[p] != WHITE) return false;
    const int libs0 = b.numLibs(p);
    if(libs0 > 2 || (defFirst && libs0 > 1)) return false;
    const int8_t defender = b.color[p];
    const int stackSize = b.xs * b.ys * 3 / 2 + 1;
    if((int)s.frames.size() < stackSize) s.frames.resize(stackSize);
    LadderFrame* f = s.frames.data();
    const int16_t savedKo = b.ko;
    if(defFirst) b.ko = NONE;
    int nodes = 0;
    int depth = 0;
    bool r = false;
    // Undoes the moves of levels 0..depth-1: the budget exit.
    auto giveUp = [&]() {
      for(int d = depth - 1; d >= 0; d--) b.undo(f[d].rec, s);
      return false;
    };
    while(true) {
      // Enter level `depth`.
      bool decided = true;
      if(depth >= stackSize - 1) {
        r = true;
      }
      else {
        if(nodes >= LADDER_NODE_BUDGET) return giveUp();
        LadderFrame& fr = f[depth];
        fr.defender = defFirst ? (depth % 2 == 0) : (depth % 2 == 1);
        fr.start = depth == 0 ? 0 : f[depth - 1].start + f[depth - 1].len;
        int len = 0;
        const int v = enter(b, p, defender, fr.defender, (size_t)fr.start, len);
        if(v >= 0) {
          r = v == 1;
        }
        else {
          fr.len = len;
          fr.cur = 0;
          decided = false;
        }
      }
      // Unwind decided levels and pick the next move to search.
      while(true) {
        if(decided) {
          if(depth == 0) {
            b.ko = savedKo;
            return r;
          }
          depth--;
          LadderFrame& fr = f[depth];
          b.undo(fr.rec, s);
          if(nodes >= LADDER_NODE_BUDGET) return giveUp();
          if(fr.defender != r) {  // the defender escaped, or the attacker captured
            continue;
          }
        }
        LadderFrame& fr = f[depth];
        const int8_t mover = fr.defender ? defender : opponent(defender);
        bool played = false;
        while(fr.cur < fr.len) {
          const int i = fr.cur++;
          if(i > 0 && nodes >= LADDER_NODE_BUDGET) return giveUp();
          const int mv = s.moves[(size_t)fr.start + i];
          if(!b.isLegalNoSuicide(mv, mover)) continue;
          fr.rec = b.playRecorded(mv, mover, s);
          nodes++;
          played = true;
          break;
        }
        if(played) break;
        r = fr.defender;  // every move tried: the defender escaped none / the attacker captured with none
        decided = true;
      }
      depth++;
    }
  }

  // Board::searchIsLadderCapturedAttackerFirst2Libs (board.cpp:1520-1565).
  bool capturedAttackerFirst2Libs(GoBoard& b, int p, std::vector<int>& working) {
    working.clear();
    if(b.color[p] != BLACK && b.color[p] != WHITE) return false;
    if(b.numLibs(p) != 2) return false;
    const int8_t opp = opponent(b.color[p]);
    int libs[2];
    int n = 0;
    int cur = p;
    do {
      for(int d = 0; d < 4 && n < 2; d++) {
        const int a = cur + ADJ[d];
        if(b.color[a] == EMPTY && (n == 0 || libs[0] != a)) libs[n++] = a;
      }
      cur = b.next[cur];
    } while(cur != p && n < 2);
    if(n < 2) return false;
    bool works[2] = {false, false};
    for(int i = 0; i < 2; i++) {
      if(!b.isLegalNoSuicide(libs[i], opp)) continue;
      const GoBoard::Record rec = b.playRecorded(libs[i], opp, s);
      works[i] = captured(b, p, true);
      b.undo(rec, s);
    }
    if(works[0]) working.push_back(libs[0]);
    if(works[1]) working.push_back(libs[1]);
    return works[0] || works[1];
  }
};

// iterLadders (nninputs.cpp:815-870): f(point, workingMoves) for each stone of
// a chain in inescapable atari or that can be put into one.
template<typename F>
void iterLadders(const GoBoard& board, Scratch& s, F&& f) {
  int solvedHeads[MAX_AREA];
  bool solvedValue[MAX_AREA];
  int numSolved = 0;
  GoBoard copy = board;
  Ladder ladder(s);
  std::vector<int>& working = s.working;
  for(int y = 0; y < board.ys; y++)
    for(int x = 0; x < board.xs; x++) {
      const int p = board.at(x, y);
      if(board.color[p] != BLACK && board.color[p] != WHITE) continue;
      const int libs = board.numLibs(p);
      if(libs != 1 && libs != 2) continue;
      const int h = board.head[p];
      int found = -1;
      for(int i = 0; i < numSolved; i++)
        if(solvedHeads[i] == h) {
          found = i;
          break;
        }
      if(found >= 0) {
        if(solvedValue[found]) {
          working.clear();
          f(p, working);
        }
        continue;
      }
      bool laddered;
      if(libs == 1) {
        laddered = ladder.captured(copy, copy.at(x, y), true);
      }
      else {
        working.clear();
        laddered = ladder.capturedAttackerFirst2Libs(copy, copy.at(x, y), working);
      }
      solvedHeads[numSolved] = h;
      solvedValue[numSolved] = laddered;
      numSolved++;
      if(laddered) f(p, working);
    }
}

// The stones iterLadders reports on a board, with the working moves of the
// first stone of each chain that has two liberties.
void ladderHits(const GoBoard& board, Scratch& s, std::vector<LadderHit>& out) {
  out.clear();
  iterLadders(board, s, [&](int p, const std::vector<int>& working) {
    LadderHit h;
    h.point = (int16_t)p;
    h.numWorking = 0;
    h.working[0] = h.working[1] = 0;
    if(board.numLibs(p) == 2)
      for(size_t k = 0; k < working.size() && k < 2; k++) h.working[h.numWorking++] = (int16_t)working[k];
    out.push_back(h);
  });
}

std::atomic<int> g_ladderCacheEntries{8};

// The ladder stones of board k of a position: from this thread's cache when
// the same board (size, ko point, colours, chain order) was analysed before,
// else computed (on `ready` when the caller has built the board) and cached.
// The result is valid until the next call on this thread.
const std::vector<LadderHit>& boardLadders(const kgn_position& pos, int k, const GoBoard* ready, Scratch& s) {
  const int xs = pos.x_size, ys = pos.y_size, area = xs * ys;
  const int8_t* colors = pos.colors[k];
  const int16_t* ch = pos.chain_head[k];
  const int16_t* cn = pos.chain_next[k];
  const bool chains = ch != nullptr && cn != nullptr;
  const int ko = pos.ko_point[k];
  auto compute = [&](std::vector<LadderHit>& out) {
    if(ready != nullptr) {
      ladderHits(*ready, s, out);
    }
    else {
      GoBoard b;
      b.init(xs, ys, colors, ko, ch, cn, s);
      ladderHits(b, s, out);
    }
  };
  const int cap = g_ladderCacheEntries.load(std::memory_order_relaxed);
  if(cap <= 0) {
    s.cache.clear();
    static thread_local std::vector<LadderHit> uncached;
    compute(uncached);
    return uncached;
  }
  if((int)s.cache.size() != cap) {
    s.cache.assign((size_t)cap, LadderCacheEntry());
    s.cacheNext = 0;
  }
  for(LadderCacheEntry& e : s.cache) {
    if(!e.valid || e.xs != xs || e.ys != ys || e.ko != ko || e.chains != chains) continue;
    if(memcmp(e.colors, colors, (size_t)area) != 0) continue;
    bool same = true;
    if(chains)
      for(int i = 0; i < area && same; i++) same = colors[i] == EMPTY || (e.head[i] == ch[i] && e.next[i] == cn[i]);
    if(same) return e.hits;
  }
  LadderCacheEntry& e = s.cache[s.cacheNext];
  s.cacheNext = (s.cacheNext + 1) % (size_t)cap;
  e.valid = false;  // until the board has been checked and searched
  compute(e.hits);
  e.xs = xs;
  e.ys = ys;
  e.ko = ko;
  e.chains = chains;
  memcpy(e.colors, colors, (size_t)area);
  for(int i = 0; i < area; i++) {
    const bool stone = chains && colors[i] != EMPTY;
    e.head[i] = stone ? ch[i] : 0;
    e.next[i] = stone ? cn[i] : 0;
  }
  e.valid = true;
  return e.hits;
}

// ---------------------------------------------------------------------------
// Pass-alive area (board.cpp:1792-2250).

void areaForPla(const GoBoard& b, int8_t pla, bool safeBig, bool unsafeBig, bool msl, int8_t* result) {
  const int8_t opp = opponent(pla);
  int16_t regionOf[MAX_AREA];
  int16_t nextInRegion[MAX_AREA];
  bool bordersDeadByHead[MAX_AREA];
  for(int i = 0; i < MAX_AREA; i++) {
    regionOf[i] = -1;
    nextInRegion[i] = 0;
    bordersDeadByHead[i] = false;
  }
  constexpr int maxRegions = (MAX_SIDE * MAX_SIDE + 1) / 2 + 1;
  int vital[maxRegions * 4];
  int vitalTotal = 0;
  int numRegions = 0;
  int regionHead[maxRegions];
  int vitalStart[maxRegions];
  int vitalLen[maxRegions];
  int internal[maxRegions];
  bool containsOpp[maxRegions];
  int queue[MAX_AREA];

  auto build = [&](int first, int r) -> int {
    int tail = first;
    bool anyVital = vitalLen[r] > 0;
    int qh = 0, qt = 1;
    queue[0] = first;
    regionOf[first] = (int16_t)r;
    while(qh != qt) {
      const int p = queue[qh++];
      if(anyVital && (msl || b.color[p] == EMPTY)) {
        int keep = 0;
        for(int i = 0; i < vitalLen[r]; i++)
          if(b.isAdjacentToHead(pla, p, vital[vitalStart[r] + i])) vital[vitalStart[r] + keep++] = vital[vitalStart[r] + i];
        vitalLen[r] = keep;
        anyVital = keep > 0;
      }
      if(internal[r] < 2 && !b.isAdjacentTo(p, pla)) internal[r]++;
      if(b.color[p] == opp) containsOpp[r] = true;
      nextInRegion[p] = (int16_t)tail;
      tail = p;
      for(int d = 0; d < 4; d++) {
        const int a = p + ADJ[d];
        if((b.color[a] == EMPTY || b.color[a] == opp) && regionOf[a] == -1) {
          queue[qt++] = a;
          regionOf[a] = (int16_t)r;
        }
      }
    }
    return tail;
  };

  bool anyPla = false;
  for(int y = 0; y < b.ys; y++)
    for(int x = 0; x < b.xs; x++) {
      const int p = b.at(x, y);
      if(regionOf[p] != -1) continue;
      if(b.color[p] != EMPTY) {
        anyPla = anyPla || b.color[p] == pla;
        continue;
      }
      const int r = numRegions++;
      regionHead[r] = p;
      vitalStart[r] = vitalTotal;
      vitalLen[r] = 0;
      internal[r] = 0;
      containsOpp[r] = false;
      for(int d = 0; d < 4; d++) {
        const int a = p + ADJ[d];
        if(b.color[a] != pla) continue;
        const int h = b.head[a];
        bool present = false;
        for(int j = 0; j < vitalLen[r]; j++) present = present || vital[vitalStart[r] + j] == h;
        if(!present) vital[vitalStart[r] + vitalLen[r]++] = h;
      }
      const int tail = build(p, r);
      nextInRegion[p] = (int16_t)tail;
      vitalTotal += vitalLen[r];
    }

  int plaHeads[MAX_SIDE * MAX_SIDE];
  int numPlaHeads = 0;
  for(int p = 0; p < MAX_AREA; p++)
    if(b.color[p] == pla && b.head[p] == p) plaHeads[numPlaHeads++] = p;
  bool killed[MAX_SIDE * MAX_SIDE];
  std::fill(killed, killed + numPlaHeads, false);
  int vitalCount[MAX_AREA];
  for(int i = 0; i < numPlaHeads; i++) vitalCount[plaHeads[i]] = 0;
  for(int r = 0; r < numRegions; r++)
    for(int j = 0; j < vitalLen[r]; j++) vitalCount[vital[vitalStart[r] + j]]++;

  // Benson: kill chains with fewer than two vital regions, until none dies.
  while(true) {
    bool any = false;
    for(int i = 0; i < numPlaHeads; i++) {
      if(killed[i]) continue;
      const int h = plaHeads[i];
      if(vitalCount[h] >= 2) continue;
      killed[i] = true;
      any = true;
      int cur = h;
      do {
        for(int d = 0; d < 4; d++) {
          const int a = cur + ADJ[d];
          const int r = regionOf[a];
          if(r >= 0 && !bordersDeadByHead[regionHead[r]] && (b.color[a] == EMPTY || b.color[a] == opp)) {
            bordersDeadByHead[regionHead[r]] = true;
            for(int k = 0; k < vitalLen[r]; k++) vitalCount[vital[vitalStart[r] + k]]--;
          }
        }
        cur = b.next[cur];
      } while(cur != h);
    }
    if(!any) break;
  }

  for(int i = 0; i < numPlaHeads; i++) {
    if(killed[i]) continue;
    const int h = plaHeads[i];
    int cur = h;
    do {
      result[cur] = pla;
      cur = b.next[cur];
    } while(cur != h);
  }
  for(int r = 0; r < numRegions; r++) {
    const int h = regionHead[r];
    bool mark = internal[r] <= 1 && !bordersDeadByHead[h] && anyPla;
    mark = mark || (safeBig && !containsOpp[r] && !bordersDeadByHead[h] && anyPla);
    if(mark) {
      int cur = h;
      do {
        result[cur] = pla;
        cur = nextInRegion[cur];
      } while(cur != h);
    }
    else if(unsafeBig && !containsOpp[r] && anyPla) {
      int cur = h;
      do {
        if(result[cur] == EMPTY) result[cur] = pla;
        cur = nextInRegion[cur];
      } while(cur != h);
    }
  }
}

// Board::calculateArea (board.cpp:1792-1813).
void calculateArea(const GoBoard& b, int8_t* result, bool nonPassAliveStones, bool safeBig, bool unsafeBig, bool msl) {
  std::fill(result, result + MAX_AREA, EMPTY);
  areaForPla(b, BLACK, safeBig, unsafeBig, msl, result);
  areaForPla(b, WHITE, safeBig, unsafeBig, msl, result);
  if(nonPassAliveStones)
    for(int y = 0; y < b.ys; y++)
      for(int x = 0; x < b.xs; x++) {
        const int p = b.at(x, y);
        if(result[p] == EMPTY) result[p] = b.color[p];
      }
}

// Board::calculateIndependentLifeArea and its helper (board.cpp:1815-1869,2169-2250).
void calculateIndependentLifeArea(const GoBoard& b, int8_t* result, int& whiteMinusBlack, bool keepTerritories, bool keepStones,
                                  bool msl) {
  int8_t basic[MAX_AREA];
  std::fill(result, result + MAX_AREA, EMPTY);
  std::fill(basic, basic + MAX_AREA, EMPTY);
  areaForPla(b, BLACK, true, true, msl, basic);
  areaForPla(b, WHITE, true, true, msl, basic);
  for(int y = 0; y < b.ys; y++)
    for(int x = 0; x < b.xs; x++) {
      const int p = b.at(x, y);
      if(basic[p] == EMPTY) basic[p] = b.color[p];
    }

  whiteMinusBlack = 0;
  bool seki[MAX_AREA];
  std::fill(seki, seki + MAX_AREA, false);
  int queue[MAX_AREA];
  for(int y = 0; y < b.ys; y++)
    for(int x = 0; x < b.xs; x++) {
      const int p = b.at(x, y);
      if(basic[p] == EMPTY || seki[p]) continue;
      bool touchesDame = false;
      for(int d = 0; d < 4; d++) {
        const int a = p + ADJ[d];
        touchesDame = touchesDame || (b.color[a] == EMPTY && basic[a] == EMPTY);
      }
      if(!((b.color[p] == basic[p] && b.numLibs(p) == 1) || touchesDame)) continue;
      const int8_t pla = basic[p];
      int qh = 0, qt = 0;
      seki[p] = true;
      queue[qt++] = p;
      while(qh != qt) {
        const int q = queue[qh++];
        for(int d = 0; d < 4; d++) {
          const int a = q + ADJ[d];
          if(basic[a] == pla && !seki[a]) {
            seki[a] = true;
            queue[qt++] = a;
          }
        }
      }
    }
  for(int y = 0; y < b.ys; y++)
    for(int x = 0; x < b.xs; x++) {
      const int p = b.at(x, y);
      if(basic[p] == EMPTY || seki[p] || result[p] == basic[p]) continue;
      const int8_t pla = basic[p];
      whiteMinusBlack += pla == WHITE ? 1 : -1;
      result[p] = basic[p];
      int qh = 0, qt = 0;
      queue[qt++] = p;
      while(qh != qt) {
        const int q = queue[qh++];
        for(int d = 0; d < 4; d++) {
          const int a = q + ADJ[d];
          if(basic[a] == pla && result[a] != basic[a]) {
            result[a] = basic[a];
            queue[qt++] = a;
          }
        }
      }
    }

  if(keepTerritories)
    for(int y = 0; y < b.ys; y++)
      for(int x = 0; x < b.xs; x++) {
        const int p = b.at(x, y);
        if(basic[p] != EMPTY && basic[p] != b.color[p]) result[p] = basic[p];
      }
  if(keepStones)
    for(int y = 0; y < b.ys; y++)
      for(int x = 0; x < b.xs; x++) {
        const int p = b.at(x, y);
        if(basic[p] != EMPTY && basic[p] == b.color[p]) result[p] = basic[p];
      }
}

// ---------------------------------------------------------------------------
// Feature assembly (nninputs.cpp:2273-2720).

constexpr int KO_SIMPLE = 0, KO_POSITIONAL = 1, KO_SITUATIONAL = 2, KO_SPIGHT = 3;
constexpr int SCORING_AREA = 0, SCORING_TERRITORY = 1;
constexpr int TAX_NONE = 0, TAX_SEKI = 1, TAX_ALL = 2;
constexpr float KOMI_CLIP_RADIUS = 20.0f;  // nninputs.h:21

void featurizeOne(const kgn_position& pos, int nnX, int nnY, bool nhwc, float* rowBin, float* rowGlobal, Scratch& s) {
  const int xs = pos.x_size, ys = pos.y_size;
  if(xs < 1 || ys < 1 || xs > MAX_SIDE || ys > MAX_SIDE || xs > nnX || ys > nnY)
    throw std::runtime_error("featurize: board size outside 1..19 or larger than the tensor");
  if(pos.next_player != BLACK && pos.next_player != WHITE) throw std::runtime_error("featurize: next_player must be 1 or 2");
  if(pos.colors[0] == nullptr) throw std::runtime_error("featurize: no current board");
  if(pos.num_moves < 0 || pos.num_moves > 5) throw std::runtime_error("featurize: num_moves outside 0..5");
  // Every board supplied must have its ko point on it (or -1), whether or
  // not the history below reaches that board.
  for(int k = 0; k < 3; k++)
    if((k == 0 || pos.colors[k] != nullptr) && (pos.ko_point[k] < -1 || pos.ko_point[k] >= xs * ys))
      throw std::runtime_error("featurize: ko_point off the board");
  const int C = KGN_FEATURES_SPATIAL_V7;
  std::fill(rowBin, rowBin + (size_t)C * nnX * nnY, 0.0f);
  std::fill(rowGlobal, rowGlobal + KGN_FEATURES_GLOBAL_V7, 0.0f);
  const int posStride = nhwc ? C : 1;
  const int featStride = nhwc ? 1 : nnX * nnY;
  auto set = [&](int x, int y, int f) { rowBin[(y * nnX + x) * posStride + f * featStride] = 1.0f; };
  auto setPoint = [&](int point, int f) { set(point % xs, point / xs, f); };

  const int8_t pla = (int8_t)pos.next_player;
  const int8_t opp = opponent(pla);
  GoBoard board;
  board.init(xs, ys, pos.colors[0], pos.ko_point[0], pos.chain_head[0], pos.chain_next[0], s);

  for(int y = 0; y < ys; y++)
    for(int x = 0; x < xs; x++) {
      const int p = board.at(x, y);
      set(x, y, 0);
      const int8_t c = board.color[p];
      if(c == pla) set(x, y, 1);
      else if(c == opp) set(x, y, 2);
      if(c == pla || c == opp) {
        const int libs = board.numLibs(p);
        if(libs == 1) set(x, y, 3);
        else if(libs == 2) set(x, y, 4);
        else if(libs == 3) set(x, y, 5);
      }
    }

  const int area0 = xs * ys;
  auto flag = [&](const uint8_t* a, int i) { return a != nullptr && a[i] != 0; };
  if(pos.encore_phase == 0) {
    if(board.ko != NONE) setPoint(pos.ko_point[0], 6);
    for(int i = 0; i < area0; i++)
      if(flag(pos.super_ko_banned, i) && i != pos.ko_point[0]) setPoint(i, 6);
  }
  else {
    for(int i = 0; i < area0; i++) {
      if(flag(pos.super_ko_banned, i)) setPoint(i, 6);
      if(flag(pos.ko_recap_blocked, i)) setPoint(i, 7);
    }
  }
  auto secondEncoreColor = [&](int i) -> int8_t {
    return pos.second_encore_start_colors == nullptr ? EMPTY : pos.second_encore_start_colors[i];
  };

  // Features 18, 19: area.
  int8_t area[MAX_AREA];
  bool hasArea = false;
  int taxAdjustForPla = 0;
  const bool msl = pos.multi_stone_suicide_legal != 0;
  if(pos.scoring_rule == SCORING_AREA && pos.tax_rule == TAX_NONE) {
    hasArea = true;
    calculateArea(board, area, true, true, true, msl);
  }
  else {
    bool keepTerritories = false, keepStones = false;
    if(pos.scoring_rule == SCORING_AREA && (pos.tax_rule == TAX_SEKI || pos.tax_rule == TAX_ALL)) {
      hasArea = true;
      keepStones = true;
    }
    else if(pos.scoring_rule == SCORING_TERRITORY && pos.tax_rule == TAX_NONE) {
      if(pos.encore_phase >= 2) {
        hasArea = true;
        keepTerritories = true;
      }
    }
    else if(pos.scoring_rule == SCORING_TERRITORY && (pos.tax_rule == TAX_SEKI || pos.tax_rule == TAX_ALL)) {
      hasArea = pos.encore_phase >= 2;
    }
    else {
      throw std::runtime_error("featurize: scoring or tax rule outside the rules' values");
    }
    if(hasArea) {
      int whiteMinusBlack = 0;
      calculateIndependentLifeArea(board, area, whiteMinusBlack, keepTerritories, keepStones, msl);
      if(pos.tax_rule == TAX_ALL) taxAdjustForPla = pla == WHITE ? -2 * whiteMinusBlack : 2 * whiteMinusBlack;
    }
  }
  bool finalPhaseNotWin = false;
  if(hasArea) {
    int scoreForPla = taxAdjustForPla;
    for(int y = 0; y < ys; y++)
      for(int x = 0; x < xs; x++) {
        const int p = board.at(x, y);
        if(area[p] == pla) {
          set(x, y, 18);
          scoreForPla++;
        }
        else if(area[p] == opp) {
          set(x, y, 19);
          scoreForPla--;
        }
        else if(pos.scoring_rule == SCORING_TERRITORY) {
          const int8_t start = secondEncoreColor(y * xs + x);
          if(board.color[p] == pla && start == pla) {
            set(x, y, 18);
            scoreForPla++;
          }
          else if(board.color[p] == opp && start == opp) {
            set(x, y, 19);
            scoreForPla--;
          }
        }
      }
    const float finalScorePla = (float)scoreForPla + pos.self_komi;
    if(finalScorePla <= 0.0) finalPhaseNotWin = true;
  }

  // Features 9-13 and globals 0-4: the last five moves.
  int maxTurns = 5;
  bool suppressPassWouldEndPhase = false;
  if(pos.pass_would_end_game && (pos.conservative_pass_and_is_root || pos.suppress_end_game_from_friendly_pass ||
                                 (pos.enable_passing_hacks && finalPhaseNotWin))) {
    maxTurns = 0;
    suppressPassWouldEndPhase = true;
  }
  else if(pos.is_game_finished || pos.is_past_normal_phase_end) {
    maxTurns = 1;
  }
  maxTurns = std::min(maxTurns, pos.max_history);
  int included = 0;
  if(maxTurns > 0) {
    const int use = std::min(maxTurns, pos.num_approx_valid_turns_this_phase);
    const int n = pos.num_moves;
    const int8_t expect[5] = {opp, pla, opp, pla, opp};
    for(int k = 0; k < 5 && k < use && k < n; k++) {
      const int i = n - 1 - k;
      if(pos.move_player[i] != expect[k]) break;
      included = k + 1;
      const int pt = pos.move_point[i];
      if(pt == KGN_MOVE_PASS) rowGlobal[k] = 1.0f;
      else if(pt != KGN_MOVE_NULL) {
        if(pt < 0 || pt >= area0) throw std::runtime_error("featurize: move point off the board");
        setPoint(pt, 9 + k);
      }
    }
  }

  // Features 14-17: ladders on this board and the two before it. A board
  // one or two moves back that is absent (a null colour array), or that the
  // history does not reach, is the board after it, whose stones are reused.
  auto setGrid = [&](int p, int f) { set(p % STRIDE - 1, p / STRIDE - 1, f); };
  const std::vector<LadderHit>* hits = &boardLadders(pos, 0, &board, s);
  for(const LadderHit& h : *hits) {
    setGrid(h.point, 14);
    if(board.color[h.point] == opp)
      for(int k = 0; k < h.numWorking; k++) setGrid(h.working[k], 17);
  }
  if(included >= 1 && pos.colors[1] != nullptr) hits = &boardLadders(pos, 1, nullptr, s);
  for(const LadderHit& h : *hits) setGrid(h.point, 15);
  if(included >= 2 && pos.colors[2] != nullptr) hits = &boardLadders(pos, 2, nullptr, s);
  for(const LadderHit& h : *hits) setGrid(h.point, 16);

  // Features 20, 21: stones at the start of the second encore.
  if(pos.encore_phase >= 2)
    for(int i = 0; i < area0; i++) {
      const int8_t c = secondEncoreColor(i);
      if(c == pla) setPoint(i, 20);
      else if(c == opp) setPoint(i, 21);
    }

  // Globals.
  float selfKomi = pos.self_komi;
  const float bArea = (float)(xs * ys);
  if(selfKomi > bArea + KOMI_CLIP_RADIUS) selfKomi = bArea + KOMI_CLIP_RADIUS;
  if(selfKomi < -bArea - KOMI_CLIP_RADIUS) selfKomi = -bArea - KOMI_CLIP_RADIUS;
  rowGlobal[5] = selfKomi / 20.0f;
  if(pos.ko_rule == KO_SIMPLE) {
  }
  else if(pos.ko_rule == KO_POSITIONAL || pos.ko_rule == KO_SPIGHT) {
    rowGlobal[6] = 1.0f;
    rowGlobal[7] = 0.5f;
  }
  else if(pos.ko_rule == KO_SITUATIONAL) {
    rowGlobal[6] = 1.0f;
    rowGlobal[7] = -0.5f;
  }
  else {
    throw std::runtime_error("featurize: ko rule outside the rules' values");
  }
  if(msl) rowGlobal[8] = 1.0f;
  if(pos.scoring_rule == SCORING_TERRITORY) rowGlobal[9] = 1.0f;
  if(pos.tax_rule == TAX_SEKI) rowGlobal[10] = 1.0f;
  else if(pos.tax_rule == TAX_ALL) {
    rowGlobal[10] = 1.0f;
    rowGlobal[11] = 1.0f;
  }
  if(pos.encore_phase > 0) rowGlobal[12] = 1.0f;
  if(pos.encore_phase > 1) rowGlobal[13] = 1.0f;
  const bool passEndsPhase = suppressPassWouldEndPhase ? false : pos.pass_would_end_phase != 0;
  rowGlobal[14] = passEndsPhase ? 1.0f : 0.0f;
  if(pos.playout_doubling_advantage != 0) {
    rowGlobal[15] = 1.0f;
    rowGlobal[16] = (float)(0.5 * pos.playout_doubling_advantage);
  }
  if(pos.has_button) rowGlobal[17] = 1.0f;
  if(pos.scoring_rule == SCORING_AREA || pos.encore_phase >= 2) {
    // Triangle wave of the komi against the nearest komi that allows a draw
    // (nninputs.cpp:2660-2718).
    const bool evenArea = (xs * ys) % 2 == 0;
    float komiFloor;
    if(evenArea) komiFloor = std::floor(selfKomi / 2.0f) * 2.0f;
    else komiFloor = std::floor((selfKomi - 1.0f) / 2.0f) * 2.0f + 1.0f;
    float delta = selfKomi - komiFloor;
    if(delta < 0.0f) delta = 0.0f;
    if(delta > 2.0f) delta = 2.0f;
    float wave;
    if(delta < 0.5f) wave = delta;
    else if(delta < 1.5f) wave = 1.0f - delta;
    else wave = delta - 2.0f;
    rowGlobal[18] = wave;
  }
}

void setErr(char* err, int32_t errlen, const std::string& msg) {
  if(err == nullptr || errlen <= 0) return;
  const size_t n = std::min(msg.size(), (size_t)errlen - 1);
  memcpy(err, msg.data(), n);
  err[n] = 0;
}

}  // namespace

extern "C" int32_t kgn_featurize_set_cache(int32_t entries) {
  if(entries < 0 || entries > KGN_FEATURIZE_MAX_CACHE) return -1;
  return g_ladderCacheEntries.exchange(entries);
}

extern "C" int32_t kgn_featurize(const kgn_position* positions, int32_t n, int32_t nn_x, int32_t nn_y, int32_t use_nhwc,
                                 float* spatial, float* global_out, int32_t num_threads, char* err, int32_t errlen) {
  if(n < 0 || (n > 0 && (positions == nullptr || spatial == nullptr || global_out == nullptr)) || nn_x < 1 || nn_y < 1 ||
     nn_x > MAX_SIDE || nn_y > MAX_SIDE) {
    setErr(err, errlen, "kgn_featurize: invalid arguments");
    return -1;
  }
  const size_t rowElts = (size_t)KGN_FEATURES_SPATIAL_V7 * nn_x * nn_y;
  int threads = num_threads > 0 ? num_threads : (int)std::max(1u, std::thread::hardware_concurrency());
  // Each worker takes runs of consecutive positions, whose boards often
  // recur one or two moves later (the ladder cache's hits).
  constexpr int RUN = 8;
  threads = std::max(1, std::min(threads, (n + RUN - 1) / RUN));
  std::atomic<int> nextRow(0);
  std::atomic<int> failedRow(-1);
  std::string failure;
  auto work = [&]() {
    static thread_local Scratch s;
    while(true) {
      const int first = nextRow.fetch_add(RUN);
      if(first >= n || failedRow.load() >= 0) return;
      for(int i = first; i < std::min(n, first + RUN); i++) {
        try {
          featurizeOne(positions[i], nn_x, nn_y, use_nhwc != 0, spatial + rowElts * i,
                       global_out + (size_t)KGN_FEATURES_GLOBAL_V7 * i, s);
        }
        catch(const std::exception& e) {
          int expected = -1;
          if(failedRow.compare_exchange_strong(expected, i)) failure = e.what();
          return;
        }
      }
    }
  };
  if(threads == 1) {
    work();
  }
  else {
    std::vector<std::thread> pool;
    for(int t = 0; t < threads; t++) pool.emplace_back(work);
    for(auto& t : pool) t.join();
  }
  if(failedRow.load() >= 0) {
    setErr(err, errlen, "kgn_featurize: position " + std::to_string(failedRow.load()) + ": " + failure);
    return -1;
  }
  return 0;
}
