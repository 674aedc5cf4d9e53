// Host-side check of the halo conv's load / barrier schedule
// (draw-instant_amd/csrc/k_conv3_sched.h, used by k_conv3.hip): replays a
// wave's issue sequence for every tile width and chunk count with loads
// retiring in order, where a wait leaves at most allow(j) loads
// outstanding, and checks that
//   - every stage's weights and its chunk's patch pieces are complete at
//     the last barrier before the iteration that reads the stage's
//     fragments;
//   - every weight / patch buffer is refilled only after a barrier that
//     follows the last read of its previous contents (barriers wait for the
//     wave's LDS reads);
//   - no wait count exceeds the 6-bit vmcnt field.
// The prologue's wait leaves prologue_allow weight stages in flight, as in
// the kernel.
// It also runs the same replay with a uniform allowance (the last five
// iterations' loads outstanding at every barrier), which leaves a chunk's
// last patch pieces in flight when the next chunk starts, and requires that
// the replay reports it.  Exit status 0 when all hold.
#include <cstdio>
#include <map>
#include <vector>

#include "k_conv3_sched.h"

using namespace di::conv3;

struct Sim {
  struct Load {
    int kind, id, piece;
  };
  std::vector<Load> loads;
  size_t done = 0;
  std::vector<int> barriers;
  std::map<int, size_t> wload;                   // stage -> load index
  std::map<std::pair<int, int>, size_t> pload;   // (chunk, piece) -> load index
  std::map<int, int> wcontent, wlast;            // buffer -> stage, last read iteration
  std::map<int, int> pcontent, plast;            // patch buffer -> chunk, last read iteration
  int errors = 0;
  const char* tag;
  bool quiet;

  bool barrier_in(int lo, int hi) const {
    for (int b : barriers)
      if (b >= lo && b <= hi) return true;
    return false;
  }
  void fail(const char* what, int a, int b, int it) {
    if (!quiet && errors < 5) printf("  %s: %s %d/%d at iteration %d\n", tag, what, a, b, it);
    errors++;
  }
  void refill(std::map<int, int>& content, std::map<int, int>& last, int buf, int id, int it,
              const char* what) {
    auto c = content.find(buf);
    if (c != content.end() && c->second != id) {
      auto l = last.find(buf);
      if (l != last.end() && !barrier_in(l->second, it - 1)) fail(what, buf, l->second, it);
    }
    if (c == content.end() || c->second != id) last.erase(buf);
    content[buf] = id;
  }
  void weight(int nbb, int stage, int it) {
    refill(wcontent, wlast, stage % nbb, stage, it, "weight buffer refilled before a barrier (buf/last read)");
    wload[stage] = loads.size();
    loads.push_back({0, stage, 0});
  }
  void patch(int chunk, int piece, int it) {
    refill(pcontent, plast, chunk & 1, chunk, it, "patch buffer refilled before a barrier (buf/last read)");
    pload[{chunk, piece}] = loads.size();
    loads.push_back({1, chunk, piece});
  }
  void wait(int allow, int it) {
    if (allow > 63) fail("wait count above 63", allow, 0, it);
    if (loads.size() > (size_t)allow && loads.size() - allow > done) done = loads.size() - allow;
  }
  void read(int nbb, int np, int stage, int it) {
    auto w = wload.find(stage);
    if (w == wload.end() || w->second >= done) fail("weights not complete for stage", stage, 0, it);
    const int chunk = stage / 9;
    for (int p = 0; p < np; p++) {
      auto q = pload.find({chunk, p});
      if (q == pload.end() || q->second >= done) fail("patch piece not complete (chunk/piece)", chunk, p, it);
    }
    wlast[stage % nbb] = it;
    plast[chunk & 1] = it;
  }
};

template <int W>
int replay(int nch, bool naive, bool quiet) {
  using G = ConvGeo<W>;
  char tag[64];
  snprintf(tag, sizeof tag, "W=%d chunks=%d%s", W, nch, naive ? " (uniform allowance)" : "");
  Sim s;
  s.tag = tag;
  s.quiet = quiet;
  auto allow = [&](int j) {
    if (!naive) return G::allow(j);
    int n = 0;
    for (int i = j - 4; i <= j; i++) n += G::issued(i);
    return n;
  };
  const int n_stages = nch * 9;
  // prologue: the first chunk's patch, weights of stages 0..NBB-2, wait all
  for (int i = 0; i < G::NP; i++) s.patch(0, i, -1);
  for (int b = 0; b + 1 < G::NBB; b++) s.weight(G::NBB, b, -1);
  s.wait(G::prologue_allow, -1);
  s.barriers.push_back(-1);
  s.read(G::NBB, G::NP, 0, -1);
  s.barriers.push_back(-1);
  int s0 = 0;
  for (; s0 + 18 <= n_stages; s0 += 18) {
    for (int j = 0; j < 18; j++) {
      const int it = s0 + j, tap = j % 9, c = s0 / 9 + j / 9;
      if (it + 1 < n_stages) s.read(G::NBB, G::NP, it + 1, it);
      s.weight(G::NBB, s0 + j + G::NBB - 1, it);
      for (int q = 0; q < G::pieces(tap); q++) s.patch(c + 1, tap * G::PPT + q, it);
      if (j % G::BAR == G::BAR - 1) {
        s.wait(allow(j), it);
        s.barriers.push_back(it);
      }
    }
  }
  if (s0 < n_stages) {
    for (int j = 0; j < 9; j++) {
      const int it = s0 + j;
      if (j + 1 < 9) s.read(G::NBB, G::NP, it + 1, it);
      if (j + G::NBB - 1 < 9) s.weight(G::NBB, s0 + j + G::NBB - 1, it);
      if (j % G::BAR == G::BAR - 1) {
        s.wait(G::tail_allow(j), it);
        s.barriers.push_back(it);
      }
    }
  }
  return s.errors;
}

template <int W>
int check_width() {
  int errors = 0;
  for (int nch = 1; nch <= 48; nch++) errors += replay<W>(nch, false, false);
  printf("W=%3d: NBB=%d BAR=%d NP=%d: %s\n", W, ConvGeo<W>::NBB, ConvGeo<W>::BAR, ConvGeo<W>::NP,
         errors ? "ERRORS" : "schedule ok for 1..48 chunks");
  return errors;
}

int main() {
  int errors = check_width<16>() + check_width<32>() + check_width<64>() + check_width<128>();
  // the replay must catch a schedule whose barriers leave too much in flight
  const int naive = replay<16>(4, true, true) + replay<64>(5, true, true);
  printf("uniform-allowance schedule: %d violations found (must be > 0)\n", naive);
  if (naive == 0) errors++;
  printf(errors ? "FAIL\n" : "OK\n");
  return errors ? 1 : 0;
}
