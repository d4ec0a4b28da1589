// Host simulation of the streaming engine's run plan and claim protocol
// (ironmule_amd/csrc/stream_runs.h, the same header the kernel compiles).
//
// Each simulated wavefront executes the kernel's sequence of events: one issue; unless
// that first tile lies past the last one, its compute and two issues; then passes of
// (compute, issue) x kDepth until a pass starts past the last tile.  A random
// scheduler interleaves the wavefronts one event at a time, sometimes letting one run a
// long burst, so that claims arrive in many orders.  The claim counters persist across
// launches, as the device's do.  After every launch it checks that every tile was
// computed exactly once, by the wavefront that loaded it, that no loaded real tile was
// left uncomputed, that no claim queue held more than two runs, and that every shard's
// counter is back at zero.
//
// Usage: stream_runs_sim [--old-length] SEED CASES LAUNCHES
//   --old-length: claimed runs all dyn_run long (the last one included), which leaves a
//   counter behind when the last run is short; the test expects a failure then.
// Prints "ok <cases>" or the first failing case and exits 1.

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <deque>
#include <vector>

#include "../ironmule_amd/csrc/stream_runs.h"

using namespace imq_runs;

namespace {

constexpr int kDepth = 2;    // tiles in flight per wavefront (stream.hip)
constexpr int kRunTarget = 16;
constexpr int kSpread = 8;

struct Rng {
  uint64_t s;
  uint64_t next() {
    s ^= s << 13;
    s ^= s >> 7;
    s ^= s << 17;
    return s;
  }
  int below(int n) { return (int)(next() % (uint64_t)n); }
};

// Run lengths that ignore where a shard's tiles end: every claimed run as long as its kind
// (the rule that left counters behind when a last run was short).
struct OldPlan : RunPlan {
  int length_of(int r, const ShardRuns& s) const {
    return r < static_runs ? run : (r - s.lo < s.nlong ? dyn_run : tail_run);
  }
};

struct Params {
  int total, grid, waves_per_group, dyn_run, pct, tail_run, tail_pct;
};

enum State { kInit, kFirst, kFirstIssue, kPassStart, kCompute, kIssue, kDone };

struct Wave {
  Pos lpos, cpos;
  ClaimQueue cq;
  State state = kInit;
  int inits = 0, d = 0, g0 = 0;
  int shard = 0;
  std::deque<int> loaded;  // tiles issued and not yet computed (-1: past the end)
};

template <class Plan>
bool launch(const ShardPlan& sp, const Plan& P, const Params& pr, std::vector<uint32_t>& ctr, Rng& rng,
            char* why, size_t why_len) {
  const int V = pr.grid * pr.waves_per_group;
  std::vector<Wave> waves((size_t)V);
  for (int v = 0; v < V; ++v) {
    waves[(size_t)v].lpos = Pos{v, 0};
    waves[(size_t)v].cpos = Pos{v, 0};
    waves[(size_t)v].shard = shard_of_group(v / pr.waves_per_group, sp.shards, sp.spread);
  }
  std::vector<int> computed((size_t)P.total, 0);
  int max_queue = 0;
  // the compute of the tile at the front of the wavefront's loads (its compute cursor's)
  auto compute = [&](Wave& w) -> bool {
    const int gd = tile_of(P, sp.shard[w.shard], w.cpos);
    const int got = w.loaded.front();
    w.loaded.pop_front();
    if (gd < P.total) {
      if (got != gd) {
        snprintf(why, why_len, "wavefront computes tile %d from the loads of tile %d", gd, got);
        return false;
      }
      ++computed[(size_t)gd];
    } else if (got >= 0) {
      snprintf(why, why_len, "loaded tile %d is dropped", got);
      return false;
    }
    step_compute(P, sp.shard[w.shard], w.cpos, w.cq);
    return true;
  };
  auto issue = [&](Wave& w) {
    const ShardRuns& sh = sp.shard[w.shard];
    const int g = tile_of(P, sh, w.lpos);
    w.loaded.push_back(g < P.total ? g : -1);
    const uint32_t last = last_claim_of(sh.count, sp.shard_waves[w.shard]);
    auto claim = [&]() {
      const uint32_t old = ctr[(size_t)w.shard]++;
      if (old == last) ctr[(size_t)w.shard] = 0;
      return claimed_run(old, sh, P.runs);
    };
    step_load(P, sh, w.lpos, w.cq, claim);
    if (w.cq.qn > max_queue) max_queue = w.cq.qn;
  };
  std::vector<int> live;
  for (int v = 0; v < V; ++v) live.push_back(v);
  int burst = 0, burst_id = -1;
  while (!live.empty()) {
    int idx = -1;
    if (burst > 0 && waves[(size_t)burst_id].state != kDone) {
      for (int i = 0; i < (int)live.size(); ++i)
        if (live[(size_t)i] == burst_id) idx = i;
      --burst;
    }
    if (idx < 0) {
      idx = rng.below((int)live.size());
      burst = rng.below(16) == 0 ? rng.below(64) : 0;
      burst_id = live[(size_t)idx];
    }
    Wave& w = waves[(size_t)live[(size_t)idx]];
    switch (w.state) {
      case kInit:  // the first tile's loads, then x is staged
        issue(w);
        w.state = kFirst;
        break;
      case kFirst:  // the first tile, computed before the next two are issued
        if (tile_of(P, sp.shard[w.shard], w.cpos) >= P.total) {
          w.state = kDone;
          break;
        }
        if (!compute(w)) return false;
        w.inits = 0;
        w.state = kFirstIssue;
        break;
      case kFirstIssue:
        issue(w);
        if (++w.inits == kDepth) w.state = kPassStart;
        break;
      case kPassStart:
        w.g0 = tile_of(P, sp.shard[w.shard], w.cpos);
        if (w.g0 >= P.total) {
          w.state = kDone;
        } else {
          w.d = 0;
          w.state = kCompute;
        }
        break;
      case kCompute:
        if (!compute(w)) return false;
        w.state = kIssue;
        break;
      case kIssue:
        issue(w);
        w.state = ++w.d < kDepth ? kCompute : kPassStart;
        break;
      case kDone:
        break;
    }
    if (w.state == kDone) {
      for (int g : w.loaded)
        if (g >= 0) {
          snprintf(why, why_len, "loaded tile %d is never computed", g);
          return false;
        }
      live[(size_t)idx] = live.back();
      live.pop_back();
    }
  }
  for (int g = 0; g < P.total; ++g)
    if (computed[(size_t)g] != 1) {
      snprintf(why, why_len, "tile %d computed %d times", g, computed[(size_t)g]);
      return false;
    }
  if (max_queue > 2) {
    snprintf(why, why_len, "a claim queue held %d runs", max_queue);
    return false;
  }
  for (int s = 0; s < sp.shards; ++s)
    if (ctr[(size_t)s] != 0) {
      snprintf(why, why_len, "shard %d counter left at %u", s, ctr[(size_t)s]);
      return false;
    }
  return true;
}

template <class Plan>
bool run_case(const Params& pr, int launches, Rng& rng, char* why, size_t n) {
  const ShardPlan sp = plan_runs(pr.total, pr.grid, pr.waves_per_group, kRunTarget, pr.dyn_run, pr.pct,
                                 pr.tail_run, pr.tail_pct, kSpread);
  // the shards cover the claimed tiles, in order, and the runs are numbered in tile order
  int next_lo = sp.plan.static_runs;
  for (int s = 0; s < kMaxShards; ++s) {
    const ShardRuns& sh = sp.shard[s];
    if (sh.count == 0) continue;
    if (sh.lo != next_lo || sp.plan.start_of(sh.lo, sh) != sh.t0) {
      snprintf(why, n, "shard %d does not follow the previous one", s);
      return false;
    }
    next_lo += sh.count;
  }
  if (next_lo != sp.plan.runs) {
    snprintf(why, n, "the shards hold %d runs of %d", next_lo - sp.plan.static_runs, sp.plan.runs - sp.plan.static_runs);
    return false;
  }
  Plan P;
  static_cast<RunPlan&>(P) = sp.plan;
  std::vector<uint32_t> ctr((size_t)kMaxShards, 0);
  for (int l = 0; l < launches; ++l) {
    if (!launch(sp, P, pr, ctr, rng, why, n)) {
      char tail[128];
      snprintf(tail, sizeof(tail), " (launch %d)", l + 1);
      strncat(why, tail, n - strlen(why) - 1);
      return false;
    }
  }
  return true;
}

}  // namespace

int main(int argc, char** argv) {
  int a = 1;
  bool old = false;
  if (a < argc && strcmp(argv[a], "--old-length") == 0) {
    old = true;
    ++a;
  }
  if (argc - a != 3) {
    fprintf(stderr, "usage: %s [--old-length] SEED CASES LAUNCHES\n", argv[0]);
    return 2;
  }
  Rng rng{(uint64_t)strtoull(argv[a], nullptr, 10) * 2654435761ull + 1};
  const int cases = atoi(argv[a + 1]), launches = atoi(argv[a + 2]);
  // fixed cases first: one workgroup of 4 wavefronts over 1250 tiles (a 5000-row,
  // K = 2560 stage whose last claimed runs are short), the 20- and 36-layer programs of
  // the streaming engine's grid (256 workgroups of 12 wavefronts), then random cases
  struct Fixed {
    int total, grid, waves;
  } fixed[] = {{1250, 1, 4},       {20480, 1, 4}, {20480, 37, 4}, {1, 1, 4},  {7, 3, 4},
               {64, 1, 4},         {129, 2, 4},   {1000, 8, 4},   {204800, 256, 12},
               {368640, 256, 12},  {5000, 2, 12}};
  const int nfixed = (int)(sizeof(fixed) / sizeof(fixed[0]));
  char why[256];
  for (int c = 0; c < nfixed + cases; ++c) {
    Params pr;
    if (c < nfixed) {
      pr = Params{fixed[c].total, fixed[c].grid, fixed[c].waves, 8, 25, 1, 30};
    } else {
      pr.waves_per_group = rng.below(2) == 0 ? 4 : 12;
      pr.grid = 1 + rng.below(rng.below(4) == 0 ? 300 : 40);
      const int per = pr.waves_per_group * pr.grid * kRunTarget;
      pr.total = 1 + rng.below(per * (1 + rng.below(6)));
      pr.dyn_run = 3 + rng.below(8);  // stream.hip: > kDepth
      pr.pct = rng.below(3) == 0 ? 50 : 25;
      pr.tail_run = 1 + rng.below(3);
      const int tails[] = {0, 30, 100};
      pr.tail_pct = tails[rng.below(3)];
    }
    why[0] = 0;
    const bool good = old ? run_case<OldPlan>(pr, launches, rng, why, sizeof(why))
                          : run_case<RunPlan>(pr, launches, rng, why, sizeof(why));
    if (!good) {
      printf("FAIL total=%d grid=%d waves=%d dyn_run=%d pct=%d tail_run=%d tail_pct=%d: %s\n", pr.total,
             pr.grid, pr.waves_per_group, pr.dyn_run, pr.pct, pr.tail_run, pr.tail_pct, why);
      return 1;
    }
  }
  printf("ok %d\n", nfixed + cases);
  return 0;
}
