// The run plan and cursor protocol of the streaming engine's independent-stage kernel
// (stream.hip), in one header that the kernel and a host simulator both compile.
//
// The program's tiles form one list [0, total).  It is cut into runs of consecutive
// tiles.  Runs [0, static_runs) are R tiles long and dealt: wavefront v of the V in the
// grid runs v, v + V, ...  The tiles after them are claimed.  They are divided between
// `shards` counters: shard s owns the tiles [t0, t1) and the runs [lo, lo + count), first
// `nlong` runs of dyn_run tiles, then runs of tail_run tiles, the last ending at t1.  The
// short runs at the end of every shard let the wavefronts finish close together: a
// wavefront that claims the last long run of a shard still has many short ones to share
// with the rest.  A wavefront claims when its load cursor steps past the end of a run with
// no dealt run left; a claim past its shard's runs returns `runs` (past the end), after
// which that wavefront claims nothing more.  So each wavefront of a shard makes exactly
// one failed claim, the shard's last claim is number (its runs + its wavefronts - 1), and
// the wavefront that receives it returns the counter to zero for the next launch.  That
// every shard's last run ends at its last tile matters: the load cursor reaches the run's
// end right after issuing its last real tile, so the failed claim is made before the
// compute cursor can leave the loop.
//
// Each wavefront keeps two cursors kDepth tiles apart: the load cursor claims runs, the
// compute cursor takes them from a two-entry queue in claim order.  A wavefront only ever
// holds runs of its own shard, so run geometry is computed from that shard's description.

#pragma once

#include <stdint.h>

#if defined(__HIP__)
#define IMQ_HD __host__ __device__ __forceinline__
#else
#define IMQ_HD inline
#endif

namespace imq_runs {

constexpr int kMaxShards = 16;

// One shard's claimed runs.
struct ShardRuns {
  int32_t lo;     // its first run index
  int32_t count;  // its runs
  int32_t t0;     // its first tile
  int32_t t1;     // one past its last tile
  int32_t nlong;  // its runs of dyn_run tiles (the rest are tail_run tiles, the last shorter)
};

struct RunPlan {
  int32_t total;        // tiles of the program
  int32_t run;          // tiles per dealt run
  int32_t static_runs;  // dealt runs
  int32_t runs;         // all runs; a run index >= runs starts past the last tile
  int32_t dyn_run;      // tiles per long claimed run
  int32_t tail_run;     // tiles per short claimed run
  int32_t waves;        // wavefronts in the grid
  int32_t pad;

  // Run r of a wavefront whose shard is `s` (a claimed r is always of that shard).
  IMQ_HD int start_of(int r, const ShardRuns& s) const {
    if (r < static_runs) return r * run;
    if (r >= runs) return total;
    const int j = r - s.lo;
    return j < s.nlong ? s.t0 + j * dyn_run : s.t0 + s.nlong * dyn_run + (j - s.nlong) * tail_run;
  }
  IMQ_HD int length_of(int r, const ShardRuns& s) const {
    if (r < static_runs) return run;
    if (r >= runs) return dyn_run;
    const int left = s.t1 - start_of(r, s);
    const int len = r - s.lo < s.nlong ? dyn_run : tail_run;
    return left < len ? left : len;
  }
};

// A position in a wavefront's sequence of tiles: run r (global), tile t of the run.
struct Pos {
  int r, t;
};

template <class Plan>
IMQ_HD int tile_of(const Plan& p, const ShardRuns& s, const Pos& q) {
  return p.start_of(q.r, s) + q.t;
}

// Runs the load cursor has claimed that the compute cursor has not reached yet.
struct ClaimQueue {
  int qa = 0, qb = 0, qn = 0;
};

// One claim's outcome: the counter's previous value `old` names run lo + old of the
// shard's `count`, or the end.
IMQ_HD int claimed_run(uint32_t old, const ShardRuns& s, int end) {
  return (int)old < s.count ? s.lo + (int)old : end;
}

// The claim number that returns a shard's counter to zero: every wavefront of the shard
// makes one failed claim.
IMQ_HD uint32_t last_claim_of(int count, int waves) { return (uint32_t)(count + waves - 1); }

// Moves the load cursor one tile on; at the end of a run it takes the next dealt run or,
// with none left, claims (claim() returns a run index, or p.runs past the end).
template <class Plan, class Claim>
IMQ_HD void step_load(const Plan& p, const ShardRuns& s, Pos& q, ClaimQueue& cq, Claim&& claim) {
  if (++q.t < p.length_of(q.r, s)) return;
  q.t = 0;
  if (q.r + p.waves < p.static_runs || p.static_runs == p.runs) {
    q.r += p.waves;  // the next dealt run (or, with nothing to claim, past the end)
  } else if (q.r < p.runs) {
    q.r = claim();
    if (cq.qn == 0)
      cq.qa = q.r;
    else
      cq.qb = q.r;
    ++cq.qn;
  }
}

// Moves the compute cursor one tile on, into the run the load cursor claimed first.
template <class Plan>
IMQ_HD void step_compute(const Plan& p, const ShardRuns& s, Pos& q, ClaimQueue& cq) {
  if (++q.t < p.length_of(q.r, s)) return;
  q.t = 0;
  if (q.r + p.waves < p.static_runs || p.static_runs == p.runs) {
    q.r += p.waves;
  } else if (q.r < p.runs) {
    q.r = cq.qa;
    cq.qa = cq.qb;
    --cq.qn;
  }
}

// The host's plan for `total` tiles over `grid` workgroups of `waves_per_group`
// wavefronts: dealt runs of `run_target` tiles or a little more in whole rounds of one
// run per wavefront; the last `dyn_percent` of the rounds (at least one, when there are
// two or more) claimed from up to kMaxShards counters, each shard's tiles in runs of
// `dyn_run`, of which the last `tail_percent` (rounded to whole tail runs) in runs of
// `tail_run`.  Workgroup b claims from shard (b / `spread`) % shards, `spread` being the
// number of consecutive workgroups that share an XCD assignment pattern, so that every
// shard is served by workgroups of all eight XCDs.
struct ShardPlan {
  RunPlan plan;
  int32_t shards, spread;
  ShardRuns shard[kMaxShards];
  int32_t shard_waves[kMaxShards];
};

IMQ_HD int shard_of_group(int block, int shards, int spread) { return (block / spread) % shards; }

inline ShardPlan plan_runs(int total, int grid, int waves_per_group, int run_target, int dyn_run,
                           int dyn_percent, int tail_run, int tail_percent, int spread) {
  ShardPlan s;
  const int V = grid * waves_per_group;
  int rounds = total / (V * run_target);
  if (rounds < 1) rounds = 1;
  const int R = (total + V * rounds - 1) / (V * rounds);
  int dealt = rounds;
  if (rounds >= 2 && dyn_percent > 0) {
    int claimed = (rounds * dyn_percent + 50) / 100;
    if (claimed < 1) claimed = 1;
    if (claimed > rounds - 1) claimed = rounds - 1;
    dealt = rounds - claimed;
  }
  int static_runs = (total + R - 1) / R;
  const bool claiming = dealt < rounds && (int64_t)V * dealt * R < total;
  if (claiming) static_runs = V * dealt;
  int shards = grid / spread;
  if (shards > kMaxShards) shards = kMaxShards;
  if (shards < 1) shards = 1;
  s.shards = shards;
  s.spread = spread;
  int nruns = static_runs;
  const int first = claiming ? static_runs * R : total;
  const int64_t claimed_tiles = total - first;
  for (int k = 0; k < kMaxShards; ++k) {
    ShardRuns& sh = s.shard[k];
    sh = ShardRuns{nruns, 0, total, total, 0};
    if (!claiming || k >= shards) continue;
    sh.t0 = first + (int)(claimed_tiles * k / shards);
    sh.t1 = first + (int)(claimed_tiles * (k + 1) / shards);
    const int n = sh.t1 - sh.t0;
    const int tail = (int)(((int64_t)n * tail_percent + 99) / 100);
    sh.nlong = (n - tail) / dyn_run;
    const int rest = n - sh.nlong * dyn_run;
    sh.count = sh.nlong + (rest + tail_run - 1) / tail_run;
    nruns += sh.count;
  }
  s.plan.total = total;
  s.plan.run = R;
  s.plan.static_runs = static_runs;
  s.plan.runs = nruns;
  s.plan.dyn_run = dyn_run;
  s.plan.tail_run = tail_run;
  s.plan.waves = V;
  s.plan.pad = 0;
  for (int k = 0; k < kMaxShards; ++k) s.shard_waves[k] = 0;
  for (int b = 0; b < grid; ++b) s.shard_waves[shard_of_group(b, shards, spread)] += waves_per_group;
  return s;
}

}  // namespace imq_runs
