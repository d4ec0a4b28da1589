// The run plan and cursor protocol of the streaming engine's independent-stage kernel
// (stream.hip), in one header that the kernel and a host simulator both compile.
//
// The program's tiles form one list [0, total).  It is cut into runs of consecutive
// tiles.  Runs [0, static_runs) are R tiles long and dealt: wavefront v of the V in the
// grid runs v, v + V, ...  Runs [static_runs, runs) are dyn_run tiles long, except the
// last, which ends at `total`; they are claimed one at a time from `shards` counters
// (shard s owns runs [shard_lo[s], shard_lo[s + 1]) and serves shard_waves[s]
// wavefronts).  A wavefront claims when its load cursor steps past the end of a run
// with no dealt run left; a claim past its shard's runs returns `runs` (past the end),
// after which that wavefront claims nothing more.  So each wavefront of a shard makes
// exactly one failed claim, the shard's last claim is number (its runs + its wavefronts
// - 1), and the wavefront that receives it returns the counter to zero for the next
// launch.  That the last run ends at `total` matters: its load cursor reaches the run's
// end right after issuing its last real tile, so the failed claim is made before the
// compute cursor can leave the loop.
//
// Each wavefront keeps two cursors kDepth tiles apart: the load cursor claims runs, the
// compute cursor takes them from a two-entry queue in claim order.

#pragma once

#include <stdint.h>

#if defined(__HIP__)
#define IMQ_HD __host__ __device__ __forceinline__
#else
#define IMQ_HD inline
#endif

namespace imq_runs {

constexpr int kMaxShards = 16;

struct RunPlan {
  int32_t total;        // tiles of the program
  int32_t run;          // tiles per dealt run
  int32_t static_runs;  // dealt runs
  int32_t runs;         // all runs; a run index >= runs starts past the last tile
  int32_t dyn_run;      // tiles per claimed run (the last may be shorter)
  int32_t waves;        // wavefronts in the grid

  IMQ_HD int start_of(int r) const {
    return r < static_runs ? r * run : (r < runs ? static_runs * run + (r - static_runs) * dyn_run : total);
  }
  IMQ_HD int length_of(int r) const {
    if (r < static_runs) return run;
    if (r >= runs) return dyn_run;
    const int left = total - start_of(r);
    return left < dyn_run ? left : dyn_run;
  }
};

// A position in a wavefront's sequence of tiles: run r (global), tile t of the run.
struct Pos {
  int r, t;
};

template <class Plan>
IMQ_HD int tile_of(const Plan& p, const Pos& q) { return p.start_of(q.r) + q.t; }

// Runs the load cursor has claimed that the compute cursor has not reached yet.
struct ClaimQueue {
  int qa = 0, qb = 0, qn = 0;
};

// One claim's outcome: the counter's previous value `old` names run lo + old of the
// shard's `count`, or the end.
IMQ_HD int claimed_run(uint32_t old, int lo, int count, int end) {
  return (int)old < count ? lo + (int)old : end;
}

// The claim number that returns a shard's counter to zero: every wavefront of the shard
// makes one failed claim.
IMQ_HD uint32_t last_claim_of(int count, int waves) { return (uint32_t)(count + waves - 1); }

// Moves the load cursor one tile on; at the end of a run it takes the next dealt run or,
// with none left, claims (claim() returns a run index, or p.runs past the end).
template <class Plan, class Claim>
IMQ_HD void step_load(const Plan& p, Pos& q, ClaimQueue& cq, Claim&& claim) {
  if (++q.t < p.length_of(q.r)) return;
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
IMQ_HD void step_compute(const Plan& p, Pos& q, ClaimQueue& cq) {
  if (++q.t < p.length_of(q.r)) return;
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
// run per wavefront, the last `dyn_percent` of the rounds (at least one, when there are
// two or more) claimed in runs of `dyn_run` tiles from up to kMaxShards counters;
// workgroup b claims from shard (b / 8) % shards, so that every shard is served by
// workgroups of all eight XCDs.
struct ShardPlan {
  RunPlan plan;
  int32_t shards;
  int32_t shard_lo[kMaxShards + 1];
  int32_t shard_waves[kMaxShards];
};

IMQ_HD int shard_of_group(int block, int shards) { return (block >> 3) % shards; }

inline ShardPlan plan_runs(int total, int grid, int waves_per_group, int run_target, int dyn_run,
                           int dyn_percent) {
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
  int static_runs = (total + R - 1) / R, nruns = static_runs;
  if (dealt < rounds && (int64_t)V * dealt * R < total) {
    static_runs = V * dealt;
    nruns = static_runs + (total - static_runs * R + dyn_run - 1) / dyn_run;
  }
  s.plan.total = total;
  s.plan.run = R;
  s.plan.static_runs = static_runs;
  s.plan.runs = nruns;
  s.plan.dyn_run = dyn_run;
  s.plan.waves = V;
  int shards = grid / 8;
  if (shards > kMaxShards) shards = kMaxShards;
  if (shards < 1) shards = 1;
  s.shards = shards;
  for (int k = 0; k <= shards; ++k)
    s.shard_lo[k] = static_runs + (int)((int64_t)(nruns - static_runs) * k / shards);
  for (int k = 0; k < kMaxShards; ++k) s.shard_waves[k] = 0;
  for (int b = 0; b < grid; ++b) s.shard_waves[shard_of_group(b, shards)] += waves_per_group;
  return s;
}

}  // namespace imq_runs
