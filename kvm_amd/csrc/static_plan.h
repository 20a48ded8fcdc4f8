// Static schedules, host side: a bundle whose dependency DAG is known before launch is compiled into one program per
// worker (reference design: include/mvm_static.h, per-worker programs from HEFT list scheduling; path choice
// mvm_exec.cu:2146-2164). On the device (kvm_static_kernel in exec.hip) a worker runs its program in order:
//   * a dependency between two tasks of one worker is its program order (a workgroup barrier, nothing else);
//   * a dependency across workers is a wait on the other worker's progress watermark: progress[w] >= n means the first
//     n tasks of w's program have finished and their stores are agent-visible. Only tasks another worker waits for
//     publish their position.
// No ready queue, no per-edge atomic. Plain C++ (no HIP types): tests drive it through kvm_static_plan on the CPU.
//
// Dissolved no-ops (reference: mvm_dissolve_noops, mvm_exec.cu:212-296, a host transform of untraced runs): a no-op
// that publishes nothing and waits for nothing only orders tasks, so with `dissolve` it gets no worker and no program
// slot. Its successors wait directly for its predecessors: the no-op becomes a wait set (per worker, the newest
// program position among its predecessors, through chains of dissolved no-ops), stored once; a successor's wait list
// holds one reference to it, Wait{-1 - count, start}, that the lanes expand.
#pragma once
#include <algorithm>
#include <cstdint>
#include <map>
#include <queue>
#include <stdexcept>
#include <string>
#include <vector>
#include "../../include/mvm_task_abi.h"

namespace kvms {

struct Wait { int32_t worker, need; };

struct Plan {
  int workers = 0, nt = 0, dissolved = 0;
  std::vector<int> prog_off, prog;          // program of worker w: prog[prog_off[w] .. prog_off[w + 1])
  std::vector<int> worker_of, pos_of;       // per task: its worker and its index in that worker's program
  std::vector<int> wait_off;                // per task: its cross-worker waits at waits[wait_off[t] .. wait_off[t + 1])
  std::vector<Wait> waits;                  // per-task lists, then the wait sets' entries
  std::vector<char> publishes;              // per task: some task of another worker waits for it
  double makespan_us = 0, work_us = 0;      // the list scheduler's prediction and the summed task costs
  int cross_edges = 0, edges = 0;
};

// The full dependency DAG: the successor CSR plus the orderings version waits imply (publishers of one variable in
// version order; a waiter after the in-bundle publisher of the newest version it needs). Duplicate edges removed.
inline std::vector<std::vector<int>> build_dag(const MvmTaskDesc* t, int n, const int32_t* succ) {
  std::vector<std::vector<int>> out(n);
  for (int i = 0; i < n; ++i)
    for (int k = 0; k < t[i].succ_cnt; ++k) out[i].push_back(succ[t[i].succ_off + k]);
  std::map<int, std::vector<std::pair<int, int>>> pubs;   // variable -> (version, publisher)
  for (int i = 0; i < n; ++i) if (t[i].pub_var >= 0) pubs[t[i].pub_var].push_back({t[i].pub_ver, i});
  for (auto& kv : pubs) {
    auto& v = kv.second;
    std::sort(v.begin(), v.end());
    for (size_t j = 1; j < v.size(); ++j) {
      if (v[j].first == v[j - 1].first) throw std::invalid_argument("two tasks publish version " + std::to_string(v[j].first) + " of variable " + std::to_string(kv.first));
      out[v[j - 1].second].push_back(v[j].second);
    }
  }
  for (int i = 0; i < n; ++i) {
    if (t[i].wait_var < 0) continue;
    auto it = pubs.find(t[i].wait_var);
    if (it == pubs.end()) continue;
    const auto& v = it->second;
    auto u = std::upper_bound(v.begin(), v.end(), std::make_pair(t[i].wait_ver, 0x7fffffff));
    if (u == v.begin()) continue;                 // satisfied by the variable's value before the run
    --u;
    if (u->second != i) out[u->second].push_back(i);
  }
  for (auto& e : out) { std::sort(e.begin(), e.end()); e.erase(std::unique(e.begin(), e.end()), e.end()); }
  return out;
}

// Whether every version wait is decided inside the graph: the newest version a waiter needs is published by a task of
// the graph, or was already reached before the run (base version). A wait on a version published elsewhere (another
// launch, the host) cannot be planned.
inline bool feasible(const MvmTaskDesc* t, int n, const int* base_versions, int nvars, std::string* why) {
  std::map<int, int> newest;   // variable -> newest version published in the graph
  for (int i = 0; i < n; ++i) if (t[i].pub_var >= 0) newest[t[i].pub_var] = std::max(newest[t[i].pub_var], t[i].pub_ver);
  for (int i = 0; i < n; ++i) {
    const int v = t[i].wait_var;
    if (v < 0) continue;
    const int have = std::max(v < nvars ? base_versions[v] : 0, newest.count(v) ? newest[v] : 0);
    if (have < t[i].wait_ver) {
      if (why) *why = "task " + std::to_string(i) + " waits for version " + std::to_string(t[i].wait_ver) + " of variable " + std::to_string(v) +
                      ", which no task of the graph publishes";
      return false;
    }
  }
  return true;
}

// HEFT list scheduling: tasks in decreasing upward rank (cost plus the longest costed path below, a cross-worker edge
// costing comm_us), each to the worker where it finishes first; a predecessor on the same worker costs no
// communication. The candidates for a task are its predecessors' workers and the worker that frees up first (every
// other worker can only start it later than that one). Rank order is topological (costs are positive), so every
// program is consistent with the DAG and a wait only ever names an earlier task: the waits cannot form a cycle. Each
// task's waits keep, per other worker, only the newest position not already covered by an earlier wait of the same
// program.
inline Plan plan(const MvmTaskDesc* t, int n, const int32_t* succ, const std::vector<double>& cost_us, int workers, double comm_us = 1.5,
                 bool dissolve = false) {
  if (n < 1 || workers < 1) throw std::invalid_argument("empty graph or no workers");
  std::vector<std::vector<int>> out = build_dag(t, n, succ);
  std::vector<std::vector<int>> in(n);
  int edges = 0;
  for (int i = 0; i < n; ++i) for (int j : out[i]) { in[j].push_back(i); ++edges; }
  // topological order (Kahn), then upward ranks in reverse
  std::vector<int> deg(n), topo;
  topo.reserve(n);
  for (int i = 0; i < n; ++i) { deg[i] = (int)in[i].size(); if (!deg[i]) topo.push_back(i); }
  for (size_t h = 0; h < topo.size(); ++h) for (int j : out[topo[h]]) if (--deg[j] == 0) topo.push_back(j);
  if ((int)topo.size() != n) throw std::invalid_argument("dependency cycle");
  std::vector<char> gone(n, 0);
  if (dissolve)
    for (int i = 0; i < n; ++i)
      gone[i] = t[i].op_id == 0 && t[i].pub_var < 0 && t[i].wait_var < 0 && !in[i].empty() && !out[i].empty();
  // Upward ranks; a dissolved no-op adds no cost and no hop of its own (the hop is counted on its in-edges).
  std::vector<double> rank(n);
  for (int k = n - 1; k >= 0; --k) {
    const int i = topo[k];
    double below = 0;
    for (int j : out[i]) below = std::max(below, (gone[i] ? 0.0 : comm_us) + rank[j]);
    rank[i] = (gone[i] ? 0.0 : cost_us[i]) + below;
  }
  std::vector<int> order(n);
  for (int i = 0; i < n; ++i) order[i] = i;
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return rank[a] > rank[b]; });
  Plan P;
  P.workers = workers; P.nt = n; P.edges = edges;
  P.worker_of.assign(n, -1); P.pos_of.assign(n, -1);
  std::vector<double> finish(n, 0), avail(workers, 0);
  std::vector<std::vector<int>> progs(workers);
  typedef std::pair<double, int> Slot;   // (free time, worker), lazily updated
  std::priority_queue<Slot, std::vector<Slot>, std::greater<Slot>> freeq;
  for (int w = 0; w < workers; ++w) freeq.push({0.0, w});
  // Wait set of a dissolved no-op: per worker (ascending) the newest position needed and the latest finish there;
  // f1 / w1 the latest finish and its worker, f2 the latest on any other worker.
  struct Set { std::vector<int> wk, need; std::vector<double> fin; double f1 = 0, f2 = 0; int w1 = -1; };
  std::vector<Set> sets(n);
  auto set_ready = [&](const Set& S, int w) {
    const double other = w == S.w1 ? S.f2 : S.f1;   // latest finish on a worker other than w (0: none)
    double r = other > 0 ? other + comm_us : 0.0;
    auto it = std::lower_bound(S.wk.begin(), S.wk.end(), w);
    if (it != S.wk.end() && *it == w) r = std::max(r, S.fin[it - S.wk.begin()]);
    return r;
  };
  std::vector<int> cand;
  std::map<int, std::pair<int, double>> acc;
  for (int i : order) {
    if (gone[i]) {
      acc.clear();
      for (int p : in[i]) {
        if (!gone[p]) {
          auto& e = acc[P.worker_of[p]];
          e.first = std::max(e.first, P.pos_of[p] + 1); e.second = std::max(e.second, finish[p]);
        } else {
          const Set& q = sets[p];
          for (size_t k = 0; k < q.wk.size(); ++k) { auto& e = acc[q.wk[k]]; e.first = std::max(e.first, q.need[k]); e.second = std::max(e.second, q.fin[k]); }
        }
      }
      Set& S = sets[i];
      for (auto& kv : acc) {
        S.wk.push_back(kv.first); S.need.push_back(kv.second.first); S.fin.push_back(kv.second.second);
        if (kv.second.second > S.f1) { S.f2 = S.f1; S.f1 = kv.second.second; S.w1 = kv.first; }
        else S.f2 = std::max(S.f2, kv.second.second);
      }
      finish[i] = S.f1;
      ++P.dissolved;
      continue;
    }
    cand.clear();
    for (int p : in[i]) cand.push_back(gone[p] ? sets[p].w1 : P.worker_of[p]);
    while (freeq.top().first != avail[freeq.top().second]) freeq.pop();   // drop stale entries
    cand.push_back(freeq.top().second);
    double best = 1e300; int bw = -1;
    for (int w : cand) {
      if (w < 0) continue;
      double ready = avail[w];
      for (int p : in[i]) ready = std::max(ready, gone[p] ? set_ready(sets[p], w) : finish[p] + (P.worker_of[p] == w ? 0.0 : comm_us));
      if (ready + cost_us[i] < best || (ready + cost_us[i] == best && w < bw)) { best = ready + cost_us[i]; bw = w; }
    }
    P.worker_of[i] = bw; P.pos_of[i] = (int)progs[bw].size();
    progs[bw].push_back(i);
    finish[i] = best;
    avail[bw] = best;
    freeq.push({best, bw});
    P.makespan_us = std::max(P.makespan_us, best);
    P.work_us += cost_us[i];
  }
  P.prog_off.assign(workers + 1, 0);
  for (int w = 0; w < workers; ++w) { P.prog_off[w + 1] = P.prog_off[w] + (int)progs[w].size(); P.prog.insert(P.prog.end(), progs[w].begin(), progs[w].end()); }
  // waits, reduced per program against what earlier tasks of the same program already waited for; a dissolved
  // predecessor is one reference to its wait set (emitted once, after the per-task lists)
  P.publishes.assign(n, 0);
  P.wait_off.assign(n + 1, 0);
  std::vector<std::vector<Wait>> tw(n);
  std::vector<int> known(workers, 0), set_ref(n, -1);
  std::vector<int> set_order;                  // dissolved no-ops referenced, in first-reference order
  for (int w = 0; w < workers; ++w) {
    std::fill(known.begin(), known.end(), 0);
    for (int i : progs[w]) {
      std::map<int, int> need;   // other worker -> newest position needed
      for (int p : in[i]) {
        if (gone[p]) continue;
        const int pw = P.worker_of[p];
        if (pw == w) continue;
        ++P.cross_edges;
        need[pw] = std::max(need[pw], P.pos_of[p] + 1);
      }
      for (int p : in[i]) {
        if (!gone[p]) continue;
        const Set& S = sets[p];
        bool covered = true;     // every entry already waited for by this program (or its own worker's order)
        for (size_t k = 0; k < S.wk.size() && covered; ++k) covered = S.wk[k] == w || S.need[k] <= known[S.wk[k]];
        if (covered) continue;
        if (set_ref[p] < 0) { set_ref[p] = (int)set_order.size(); set_order.push_back(p); }
        tw[i].push_back(Wait{-1 - (int)S.wk.size(), p});   // start index fixed below
        for (size_t k = 0; k < S.wk.size(); ++k) {
          if (S.wk[k] == w) continue;
          ++P.cross_edges;
          known[S.wk[k]] = std::max(known[S.wk[k]], S.need[k]);
          P.publishes[P.prog[P.prog_off[S.wk[k]] + S.need[k] - 1]] = 1;
        }
      }
      for (auto& kv : need)
        if (kv.second > known[kv.first]) {
          known[kv.first] = kv.second;
          tw[i].push_back(Wait{kv.first, kv.second});
          P.publishes[P.prog[P.prog_off[kv.first] + kv.second - 1]] = 1;
        }
    }
  }
  for (int i = 0; i < n; ++i) P.wait_off[i + 1] = P.wait_off[i] + (int)tw[i].size();
  for (int i = 0; i < n; ++i) P.waits.insert(P.waits.end(), tw[i].begin(), tw[i].end());
  std::vector<int> set_start(n, -1);
  for (int p : set_order) {
    set_start[p] = (int)P.waits.size();
    const Set& S = sets[p];
    for (size_t k = 0; k < S.wk.size(); ++k) P.waits.push_back(Wait{S.wk[k], S.need[k]});
  }
  for (int k = 0; k < P.wait_off[n]; ++k)
    if (P.waits[k].worker < 0) P.waits[k].need = set_start[P.waits[k].need];
  return P;
}

}  // namespace kvms
