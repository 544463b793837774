// On-device scheduler: the algorithm of sas_metadata_build (sas_metadata.cpp),
// run by one workgroup on the GPU from device-resident sequence lengths, with
// the same output word for word. A call then needs no host synchronisation:
// the lengths never leave the GPU, and a caller can capture scheduler,
// attention and merge in one HIP graph.
//
// Parallel parts: per-item block counts, the budget bisection (each round
// evaluates the greedy fill at every midpoint of the next ten levels of the
// bisection tree, one midpoint per thread, then one thread replays the
// host's exact bisection path through those results), the per-core costs.
// Sequential parts (thread 0, O(items + cores)): the final greedy fill with
// its cursors, the FA rows, partial slots and FD rows.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/sas_mi355x.h"
#include "sas_items.h"

namespace sas {
void set_error(const std::string& msg);
}

namespace sasdev {

constexpr int NT = 1024;            // threads of the scheduling workgroup
constexpr int LEVELS = 10;          // bisection levels evaluated per round (NT - 1 nodes)
constexpr int64_t NO_SPLIT = INT64_MAX / 4;
constexpr int64_t SPLIT_PENALTY = 3;  // same rule and constant as the host scheduler

struct Cursor {
  int32_t i;  // item index
  int32_t j;  // first block not yet assigned inside item i
};

// Greedy fill under `budget` (sas_metadata.cpp: greedy). Counts cores, stopping
// once the count exceeds `stop_after` (the bisection only asks "<= num_cores");
// records the end cursors when `ends` is given.
__device__ int greedy(const int32_t* nblk, int n, int64_t c_item, int64_t budget,
                      int64_t min_split, int stop_after, Cursor* ends) {
  int i = 0;
  int64_t j = 0;
  int cores = 0;
  while (i < n) {
    ++cores;
    if (cores > stop_after) return cores;
    int64_t used = 0;
    while (i < n) {
      const int64_t left = (int64_t)nblk[i] - j;
      const int64_t need = c_item + left;
      if (used + need <= budget) {
        used += need;
        ++i;
        j = 0;
        continue;
      }
      const int64_t room = budget - used - c_item;
      if (used == 0) {
        const int64_t take = room > min_split ? room : min_split;
        if (take >= left || left - take < min_split) {
          ++i;
          j = 0;
        } else {
          j += take;
        }
        break;
      }
      if (room >= min_split && left - room >= min_split) j += room;
      break;
    }
    if (ends) ends[cores - 1] = Cursor{i, (int32_t)j};
  }
  return cores;
}

// cost of core c's range [s, e) (sas_metadata.cpp: makespan, one term)
__device__ int64_t core_cost(const int32_t* nblk, int n, int64_t c_item, Cursor s, Cursor e) {
  int64_t cost = 0;
  for (int i = s.i; i < n && (i < e.i || (i == e.i && e.j > 0)); ++i) {
    const int64_t lo = i == s.i ? s.j : 0;
    const int64_t hi = i == e.i ? e.j : nblk[i];
    cost += c_item + (hi - lo);
  }
  return cost;
}

struct Params {
  int32_t* meta;
  const int32_t* act_q;         // [batch] query rows, or null: every batch has uniform_q
  const int32_t* seqused_kv;    // [batch]
  int32_t batch, uniform_q, num_heads, m_base, ori_win_left, scenario, cmp_ratio, cmp_topk;
  int32_t num_cores, s2_base, min_split_blocks, fd_head_chunk;
};

__global__ __launch_bounds__(NT) void sched_kernel(const Params p) {
  __shared__ int32_t nblk[SAS_DEV_SCHED_MAX_ITEMS];
  __shared__ int32_t istart[SAS_DEV_SCHED_MAX_BATCH + 1];  // first item of each batch
  __shared__ Cursor ends[SAS_AIC_CORE_NUM];
  __shared__ uint8_t pred[NT];
  __shared__ int64_t s_lo, s_hi, s_total, s_longest, s_span;
  __shared__ int s_err, s_ncore, s_nsplit_ok;

  const int tid = threadIdx.x;
  int32_t* meta = p.meta;
  // clear the whole buffer with vector stores (no memset node when captured)
  for (int k = tid; k < SAS_META_SIZE; k += NT) meta[k] = 0;
  if (tid == 0) {
    s_err = 0;
    s_total = 0;
    s_longest = 0;
    s_span = 0;
  }
  __syncthreads();

  const int batch = p.batch;
  const int hblocks = (p.num_heads + p.m_base - 1) / p.m_base;
  // ---- items per batch and their prefix (thread 0 scans; batch <= MAX_BATCH) ----
  if (tid == 0) {
    int64_t acc = 0;
    for (int b = 0; b < batch; ++b) {
      const int aq = p.act_q ? p.act_q[b] : p.uniform_q;
      const int ak = p.seqused_kv[b];
      istart[b] = (int32_t)acc;
      if (aq < 0 || ak < 0) s_err = 1;
      acc += (int64_t)(aq > 0 ? aq : 0) * hblocks;
      if (acc > SAS_DEV_SCHED_MAX_ITEMS) {
        s_err = 2;
        acc = SAS_DEV_SCHED_MAX_ITEMS;
      }
    }
    istart[batch] = (int32_t)acc;
  }
  __syncthreads();
  if (s_err) {
    if (tid == 0) meta[SAS_CFG_OFFSET + 1] = -s_err;  // no magic: the attention kernel refuses it
    return;
  }
  const int n = istart[batch];
  const int64_t c_item = 1 + ((p.num_heads < p.m_base ? p.num_heads : p.m_base) + 31) / 32;

  // ---- block count of every item (golden item geometry, sas_items.h) ----
  int64_t my_total = 0, my_longest = 0;
  for (int i = tid; i < n; i += NT) {
    int lo = 0, hi = batch;  // last b with istart[b] <= i
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (istart[mid] <= i) lo = mid; else hi = mid;
    }
    const int b = lo;
    const int s = (i - istart[b]) / hblocks;
    const int aq = p.act_q ? p.act_q[b] : p.uniform_q;
    const sas::ItemGeom g = sas::item_geom(aq, p.seqused_kv[b], s, p.ori_win_left, p.scenario,
                                           p.cmp_ratio, p.cmp_topk);
    const int64_t len = (int64_t)g.n_win + g.n_cmp;
    const int32_t nb = (int32_t)((len + p.s2_base - 1) / p.s2_base);
    nblk[i] = nb;
    my_total += c_item + nb;
    my_longest = my_longest > c_item + nb ? my_longest : c_item + nb;
  }
  atomicAdd((unsigned long long*)&s_total, (unsigned long long)my_total);
  atomicMax((unsigned long long*)&s_longest, (unsigned long long)my_longest);
  __syncthreads();

  int ncore = 1;
  if (n > 0) {
    // ---- bisection over the budget, ten levels per round ----
    if (tid == 0) {
      s_lo = 1;
      s_hi = s_total;
    }
    __syncthreads();
    for (;;) {
      const int64_t lo = s_lo, hi = s_hi;
      if (lo >= hi) break;
      if (tid < NT - 1) {
        const int node = tid + 1;  // heap numbering; depth = floor(log2(node))
        const int depth = 31 - __clz(node);
        int64_t l = lo, h = hi;
        bool live = true;
        for (int d = depth - 1; d >= 0; --d) {
          if (l >= h) {
            live = false;
            break;
          }
          const int64_t mid = l + (h - l) / 2;
          if ((node >> d) & 1) l = mid + 1; else h = mid;
        }
        if (live && l < h) {
          const int64_t mid = l + (h - l) / 2;
          pred[tid] = greedy(nblk, n, c_item, mid, p.min_split_blocks, p.num_cores, nullptr) <=
                      p.num_cores;
        }
      }
      __syncthreads();
      if (tid == 0) {
        int64_t l = lo, h = hi;
        int node = 1;
        for (int d = 0; d < LEVELS && l < h; ++d) {
          const int64_t mid = l + (h - l) / 2;
          if (pred[node - 1]) {
            h = mid;
            node = 2 * node;
          } else {
            l = mid + 1;
            node = 2 * node + 1;
          }
        }
        s_lo = l;
        s_hi = h;
      }
      __syncthreads();
    }
    // ---- the fill at the chosen budget, then the no-split alternative ----
    if (tid == 0)
      s_ncore = greedy(nblk, n, c_item, s_lo, p.min_split_blocks, SAS_AIC_CORE_NUM, ends);
    if (tid == 64)  // another wave, concurrently
      s_nsplit_ok = greedy(nblk, n, c_item, s_longest, NO_SPLIT, p.num_cores, nullptr) <=
                    p.num_cores;
    __syncthreads();
    ncore = s_ncore;
    int64_t my_span = 0;
    for (int c = tid; c < ncore && ncore <= SAS_AIC_CORE_NUM; c += NT) {
      const Cursor s = c == 0 ? Cursor{0, 0} : ends[c - 1];
      const int64_t cost = core_cost(nblk, n, c_item, s, ends[c]);
      my_span = my_span > cost ? my_span : cost;
    }
    atomicMax((unsigned long long*)&s_span, (unsigned long long)my_span);
    __syncthreads();
    if (tid == 0 && s_longest <= s_span + SPLIT_PENALTY && s_nsplit_ok)
      s_ncore = greedy(nblk, n, c_item, s_longest, NO_SPLIT, SAS_AIC_CORE_NUM, ends);
    __syncthreads();
    ncore = s_ncore;
    if (ncore > p.num_cores) {
      if (tid == 0) meta[SAS_CFG_OFFSET + 1] = -3;  // capacity
      return;
    }
  } else if (tid == 0) {
    ends[0] = Cursor{0, 0};
  }
  __syncthreads();
  if (tid != 0) return;

  // ---- FA rows, partial slots, FD rows (thread 0; the host's loops) ----
  auto item_bm = [&](int i, int32_t* out2) {
    int lo = 0, hi = batch;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (istart[mid] <= i) lo = mid; else hi = mid;
    }
    out2[0] = lo;
    out2[1] = i - istart[lo];  // m = s * hblocks + hb
  };
  auto put_cursor = [&](int32_t* row, Cursor c) {
    if (c.i < n) {
      item_bm(c.i, row);
      row[2] = c.j;
    } else {
      row[0] = batch;
      row[1] = 0;
      row[2] = 0;
    }
  };
  // pass 1: FA rows and the number of split items; a piece is partial iff it
  // is the first piece of a core that starts inside an item or the last of a
  // core that ends inside one (such items always have two or more pieces)
  int32_t slots = 0;
  int split_items = 0;
  Cursor start{0, 0};
  for (int c = 0; c < ncore; ++c) {
    int32_t* row = meta + c * SAS_FA_METADATA_SIZE;
    row[0] = 1;
    if (c == 0) {
      row[1] = row[2] = row[3] = 0;
    } else {
      put_cursor(row + 1, start);
    }
    const Cursor e = ends[c];
    put_cursor(row + 4, e);
    row[7] = slots;
    const bool first_partial = start.j > 0 && start.i < n;
    const bool last_partial = e.j > 0 && e.i < n && !(first_partial && e.i == start.i);
    slots += (first_partial ? 1 : 0) + (last_partial ? 1 : 0);
    if (last_partial) ++split_items;  // an item's first piece ends a core
    start = e;
  }
  const int mb_heads = p.num_heads < p.m_base ? p.num_heads : p.m_base;
  int chunk = p.fd_head_chunk < mb_heads ? p.fd_head_chunk : mb_heads;
  if (chunk < 1) chunk = 1;
  while ((int64_t)split_items * ((mb_heads + chunk - 1) / chunk) > SAS_AIV_CORE_NUM &&
         chunk < mb_heads)
    chunk = 2 * chunk < mb_heads ? 2 * chunk : mb_heads;
  // pass 2: FD rows, in item order (= core order of the pieces)
  int32_t nfd = 0;
  int32_t slot = 0;
  int cur = -1, cur_first = 0, cur_count = 0;
  auto flush = [&]() -> bool {
    if (cur < 0 || cur_count < 2) return true;
    for (int h0 = 0; h0 < mb_heads; h0 += chunk) {
      if (nfd >= SAS_AIV_CORE_NUM) return false;
      int32_t* row = meta + SAS_FD_OFFSET + nfd * SAS_FD_METADATA_SIZE;
      row[0] = 1;
      item_bm(cur, row + 1);
      row[3] = cur_first;
      row[4] = cur_count;
      row[5] = h0;
      row[6] = chunk < mb_heads - h0 ? chunk : mb_heads - h0;
      ++nfd;
    }
    return true;
  };
  auto piece = [&](int item) -> bool {
    if (item != cur) {
      if (!flush()) return false;
      cur = item;
      cur_first = slot;
      cur_count = 0;
    }
    ++cur_count;
    ++slot;
    return true;
  };
  start = Cursor{0, 0};
  bool ok = true;
  for (int c = 0; c < ncore && ok; ++c) {
    const Cursor e = ends[c];
    const bool first_partial = start.j > 0 && start.i < n;
    const bool last_partial = e.j > 0 && e.i < n && !(first_partial && e.i == start.i);
    if (first_partial) ok = piece(start.i);
    if (ok && last_partial) ok = piece(e.i);
    start = e;
  }
  if (ok) ok = flush();
  if (!ok) {
    meta[SAS_CFG_OFFSET + 1] = -3;
    return;
  }

  int32_t* cfg = meta + SAS_CFG_OFFSET;
  cfg[1] = p.s2_base;
  cfg[2] = ncore;
  cfg[3] = nfd;
  cfg[4] = slots;
  cfg[5] = p.num_heads;
  cfg[6] = p.m_base;
  cfg[7] = n;
  cfg[0] = SAS_META_MAGIC;
}

}  // namespace sasdev

extern "C" int sas_metadata_build_device(int32_t* meta, int batch, const int32_t* act_q,
                                         int uniform_q, const int32_t* seqused_kv, int num_heads,
                                         int m_base, int ori_win_left, int scenario, int cmp_ratio,
                                         int cmp_topk, int num_cores, int s2_base,
                                         int min_split_blocks, int fd_head_chunk, void* stream) {
  if (!meta || batch < 0 || batch > SAS_DEV_SCHED_MAX_BATCH || (batch > 0 && !seqused_kv) ||
      (!act_q && uniform_q < 0)) {
    sas::set_error("sas_metadata_build_device: null pointer or batch out of range");
    return SAS_E_INVALID;
  }
  if (num_heads < 1 || num_heads > 4096 || m_base < 1 || m_base > 4096 || scenario < 1 ||
      scenario > 3 || (scenario >= 2 && cmp_ratio < 1) || cmp_topk < 0 || num_cores < 1 ||
      num_cores > SAS_AIC_CORE_NUM || s2_base < 32 || s2_base % 32 != 0 ||
      min_split_blocks < 1 || fd_head_chunk < 1 || ori_win_left < -1) {
    sas::set_error("sas_metadata_build_device: argument out of range");
    return SAS_E_INVALID;
  }
  sasdev::Params p;
  p.meta = meta;
  p.act_q = act_q;
  p.seqused_kv = seqused_kv;
  p.batch = batch;
  p.uniform_q = uniform_q;
  p.num_heads = num_heads;
  p.m_base = m_base;
  p.ori_win_left = ori_win_left;
  p.scenario = scenario;
  p.cmp_ratio = cmp_ratio;
  p.cmp_topk = cmp_topk;
  p.num_cores = num_cores;
  p.s2_base = s2_base;
  p.min_split_blocks = min_split_blocks;
  p.fd_head_chunk = fd_head_chunk;
  hipLaunchKernelGGL(sasdev::sched_kernel, dim3(1), dim3(sasdev::NT), 0, (hipStream_t)stream, p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    sas::set_error(std::string("sas_metadata_build_device: ") + hipGetErrorString(e));
    return SAS_E_HIP;
  }
  return SAS_OK;
}
