// On-device scheduler: the algorithm of sas_metadata_build (sas_metadata.cpp),
// run by one workgroup on the GPU from device-resident sequence lengths, with
// the same output word for word. A call then needs no host synchronisation:
// the lengths never leave the GPU, and a caller can capture scheduler,
// attention and merge in one HIP graph.
//
// Work split: the per-batch prefix, slot numbers and merge-row numbers are
// block-wide scans; block counts and per-core costs are one item / core per
// thread; the budget bisection evaluates the greedy fill at every midpoint of
// the next ten levels of the bisection tree at once (one lane per midpoint),
// then one thread replays the host's exact bisection path through those
// results; the fills themselves walk the items in order with the item index
// uniform across the wave; FA and FD rows are written one core per thread.
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
constexpr int NWAVE = NT / 64;
constexpr int BWAVES = 4;           // waves evaluating bisection nodes (one per SIMD)
constexpr int BNODES = 64 * BWAVES - 1;  // nodes of BLEVELS complete levels
constexpr int BLEVELS = 8;
constexpr int64_t NO_SPLIT = INT64_MAX / 4;
constexpr int64_t SPLIT_PENALTY = 3;  // same rule and constant as the host scheduler

struct Cursor {
  int32_t i;  // item index
  int32_t j;  // first block not yet assigned inside item i
};

// The greedy fill of sas_metadata.cpp restated item by item, run by a whole
// wave: the item index is uniform (its block count is broadcast from a
// register with v_readlane, one LDS read per 64 items), and each lane fills
// under its own `budget` in O(1) per item. Per lane: the number of cores,
// counted until it exceeds `stop_after`. With `ends` (all lanes on one
// budget) lane 0 records the end cursor of every core, as the host does.
// The host's loop, item by item: a core that is open (it holds something, so
// used > 0) either takes the whole item ("fits"), or takes `room` blocks when
// both parts keep >= min_split, and closes. Then fresh cores: the rest fits in
// one (it stays open), or the core takes T = max(budget - c_item, min_split)
// blocks and closes, while at least T + min_split blocks are left -- that run
// is counted in closed form -- and the last of them takes the remainder,
// staying open when it fits the budget, closing otherwise.
__device__ int greedy_wave(const int32_t* nblk, int n, int64_t c, int64_t b, int64_t ms,
                           int stop_after, Cursor* ends) {
  const int lane = threadIdx.x & 63;
  const bool rec = ends != nullptr && lane == 0;
  int cores = 0;
  bool open = false, dead = false;
  int64_t used = 0;
  for (int i0 = 0; i0 < n; i0 += 64) {
    const int32_t chunk = i0 + lane < n ? nblk[i0 + lane] : 0;
    const int lim = n - i0 < 64 ? n - i0 : 64;
    for (int k = 0; k < lim; ++k) {
      const int i = i0 + k;
      const int64_t nb = __builtin_amdgcn_readlane(chunk, k);
      if (dead) continue;
      int64_t L = nb;
      if (open) {
        if (used + c + L <= b) {
          used += c + L;
          continue;
        }
        const int64_t room = b - used - c;
        if (room >= ms && L - room >= ms) L -= room;
        open = false;
        if (rec) ends[cores - 1] = Cursor{i, (int32_t)(nb - L)};
      }
      if (c + L <= b) {  // one fresh core holds the rest
        if (++cores > stop_after) {
          dead = true;
          continue;
        }
        open = true;
        used = c + L;
        continue;
      }
      const int64_t T = b - c > ms ? b - c : ms;
      // cores that take T and close; when there are any, T < L <= the item's
      // block count, so the division is a 32-bit one
      const int64_t ks = L >= T + ms ? (int64_t)((uint32_t)(L - T - ms) / (uint32_t)T) + 1 : 0;
      if (cores + ks + 1 > stop_after) {
        cores = stop_after + 1;
        dead = true;
        continue;
      }
      if (rec)
        for (int64_t q = 1; q <= ks; ++q) ends[cores + q - 1] = Cursor{i, (int32_t)(nb - L + q * T)};
      cores += (int)ks + 1;
      L -= ks * T;
      if (L <= b - c) {
        open = true;
        used = c + L;
      } else {
        open = false;
        if (rec) ends[cores - 1] = Cursor{i + 1, 0};
      }
    }
  }
  if (!dead && open && rec) ends[cores - 1] = Cursor{n, 0};
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

// Exclusive prefix sum of one value per thread over the workgroup (wave scans
// with shuffles, then the sixteen wave totals); *total gets the sum. Two
// barriers; `wsum` is reusable once every thread has returned.
__device__ int64_t block_excl_scan(int64_t v, int64_t* wsum, int64_t* total) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  int64_t x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int64_t y = __shfl_up(x, off);
    if (lane >= off) x += y;
  }
  if (lane == 63) wsum[wid] = x;
  __syncthreads();
  if (wid == 0) {
    int64_t t = lane < NWAVE ? wsum[lane] : 0;
#pragma unroll
    for (int off = 1; off < NWAVE; off <<= 1) {
      const int64_t y = __shfl_up(t, off);
      if (lane >= off) t += y;
    }
    if (lane < NWAVE) wsum[NWAVE + lane] = t;  // inclusive wave prefixes
  }
  __syncthreads();
  *total = wsum[2 * NWAVE - 1];
  return (wid > 0 ? wsum[NWAVE + wid - 1] : 0) + x - v;
}

struct Params {
  int32_t* meta;
  const int32_t* act_q;         // [batch] query rows, or null: every batch has uniform_q
  const int32_t* seqused_kv;    // [batch]
  int32_t batch, uniform_q, num_heads, m_base, ori_win_left, scenario, cmp_ratio, cmp_topk;
  int32_t num_cores, s2_base, min_split_blocks, fd_head_chunk;
  int32_t reuse;  // nonzero: a buffer already holding this schedule's key is kept
};

constexpr int BPT = (SAS_DEV_SCHED_MAX_BATCH + NT - 1) / NT;  // batches per thread in the prefix

__global__ __launch_bounds__(NT) void sched_kernel(const Params p) {
  __shared__ int32_t nblk[SAS_DEV_SCHED_MAX_ITEMS];
  __shared__ int32_t istart[SAS_DEV_SCHED_MAX_BATCH + 1];  // first item of each batch
  __shared__ Cursor ends[SAS_AIC_CORE_NUM];
  __shared__ uint8_t pred[NT];
  __shared__ int64_t wsum[2 * NWAVE];
  __shared__ int64_t s_lo, s_hi, s_total, s_longest, s_span;
  __shared__ int s_err, s_ncore, s_nsplit_ok, s_miss;

  const int tid = threadIdx.x;
  const int wid = tid >> 6;
  int32_t* meta = p.meta;
  int32_t* const cfg = meta + SAS_CFG_OFFSET;
  int32_t* const key = meta + SAS_META_KEY_OFFSET;
  if (tid == 0) {
    s_miss = 0;
    s_err = 0;
    s_total = 0;
    s_longest = 0;
    s_span = 0;
  }
  __syncthreads();

  const int batch = p.batch;
  const int hblocks = (p.num_heads + p.m_base - 1) / p.m_base;
  auto rows_of = [&](int b) { return p.act_q ? p.act_q[b] : p.uniform_q; };
  // ---- first item of every batch: thread t owns batches BPT t .. BPT t + BPT - 1 ----
  {
    int64_t cnt[BPT];
    int64_t mine = 0;
#pragma unroll
    for (int e = 0; e < BPT; ++e) {
      const int b = BPT * tid + e;
      cnt[e] = 0;
      if (b < batch) {
        const int aq = rows_of(b), ak = p.seqused_kv[b];
        if (aq < 0 || ak < 0) atomicOr(&s_err, 1);
        cnt[e] = (int64_t)(aq > 0 ? aq : 0) * hblocks;
      }
      mine += cnt[e];
    }
    int64_t total_items;
    int64_t at = block_excl_scan(mine, wsum, &total_items);
#pragma unroll
    for (int e = 0; e < BPT; ++e) {
      const int b = BPT * tid + e;
      if (b < batch) istart[b] = (int32_t)(at < SAS_DEV_SCHED_MAX_ITEMS ? at : SAS_DEV_SCHED_MAX_ITEMS);
      at += cnt[e];
    }
    if (tid == 0) {
      if (total_items > SAS_DEV_SCHED_MAX_ITEMS) atomicOr(&s_err, 2);
      istart[batch] = (int32_t)(total_items < SAS_DEV_SCHED_MAX_ITEMS ? total_items
                                                                      : SAS_DEV_SCHED_MAX_ITEMS);
    }
  }
  __syncthreads();
  if (s_err) {
    if (tid == 0) {
      cfg[0] = 0;  // no magic: refused
      cfg[1] = (s_err & 1) ? -1 : -2;
      key[0] = 0;
    }
    return;
  }
  const int n = istart[batch];
  const int64_t c_item = 1 + ((p.num_heads < p.m_base ? p.num_heads : p.m_base) + 31) / 32;
  auto batch_of = [&](int i) {  // last b with istart[b] <= i
    int lo = 0, hi = batch;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (istart[mid] <= i) lo = mid; else hi = mid;
    }
    return lo;
  };

  // ---- block count of every item (golden item geometry, sas_items.h) ----
  int64_t my_total = 0, my_longest = 0;
  for (int i = tid; i < n; i += NT) {
    const int b = batch_of(i);
    const int s = (i - istart[b]) / hblocks;
    const sas::ItemGeom g = sas::item_geom(rows_of(b), p.seqused_kv[b], s, p.ori_win_left,
                                           p.scenario, p.cmp_ratio, p.cmp_topk);
    const int64_t len = (int64_t)g.n_win + g.n_cmp;
    const int32_t nb = len < (1ll << 31)  // 32-bit division unless it could overflow
                           ? (int32_t)((uint32_t)(len + p.s2_base - 1) / (uint32_t)p.s2_base)
                           : (int32_t)((len + p.s2_base - 1) / p.s2_base);
    nblk[i] = nb;
    my_total += c_item + nb;
    my_longest = my_longest > c_item + nb ? my_longest : c_item + nb;
  }
  // wave sums first: one LDS atomic per wave
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    my_total += __shfl_xor(my_total, off);
    const int64_t o = __shfl_xor(my_longest, off);
    my_longest = my_longest > o ? my_longest : o;
  }
  if ((tid & 63) == 0) {
    atomicAdd((unsigned long long*)&s_total, (unsigned long long)my_total);
    atomicMax((unsigned long long*)&s_longest, (unsigned long long)my_longest);
  }
  __syncthreads();

  // ---- the buffer already holds the schedule of these inputs: keep it ----
  // Only for a buffer its owner declares persistent (p.reuse): one that nothing
  // but this scheduler writes between calls, such as a captured graph's static
  // buffer. A freshly allocated buffer may hold a stale key and config row over
  // rows that something else has since overwritten, so it is always rebuilt.
  const int keyw = 16 + batch + n;  // key words
  const bool keyable = keyw <= SAS_CFG_OFFSET - SAS_META_KEY_OFFSET;
  auto key_word = [&](int w) -> int32_t {
    if (w >= 16 + batch) return nblk[w - 16 - batch];
    if (w >= 16) return rows_of(w - 16);
    const int32_t hdr[16] = {(int32_t)SAS_KEY_MAGIC, n, batch, p.num_heads, p.m_base,
                             p.ori_win_left, p.scenario, p.cmp_ratio, p.cmp_topk, p.num_cores,
                             p.s2_base, p.min_split_blocks, p.fd_head_chunk, 0, 0, 0};
    return hdr[w];
  };
  if (keyable && p.reuse) {
    bool miss = tid == 0 && cfg[0] != SAS_META_MAGIC;
    for (int w = tid; w < keyw; w += NT) miss = miss || key[w] != key_word(w);
    if (miss) s_miss = 1;
    __syncthreads();
    if (!s_miss) return;
  }
  // ---- rebuild: clear everything (vector stores; no memset node when captured) ----
  for (int k = tid; k < SAS_META_SIZE; k += NT) meta[k] = 0;  // rows, key region, config
  __syncthreads();

  int ncore = 1;
  if (n > 0) {
    // ---- smallest budget whose fill fits num_cores (the host's search) ----
    // doubling search: lane k of wave 0 evaluates h_k = min(total, h_0 2^k)
    if (wid == 0) {
      const int64_t h0 = (s_total + p.num_cores - 1) / p.num_cores;
      int64_t hk = h0 > 1 ? h0 : 1;
      for (int k = 0; k < (tid & 63) && hk < s_total; ++k) hk = 2 * hk < s_total ? 2 * hk : s_total;
      const int cores = greedy_wave(nblk, n, c_item, hk, p.min_split_blocks, p.num_cores, nullptr);
      const bool stop = hk >= s_total || cores <= p.num_cores;
      const unsigned long long m = __ballot(stop);  // lane 63 reaches total for any total
      const int ks = __ffsll((long long)m) - 1;
      const int64_t hi = __shfl(hk, ks);
      const int64_t prev = __shfl(hk, ks > 0 ? ks - 1 : 0);
      if (tid == 0) {
        s_lo = ks > 0 ? prev + 1 : 1;
        s_hi = hi;
      }
    }
    __syncthreads();
    // bisection on [lo, hi]: each round evaluates every midpoint of the next
    // BLEVELS levels of the bisection tree (one lane per node, one wave per
    // SIMD), then thread 0 replays the host's path through them
    for (;;) {
      const int64_t lo = s_lo, hi = s_hi;
      if (lo >= hi) break;
      if (wid < BWAVES) {
        const int node = tid + 1;  // heap numbering; depth = floor(log2(node))
        const int depth = 31 - __clz(node);
        int64_t l = lo, h = hi;
        bool live = tid < BNODES;
        for (int d = depth - 1; d >= 0 && live; --d) {
          if (l >= h) {
            live = false;
            break;
          }
          const int64_t mid = l + (h - l) / 2;
          if ((node >> d) & 1) l = mid + 1; else h = mid;
        }
        live = live && l < h;
        const int64_t mid = live ? l + (h - l) / 2 : hi;  // every lane takes part
        const int cores = greedy_wave(nblk, n, c_item, mid, p.min_split_blocks, p.num_cores,
                                      nullptr);
        if (live) pred[tid] = cores <= p.num_cores;
      }
      __syncthreads();
      if (tid == 0) {
        int64_t bl = lo, bh = hi;
        int nd = 1;
        for (int d = 0; d < BLEVELS && bl < bh; ++d) {
          const int64_t m = bl + (bh - bl) / 2;
          if (pred[nd - 1]) {
            bh = m;
            nd = 2 * nd;
          } else {
            bl = m + 1;
            nd = 2 * nd + 1;
          }
        }
        s_lo = bl;
        s_hi = bh;
      }
      __syncthreads();
    }
    // ---- the fill at the chosen budget (wave 0) and the no-split count (wave 1) ----
    if (wid == 0) {
      const int c = greedy_wave(nblk, n, c_item, s_lo, p.min_split_blocks, SAS_AIC_CORE_NUM, ends);
      if (tid == 0) s_ncore = c;
    } else if (wid == 1) {
      const int c = greedy_wave(nblk, n, c_item, s_longest, NO_SPLIT, p.num_cores, nullptr);
      if (tid == 64) s_nsplit_ok = c <= p.num_cores;
    }
    __syncthreads();
    ncore = s_ncore;
    int64_t my_span = 0;
    for (int c = tid; c < ncore && ncore <= SAS_AIC_CORE_NUM; c += NT) {
      const Cursor s = c == 0 ? Cursor{0, 0} : ends[c - 1];
      const int64_t cost = core_cost(nblk, n, c_item, s, ends[c]);
      my_span = my_span > cost ? my_span : cost;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const int64_t o = __shfl_xor(my_span, off);
      my_span = my_span > o ? my_span : o;
    }
    if ((tid & 63) == 0) atomicMax((unsigned long long*)&s_span, (unsigned long long)my_span);
    __syncthreads();
    if (s_longest <= s_span + SPLIT_PENALTY && s_nsplit_ok && wid == 0) {
      const int c = greedy_wave(nblk, n, c_item, s_longest, NO_SPLIT, SAS_AIC_CORE_NUM, ends);
      if (tid == 0) s_ncore = c;
    }
    __syncthreads();
    ncore = s_ncore;
    if (ncore > p.num_cores) {
      if (tid == 0) cfg[1] = -3;  // over capacity
      return;
    }
  } else if (tid == 0) {
    ends[0] = Cursor{0, 0};
  }
  __syncthreads();

  // ---- FA rows (one core per thread) and partial slots ----
  // A piece is partial iff it is the first piece of a core that starts inside
  // an item or the last one of a core that ends inside one; the host numbers
  // them in core order, first before last. An item is split iff it owns such
  // a piece, and its first piece is the "last" partial piece of some core.
  auto put_cursor = [&](int32_t* row, Cursor c) {
    if (c.i < n) {
      const int b = batch_of(c.i);
      row[0] = b;
      row[1] = c.i - istart[b];  // m = query row * head blocks + head block
      row[2] = c.j;
    } else {
      row[0] = batch;
      row[1] = 0;
      row[2] = 0;
    }
  };
  const int c = tid;  // ncore <= SAS_AIC_CORE_NUM < NT
  Cursor cs{0, 0}, ce{0, 0};
  bool first_partial = false, last_partial = false;
  if (c < ncore) {
    cs = c == 0 ? Cursor{0, 0} : ends[c - 1];
    ce = ends[c];
    first_partial = cs.j > 0 && cs.i < n;
    last_partial = ce.j > 0 && ce.i < n && !(first_partial && ce.i == cs.i);
  }
  int64_t slots_total, split_total;
  const int64_t slot_base =
      block_excl_scan((first_partial ? 1 : 0) + (last_partial ? 1 : 0), wsum, &slots_total);
  __syncthreads();  // wsum reused
  const int64_t split_before = block_excl_scan(last_partial ? 1 : 0, wsum, &split_total);
  if (c < ncore) {
    int32_t* row = meta + c * SAS_FA_METADATA_SIZE;
    row[0] = 1;
    if (c == 0) {
      row[1] = row[2] = row[3] = 0;  // core 0 starts at the origin (metadata.py:985-987)
    } else {
      put_cursor(row + 1, cs);
    }
    put_cursor(row + 4, ce);
    row[7] = (int32_t)slot_base;
  }
  // ---- FD rows: the split items in order, each in head chunks ----
  const int mb_heads = p.num_heads < p.m_base ? p.num_heads : p.m_base;
  int chunk = p.fd_head_chunk < mb_heads ? p.fd_head_chunk : mb_heads;
  if (chunk < 1) chunk = 1;
  while (split_total * ((mb_heads + chunk - 1) / chunk) > SAS_AIV_CORE_NUM && chunk < mb_heads)
    chunk = 2 * chunk < mb_heads ? 2 * chunk : mb_heads;
  const int per_item = (mb_heads + chunk - 1) / chunk;
  const int64_t nfd = split_total * per_item;
  if (nfd > SAS_AIV_CORE_NUM) {
    if (tid == 0) cfg[1] = -3;
    return;
  }
  if (last_partial) {
    const int i = ce.i;
    int c2 = c + 1;  // cores wholly inside item i, then the one with its last piece
    while (ends[c2].i == i && ends[c2].j > 0) ++c2;
    const int32_t first_slot = (int32_t)slot_base + (first_partial ? 1 : 0);
    const int b = batch_of(i);
    int k = (int)split_before * per_item;
    for (int h0 = 0; h0 < mb_heads; h0 += chunk, ++k) {
      int32_t* row = meta + SAS_FD_OFFSET + k * SAS_FD_METADATA_SIZE;
      row[0] = 1;
      row[1] = b;
      row[2] = i - istart[b];
      row[3] = first_slot;
      row[4] = c2 - c + 1;
      row[5] = h0;
      row[6] = chunk < mb_heads - h0 ? chunk : mb_heads - h0;
    }
  }
  if (keyable)
    for (int w = tid; w < keyw; w += NT) key[w] = key_word(w);
  if (tid == 0) {
    cfg[1] = p.s2_base;
    cfg[2] = ncore;
    cfg[3] = (int32_t)nfd;
    cfg[4] = (int32_t)slots_total;
    cfg[5] = p.num_heads;
    cfg[6] = p.m_base;
    cfg[7] = n;
    cfg[0] = SAS_META_MAGIC;
  }
}

}  // namespace sasdev

extern "C" int sas_metadata_build_device(int32_t* meta, int batch, const int32_t* act_q,
                                         int uniform_q, const int32_t* seqused_kv, int num_heads,
                                         int m_base, int ori_win_left, int scenario, int cmp_ratio,
                                         int cmp_topk, int num_cores, int s2_base,
                                         int min_split_blocks, int fd_head_chunk, int reuse,
                                         void* stream) {
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
  p.reuse = reuse != 0;
  hipLaunchKernelGGL(sasdev::sched_kernel, dim3(1), dim3(sasdev::NT), 0, (hipStream_t)stream, p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    sas::set_error(std::string("sas_metadata_build_device: ") + hipGetErrorString(e));
    return SAS_E_HIP;
  }
  return SAS_OK;
}
