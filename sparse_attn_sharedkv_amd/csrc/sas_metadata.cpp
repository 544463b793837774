// Host scheduler: splits the decode work of one call over the GPU's workgroups.
//
// Role of the reference's SparseAttnSharedkvMetadata scheduler
// (metadata.py:258-1015, a port of the AICPU C++): cost-balanced contiguous
// ranges of (bn2, m, s2-block) work per core, plus FlashDecode ("FD") merge
// tasks for items whose blocks land on more than one core. Differences, by
// design: split-KV is enabled (the reference gates it off, metadata.py:323-325)
// because decode has far fewer items than MI355X's 256 CUs; the budget is found
// by a doubling search and bisection over a greedy fill instead of the
// reference's tolerance walk;
// blocks are s2_base positions of the item's concatenated [window ++ compressed]
// list rather than separately aligned window / compressed 512-blocks.
#include <stdio.h>
#include <string.h>

#include <stdint.h>

#include <algorithm>
#include <string>
#include <vector>

#include "../../include/sas_mi355x.h"
#include "sas_items.h"

namespace sas {
void set_error(const std::string& msg);
}

namespace {

struct Item {
  int32_t b, m;  // batch, m-block (query row * head blocks + head block)
  int64_t nblk;
};

struct Cursor {
  size_t i;   // item index
  int64_t j;  // first block not yet assigned inside item i
};

// Greedy fill under `budget`: each core takes whole items while they fit;
// an item that does not fit is split when both pieces keep >= min_split
// blocks. A core that is still empty always makes progress. Every piece of
// an item costs `c_item` on top of its blocks (query load + epilogue).
int greedy(const std::vector<Item>& items, int64_t c_item, int64_t budget, int64_t min_split,
           std::vector<Cursor>* ends) {
  size_t i = 0;
  int64_t j = 0;
  int cores = 0;
  const size_t n = items.size();
  while (i < n) {
    ++cores;
    int64_t used = 0;
    while (i < n) {
      const int64_t left = items[i].nblk - j;
      const int64_t need = c_item + left;
      if (used + need <= budget) {
        used += need;
        ++i;
        j = 0;
        continue;
      }
      const int64_t room = budget - used - c_item;
      if (used == 0) {
        const int64_t take = std::max(room, min_split);
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
    if (ends) ends->push_back(Cursor{i, j});
  }
  return cores;
}

// Largest per-core cost of a schedule given by its end cursors.
int64_t makespan(const std::vector<Item>& items, int64_t c_item, const std::vector<Cursor>& ends) {
  int64_t worst = 0;
  Cursor s{0, 0};
  for (const Cursor& e : ends) {
    int64_t cost = 0;
    for (size_t i = s.i; i < items.size() && (i < e.i || (i == e.i && e.j > 0)); ++i) {
      const int64_t lo = i == s.i ? s.j : 0;
      const int64_t hi = i == e.i ? e.j : items[i].nblk;
      cost += c_item + (hi - lo);
    }
    worst = std::max(worst, cost);
    s = e;
  }
  return worst;
}

}  // namespace

extern "C" int sas_metadata_build(int32_t* meta, int batch, const int32_t* act_q,
                                  const int32_t* act_kv, int num_heads, int m_base,
                                  int ori_win_left,
                                  int scenario, int cmp_ratio, int cmp_topk, int num_cores,
                                  int s2_base, int min_split_blocks, int fd_head_chunk) {
  if (!meta || batch < 0 || (batch > 0 && (!act_q || !act_kv))) {
    sas::set_error("sas_metadata_build: null pointer or negative batch");
    return SAS_E_INVALID;
  }
  if (num_heads < 1 || num_heads > 4096 || m_base < 1 || m_base > 4096 || scenario < 1 ||
      scenario > 3 ||
      (scenario >= 2 && cmp_ratio < 1) || cmp_topk < 0 || num_cores < 1 ||
      num_cores > SAS_AIC_CORE_NUM || s2_base < 32 || s2_base % 32 != 0 ||
      min_split_blocks < 1 || fd_head_chunk < 1 || ori_win_left < -1) {
    sas::set_error("sas_metadata_build: argument out of range");
    return SAS_E_INVALID;
  }
  memset(meta, 0, sizeof(int32_t) * SAS_META_SIZE);

  const int hblocks = (num_heads + m_base - 1) / m_base;
  std::vector<Item> items;
  for (int b = 0; b < batch; ++b) {
    if (act_q[b] < 0 || act_kv[b] < 0) {
      sas::set_error("sas_metadata_build: negative sequence length");
      return SAS_E_INVALID;
    }
    for (int s = 0; s < act_q[b]; ++s) {
      const sas::ItemGeom g =
          sas::item_geom(act_q[b], act_kv[b], s, ori_win_left, scenario, cmp_ratio, cmp_topk);
      const int64_t len = (int64_t)g.n_win + g.n_cmp;
      for (int hb = 0; hb < hblocks; ++hb)
        items.push_back(Item{b, s * hblocks + hb, (len + s2_base - 1) / s2_base});
    }
  }

  const int64_t c_item = 1 + (std::min(num_heads, m_base) + 31) / 32;
  std::vector<Cursor> ends;
  if (items.empty()) {
    ends.push_back(Cursor{0, 0});
  } else {
    int64_t total = 0;
    for (const Item& it : items) total += c_item + it.nblk;
    // smallest budget whose fill fits num_cores: doubling search up from the
    // average load (greedy(total) is one core, so it ends), then bisection
    int64_t lo = 1, hi = std::max<int64_t>(1, (total + num_cores - 1) / num_cores);
    while (hi < total && greedy(items, c_item, hi, min_split_blocks, nullptr) > num_cores) {
      lo = hi + 1;
      hi = std::min(total, 2 * hi);
    }
    while (lo < hi) {
      const int64_t mid = lo + (hi - lo) / 2;
      if (greedy(items, c_item, mid, min_split_blocks, nullptr) <= num_cores)
        hi = mid;
      else
        lo = mid + 1;
    }
    greedy(items, c_item, lo, min_split_blocks, &ends);
    // Splitting an item costs a merge kernel over its pieces (about
    // SPLIT_PENALTY blocks of attention time): keep whole items when they fit
    // the cores and the longest one is within that of the split makespan.
    int64_t longest = 0;
    for (const Item& it : items) longest = std::max(longest, c_item + it.nblk);
    constexpr int64_t SPLIT_PENALTY = 3;
    constexpr int64_t NO_SPLIT = INT64_MAX / 4;
    if (longest <= makespan(items, c_item, ends) + SPLIT_PENALTY &&
        greedy(items, c_item, longest, NO_SPLIT, nullptr) <= num_cores) {
      ends.clear();
      greedy(items, c_item, longest, NO_SPLIT, &ends);
    }
    if ((int)ends.size() > num_cores) {
      sas::set_error("sas_metadata_build: schedule exceeds num_cores");
      return SAS_E_CAPACITY;
    }
  }

  const size_t n = items.size();
  auto put_cursor = [&](int32_t* row, Cursor c) {
    if (c.i < n) {
      row[0] = items[c.i].b;
      row[1] = items[c.i].m;
      row[2] = (int32_t)c.j;
    } else {
      row[0] = batch;
      row[1] = 0;
      row[2] = 0;
    }
  };

  // Partial slots: in core order, one per piece that does not cover its whole item.
  std::vector<int32_t> first_slot(n, -1), n_pieces(n, 0);
  int32_t slots = 0;
  Cursor start{0, 0};
  for (size_t c = 0; c < ends.size(); ++c) {
    int32_t* row = meta + c * SAS_FA_METADATA_SIZE;
    row[0] = 1;
    if (c == 0) {
      row[1] = row[2] = row[3] = 0;  // core 0 starts at the origin (metadata.py:985-987)
    } else {
      put_cursor(row + 1, start);
    }
    put_cursor(row + 4, ends[c]);
    row[7] = slots;
    const Cursor e = ends[c];
    for (size_t i = start.i; i < n && (i < e.i || (i == e.i && e.j > 0)); ++i) {
      const bool partial = (i == start.i && start.j > 0) || (i == e.i);
      if (!partial) continue;
      if (first_slot[i] < 0) first_slot[i] = slots;
      ++n_pieces[i];
      ++slots;
    }
    start = e;
  }

  // Merge tasks: every split item, in head chunks.
  int64_t split_items = 0;
  for (size_t i = 0; i < n; ++i) split_items += n_pieces[i] > 1;
  const int mb_heads = std::min(num_heads, m_base);
  int chunk = std::max(1, std::min(fd_head_chunk, mb_heads));
  while (split_items * ((mb_heads + chunk - 1) / chunk) > SAS_AIV_CORE_NUM && chunk < mb_heads)
    chunk = std::min(mb_heads, chunk * 2);
  int32_t nfd = 0;
  for (size_t i = 0; i < n; ++i) {
    if (n_pieces[i] < 2) continue;
    for (int h0 = 0; h0 < mb_heads; h0 += chunk) {
      if (nfd >= SAS_AIV_CORE_NUM) {
        sas::set_error("sas_metadata_build: merge tasks exceed capacity");
        return SAS_E_CAPACITY;
      }
      int32_t* row = meta + SAS_FD_OFFSET + nfd * SAS_FD_METADATA_SIZE;
      row[0] = 1;
      row[1] = items[i].b;
      row[2] = items[i].m;
      row[3] = first_slot[i];
      row[4] = n_pieces[i];
      row[5] = h0;
      row[6] = std::min(chunk, mb_heads - h0);
      ++nfd;
    }
  }

  // schedule key: every input the words above are a function of
  int32_t* key = meta + SAS_META_KEY_OFFSET;
  if (16 + (int64_t)batch + (int64_t)n <= SAS_CFG_OFFSET - SAS_META_KEY_OFFSET) {
    const int32_t hdr[16] = {(int32_t)SAS_KEY_MAGIC, (int32_t)n, batch, num_heads, m_base,
                             ori_win_left, scenario, cmp_ratio, cmp_topk, num_cores, s2_base,
                             min_split_blocks, fd_head_chunk, 0, 0, 0};
    for (int w = 0; w < 16; ++w) key[w] = hdr[w];
    for (int b = 0; b < batch; ++b) key[16 + b] = act_q[b];
    for (size_t i = 0; i < n; ++i) key[16 + batch + i] = (int32_t)items[i].nblk;
  }

  int32_t* cfg = meta + SAS_CFG_OFFSET;
  cfg[0] = SAS_META_MAGIC;
  cfg[1] = s2_base;
  cfg[2] = (int32_t)ends.size();
  cfg[3] = nfd;
  cfg[4] = slots;
  cfg[5] = num_heads;
  cfg[6] = m_base;
  cfg[7] = (int32_t)n;
  return (int)ends.size();
}

extern "C" int64_t sas_workspace_bytes(int num_partial_slots, int m_base, int head_dim_v) {
  if (num_partial_slots < 0 || m_base < 0 || head_dim_v < 0) return 0;
  // fp16 partials, then fp32 lse and fp32 inverse scales
  return (int64_t)num_partial_slots * m_base * (2 * (int64_t)head_dim_v + 8);
}
