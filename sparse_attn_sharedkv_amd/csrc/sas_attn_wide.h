// Attention kernel, wide form: 128 query-head columns per workgroup — items of
// 128 heads (native bf16 / fp16 rows, or fp8 rows in either Q·Kᵀ form), or two
// consecutive query rows of 64 heads (row pairs, native rows).
//
// Included by sas_attn.hip after the shared helpers (DMA issue, index loads,
// zero row, partial scales, item geometry).
//
// One workgroup of 8 waves (two per SIMD) per item piece; wave w owns heads
// 16 w .. 16 w + 15 of the item over the whole d_qk and d_v. A gathered 32-row
// tile serves every query head of the token (the shared-KV property: one
// latent row is K for all heads and, in its first d_v columns, V), and nothing
// but the tile itself passes between waves: no partial scores, no P, no
// rescale factors go through LDS.
//   Q·Kᵀ:  Sᵀ[32 rows x 16 heads] = K·Qᵀ as two 16-row blocks with
//          v_mfma_f32_16x16x32 (A = K rows from LDS, B = Qᵀ in VGPRs). Block rb
//          holds tile row 16 rb + 4 (l / 16) + i in element i of lane l, whose
//          head is l % 16.
//   softmax: in registers; a head's 32 rows sit in lanes l, l ^ 16, l ^ 32,
//          l ^ 48 (max and sum by permlane swaps). The running max moves at every
//          tile whose max exceeds it (golden.py:187-191's rule at 32-row tiles),
//          so the largest score so far has P = 1 exactly when P is rounded to
//          the input type (golden.py:192-196).
//   P·V:   Oᵀ[512 dv x 16 heads] += Vᵀ·Pᵀ, 32 MFMAs per tile. The B operand Pᵀ
//          (k = 8 (l / 16) + e in lane l) is the lane's own eight P values:
//          element e < 4 from block 0, e >= 4 from block 1, so k = 8 g + e means
//          tile row 4 g + e (e < 4) or 16 + 4 g + e - 4 (e >= 4), and the A
//          operand Vᵀ is read (ds_read_b64_tr_b16) from exactly those rows.
// Ring of 4 stages and one barrier per tile: at the top of tile t every wave
// has waited for its own DMAs of t; the barrier publishes t and frees the
// stage of t - 1, into which the DMAs of t + 3 go between the P·V MFMAs of t.
// fp8 rows: a raw ring of 656-byte rows (3 stages, 4 in the fp8 Q·Kᵀ form) feeds
// two bf16 stages, each tile dequantized one tile ahead (see the kernel).
#pragma once

#ifndef SAS_WKPF
#define SAS_WKPF 3  // K operands in flight per wave (wide_kernel)
#endif
#ifndef SAS_WVPF
#define SAS_WVPF 3  // Vᵀ operands in flight per wave (wide_kernel)
#endif


namespace sas {

// LDS stage layout of the wide kernel (one 32-row tile).
//   main part, dims 0..511: row r in natural dim order (one 1 KB DMA
//     instruction) at wide_row_base(r) = 1056 r;
//   rope part, dims 512..575: 32 slot rows of 128 B after the main part; slot
//     row p holds tile row wide_perm(p), its 16-byte chunk c at slot
//     8 p + (c ^ ((p >> 1) & 7)) (one DMA instruction fills 8 slot rows).
// Both were chosen by measuring SQ_LDS_BANK_CONFLICT on MI355X over probe kernels
// that issue one access pattern each: the K-operand reads (ds_read_b128, lane l:
// row l % 16 of a 16-row block, 16-byte chunk 4 ks + l / 16) and the Vᵀ reads
// (ds_read_b64_tr_b16, lanes 4 a + c of group g: row 4 g + a, 8 bytes at 32 d + 8 c)
// are conflict-free in 1056-byte rows in natural order, while 1040-, 1072- and
// 1088-byte rows, and 1056-byte rows offset by 32 bytes from row 8 on, conflict
// 2-way on one pattern or the other; the rope reads are conflict-free under this
// permutation and swizzle (and 2- to 4-way without them).
constexpr int WROW = 1056;
constexpr int WMAIN = TILE * WROW;  // 33792
constexpr int WROPE = TILE * 128;   // 4096
__device__ __host__ inline int wide_row_base(int r) { return r * WROW; }
__device__ __host__ inline int wide_perm(int p) { return p ^ ((p >> 1) & 1); }
__device__ __host__ inline int wide_rope_slot(int p, int c) { return 8 * p + (c ^ ((p >> 1) & 7)); }

// The lane's index within its wave, computed where it is used: the LDS operand
// offsets below derive from it inside the tile loop, so the compiler neither
// keeps them in registers across the loop nor spills them (a spill reload there
// would wait for every DMA in flight).
__device__ inline int lane_id_here() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}
// Per-lane LDS offsets of the wide kernel's MFMA operands within a stage.
//   K (A of 16x16x32): row 16 rb + l % 16, dims 32 ks + 8 (l / 16). Main part:
//     k_main + 64 ks (+ 16 rows for rb = 1). Rope part (k-step 16 +
//     kr): slot row p = wide_perm(16 rb + l % 16) = 16 rb + wide_perm(l % 16) with
//     the same swizzle, so rb = 1 is + 16 slot rows; chunk 4 kr + l / 16 =
//     (l / 16) ^ 4 kr sits at slot (l / 16 ^ sw) ^ 4 kr, i.e. +/- 4 slots from
//     k-step 16's.
//   Vᵀ (A of 16x16x32, ds_read_b64_tr_b16): group g4 = l / 16's lanes 4 a + c point
//     at row 4 g4 + a (first read) / 16 + 4 g4 + a (second read), dv 16 d + 4 c ..
//     + 3, and lane j of the group receives dv 16 d + j of those four rows.
// Each is computed where it is first needed, so only the operand base of the
// current phase occupies a register.
__device__ inline int wide_k_main(int l) { return wide_row_base(l & 15) + 16 * (l >> 4); }
__device__ inline int wide_rope0(int l) {
  return WMAIN + 16 * wide_rope_slot(wide_perm(l & 15), l >> 4);
}
__device__ inline int wide_rope1(int l) {
  const int g4 = l >> 4, p = wide_perm(l & 15);
  return wide_rope0(l) + ((((g4 ^ ((p >> 1) & 7)) & 4) != 0) ? -64 : 64);
}
__device__ inline int wide_v(int l) { return wide_row_base(4 * (l >> 4) + ((l & 15) >> 2)) + 8 * (l & 3); }

template <int DQK, int DV, typename T, int KVF = SAS_KV_NATIVE, bool PAIR = false, bool QK8 = false>
__global__ __launch_bounds__(512) void wide_kernel(const SasAttnArgs a) {
  constexpr int NW = 8;                  // waves per workgroup
  constexpr int MB = 128;                // query heads per workgroup (columns of Sᵀ)
  // PAIR: items of 64 heads (at most 64 heads, one head block), two consecutive
  // query rows of a sequence at a time — waves 0..3 take row s, waves 4..7 row
  // s + 1, over the union of the two rows' positions, each wave masking the
  // positions its own row does not attend. Windows and dense compressed
  // prefixes only (scenarios 1, 2); a piece of a split item runs alone.
  constexpr int IMB = PAIR ? 64 : MB;    // heads per item (m-block)
  constexpr int NT = 64 * NW;            // threads
  constexpr bool ROPE = DQK == 576;      // 64 extra rope dims after the 512 main dims
  // fp8 rows (SAS_KV_FP8_DS_MLA): tiles arrive by DMA as raw 656-byte rows in a
  // ring of their own and are dequantized into the bf16 stage layout one tile
  // ahead of their use (the same bf16 values the native path computes on)
  constexpr bool FP8 = KVF == SAS_KV_FP8_DS_MLA;
  // QK8 (fp8 rows, SAS_PHASE_FP8_QK): Q·Kᵀ on v_mfma_f32_16x16x128_f8f6f4 straight
  // from the raw ring (e4m3 K blocks, bf16 rope) with the query quantized per head,
  // the block scales applied to the four block dot products; P·V on the dequantized
  // bf16 stage as in the bf16 form. The raw tile is read until its Q·Kᵀ is done, so
  // the raw ring holds one tile more, and the bf16 stages drop their rope part.
  constexpr int ROWB = FP8 ? SAS_FP8_ROW_BYTES : DQK * 2;  // bytes per cache row in HBM
  constexpr int NKS = DQK / 32;          // 16x16x32 k-steps over d_qk (18 or 16)
  constexpr int NKS_MAIN = 16;           // k-steps over the 512 main dims
  constexpr int NDV = DV / 16;           // 16-wide dv blocks (32)
  constexpr int NSTG = FP8 ? 2 : 4;      // bf16 ring depth (fp8: the tile in use, the one filled)
  constexpr int STAGE_BYTES = WMAIN + (ROPE && !QK8 ? WROPE : 0);
  constexpr int RAW_CH = SAS_FP8_ROW_BYTES / 16;  // 16-byte chunks per fp8 row (41)
  constexpr int LATENT_BYTES = 512;      // fp8 row: e4m3 dims 0..511, then 4 fp32 scales, rope
  constexpr int RAW_DMA = TILE / NW;     // fp8: raw DMA instructions per wave and tile, a row each
  constexpr uint64_t RAW_LANES = (1ull << RAW_CH) - 1;  // the lanes of a row's DMA (0 .. 40)
  constexpr int RAW_STAGE = TILE * SAS_FP8_ROW_BYTES;   // 32 rows x 656 B
  constexpr int NRAW = FP8 ? (QK8 ? 4 : 3) : 0;  // raw ring depth
  constexpr int LDS_BYTES = NSTG * STAGE_BYTES + NRAW * RAW_STAGE;
  static_assert(!FP8 || (DQK == 576 && __is_same(T, __bf16)), "fp8 rows: d_qk 576, bf16");
  static_assert(!(PAIR && FP8), "row pairs: native rows");
  static_assert(!QK8 || FP8, "fp8 Q·Kᵀ reads fp8 rows");
  static_assert(RAW_CH <= 64 && RAW_CH * 16 == SAS_FP8_ROW_BYTES, "one fp8 row per DMA");
  constexpr int RPW = TILE / NW;         // main-part DMA instructions per wave and tile (4)
  constexpr int NROPE = ROPE ? TILE / 8 : 0;  // rope DMA instructions per tile (waves w < 4)
  constexpr int RCH = 1024;              // positions resolved into LDS at a time
  constexpr int PER = RCH / NT;          // positions per thread (2)
  static_assert(DQK == 512 || DQK == 576, "head_dim");
  static_assert(DV == 512, "head_dim_v");
  static_assert(NROPE <= NW, "rope DMA split");
  static_assert(MB * (DV * 2 + 16) <= LDS_BYTES, "output staging");
  typedef MfmaOps<T> Ops;
  typedef typename Ops::vec8 vec8;

  __shared__ __attribute__((aligned(1024))) unsigned char kv_lds[LDS_BYTES];
  __shared__ uint32_t rowid[RCH];
  __shared__ uint32_t tmask[RCH / TILE];
  __shared__ int first_neg[2];  // first -1 of the top-k scan (the slots alternate between scans)
  __shared__ int merge_word;    // split_arrive's answer to the workgroup
  // QK8: the block scales of the tiles in the two bf16 stages, [stage][block][row]
  // (36-float block stride: the four writers of a row hit four banks)
  constexpr int K8_SSTRIDE = 36;
  __shared__ float k8s[QK8 ? 2 : 1][4][K8_SSTRIDE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15;
  const int g4 = lane >> 4;                // 16-lane group
  const int srow = 16 * w + r16;           // the lane's column (staging row) in the workgroup
  const int gsel = PAIR ? (w >> 2) : 0;    // row pairs: which of the two rows
  const int hlocal = PAIR ? srow & 63 : srow;  // head within the item's m-block
  const bool has_rope = ROPE && w < NROPE; // this wave issues rope DMA instruction w
  int s2b = a.s2_base;
  int nfa = a.num_fa;
  if (a.num_fd == SAS_SCHED_DEVICE) {
    if (!dev_sched_ok(a, IMB)) {
      if (blockIdx.x == 0) nan_fill<T>(a, tid, NT);
      return;
    }
    s2b = a.metadata[SAS_CFG_OFFSET + 1];
    nfa = a.metadata[SAS_CFG_OFFSET + 2];  // rows in use (the grid is sized for num_fa)
  }
  // XCD-aware row mapping: consecutive FA rows (pieces of one item) share an XCD.
  const int per_xcd = (nfa + 7) >> 3;
  const int fa_row = (int)(blockIdx.x & 7) * per_xcd + (int)(blockIdx.x >> 3);
  if (fa_row >= nfa || (int)(blockIdx.x >> 3) >= per_xcd) return;
  const int32_t* fa = a.metadata + fa_row * SAS_FA_METADATA_SIZE;
  if (fa[0] == 0) return;
  int b = fa[1], m = fa[2];
  const int j_start = fa[3];
  const int b_end = fa[4], s_end = fa[5], j_end = fa[6];
  int slot = fa[7];
  const uint32_t kv_base = (uint32_t)(uintptr_t)kv_lds;
  // in-kernel merge: the start cursors of the rows before this one, when its
  // first item continues a split item (loaded beside the lengths)
  const bool merge_here = a.merge_sync != nullptr && a.workspace != nullptr;
  ContScan cscan = {-1, 0, 0};
  if (merge_here && j_start > 0) cscan = cont_scan_load(a, fa_row, lane);

  const char* ori_kv = (const char*)a.ori_kv;
  const char* cmp_kv = (const char*)(a.cmp_kv ? a.cmp_kv : a.ori_kv);
  const float sc = a.softmax_scale * LOG2E;
  // With at most 64 batches, every batch's lengths and query offset sit in one
  // lane each, loaded at the start beside the metadata row; otherwise they are
  // scalar loads per item.
  const bool lens_in_lanes = a.batch <= 64;
  int lane_aq = 0, lane_kv = 0, lane_qp = 0;
  if (lens_in_lanes) {
    const int lb = lane < a.batch ? lane : a.batch - 1;
    lane_aq = a.act_q_lens[lb];
    lane_kv = a.seqused_kv[lb];
    lane_qp = a.q_prefix[lb];
  }
  if (tid < 2) first_neg[tid] = INT32_MAX;
  // piece index of the first item when it continues a split item
  const int cont_k = (merge_here && j_start > 0) ? continued_piece_index(a, fa_row, b, m, cscan) : 0;
  __syncthreads();
  // sink of this lane's head (an item holds every head: one head block)
  const float sink_h = hlocal < a.num_heads ? a.sinks[hlocal] : -INFINITY;
  asm volatile("" ::"v"(lane_aq), "v"(lane_kv), "v"(lane_qp));
  int item_par = 0;  // which first_neg slot the next top-k scan uses
  bool first_item = true;
  const int hblocks = (a.num_heads + IMB - 1) / IMB;
  auto batch_lens = [&](int bb, int& aq, int& akv, int& qp) {
    const int bc = bb < a.batch ? bb : a.batch - 1;
    if (lens_in_lanes) {
      aq = __builtin_amdgcn_readlane(lane_aq, bc);
      akv = __builtin_amdgcn_readlane(lane_kv, bc);
      qp = __builtin_amdgcn_readlane(lane_qp, bc);
    } else {
      aq = ld_uniform(a.act_q_lens + bc);
      akv = ld_uniform(a.seqused_kv + bc);
      qp = ld_uniform(a.q_prefix + bc);
    }
  };
  for (;;) {
    b = __builtin_amdgcn_readfirstlane(b);
    m = __builtin_amdgcn_readfirstlane(m);
    int act_q, act_kv, qpre;
    batch_lens(b, act_q, act_kv, qpre);
    // normalise the cursor: skip batches with no (more) query rows
    while (b < a.batch && b <= b_end && m >= act_q * hblocks) {
      ++b;
      m = 0;
      batch_lens(b, act_q, act_kv, qpre);
    }
    if (b >= a.batch || b > b_end || (b == b_end && m > s_end)) break;
    const bool is_end = (b == b_end && m == s_end);
    const int s = m / hblocks;
    const int hb = m - s * hblocks;
    const int head = hb * IMB + hlocal;
    if (is_end && j_end == 0) break;

    const int tok = qpre + s;
    const bool partial = (first_item && j_start > 0) || is_end;
    ItemGeom g = item_geom(act_q, act_kv, s, a.ori_win_left, a.scenario, a.cmp_ratio, a.topk);
    // row pairs: the next row joins when neither row is a piece of a split item,
    // and g becomes the union of the two rows' lists (the window rows of row
    // s + 1 start at or after those of row s, and the two windows touch)
    bool pair = false;
    ItemGeom gA = g, gB = g;
    if constexpr (PAIR) {
      if (!partial && hblocks == 1 && a.scenario <= 2 && m + 1 < act_q &&
          !(b == b_end && m + 1 >= s_end)) {
        gB = item_geom(act_q, act_kv, s + 1, a.ori_win_left, a.scenario, a.cmp_ratio, a.topk);
        const int hiA = gA.win_lo + gA.n_win, hiB = gB.win_lo + gB.n_win;
        if (gA.n_win == 0 && gB.n_win == 0) {
          pair = true;
        } else if (gA.n_win > 0 && gB.n_win > 0 && gB.win_lo >= gA.win_lo && gB.win_lo <= hiA) {
          pair = true;
          g.n_win = (hiB > hiA ? hiB : hiA) - gA.win_lo;
        }
        if (pair) {
          g.thr = gB.thr > gA.thr ? gB.thr : gA.thr;
          g.n_cmp = gB.n_cmp > gA.n_cmp ? gB.n_cmp : gA.n_cmp;
        }
      }
    }
    // this wave's row: its token, whether its head is real, and where its own
    // positions lie in the list g (window part [wlo, whi), compressed [clo, chi))
    const int tok_w = tok + (pair ? gsel : 0);
    const bool head_ok = head < a.num_heads && (gsel == 0 || pair);
    int wlo = 0, whi = 0, clo = 0, chi = 0;
    if constexpr (PAIR) {
      if (gsel == 0 || pair) {
        const ItemGeom& gg = gsel ? gB : gA;
        wlo = gg.win_lo - g.win_lo;
        whi = wlo + gg.n_win;
        clo = g.n_win;
        chi = g.n_win + gg.n_cmp;
      }
    }
    const int L = g.n_win + g.n_cmp;
    const int nblk = (L + s2b - 1) / s2b;
    const int blo = first_item ? j_start : 0;
    int bhi = is_end ? j_end : nblk;
    if (bhi > nblk) bhi = nblk;
    const int p_lo = blo * s2b;
    const int p_hi = bhi * s2b < L ? bhi * s2b : L;
    const bool tok_ok = tok >= 0 && tok < a.total_tokens;
    const bool tok_ok_w = tok_w >= 0 && tok_w < a.total_tokens;

    // ---- online-softmax state of this lane's head (golden.py:156-160 seeds m =
    // sink, l = 1; the 1 goes to the lanes of group 0, whose row sums are added to
    // the other groups' at the end) ----
    auto seed_m = [&]() -> float {
      return partial ? -INFINITY : (head_ok ? sink_h * LOG2E : -INFINITY);
    };
    float m_run = -INFINITY;
    float l_part = (partial || g4 != 0) ? 0.0f : 1.0f;
    f32x4 acc[NDV];
#pragma unroll
    for (int d = 0; d < NDV; ++d) acc[d] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    // query fragment of the wave's 16 heads (B operand of Sᵀ = K·Qᵀ): k-step ks holds
    // dims 32 ks + 8 g4 .. + 7 of head `head`
    i16x8 qf[NKS];
    // QK8: the e4m3 query of block blk (the 16x16x128 B operand: byte p of lane l is
    // dim 128 blk + 32 (l / 16) + p of head l % 16) and its scale
    i32x8 q8[QK8 ? 4 : 1];
    float sq = 1.0f;

    // ---- scenario 3: position of the first -1 among the scanned top-k slots ----
    // (golden.py:48-53: the scan stops at the first -1). The first chunk's own
    // top-k loads double as the scan of its range; the slots outside it are
    // loaded in the same batch, and the block-table loads of the chunk are
    // issued before the barrier that publishes the result (the -1 cut is
    // applied when the row ids are packed). The two first_neg slots alternate
    // between scans, so a slot is reset without a barrier of its own.
    const int32_t* idx_row =
        a.cmp_indices ? a.cmp_indices + (size_t)(tok_ok ? tok : 0) * a.topk : nullptr;
    const bool scan3 = a.scenario == 3 && idx_row != nullptr && a.topk > 0;
    const int jmax = (scan3 && p_hi > g.n_win) ? min(p_hi - g.n_win, g.n_cmp) : 0;
    bool stop_pending = jmax > 0;
    int cmp_stop = g.n_cmp;

    for (int c0 = p_lo; c0 < p_hi; c0 += RCH) {
      const int clen = (p_hi - c0) < RCH ? (p_hi - c0) : RCH;
      const int ntile = (clen + TILE - 1) / TILE;
      // query fragment of the wave's 16 heads (B operand of Sᵀ = K·Qᵀ), loaded at
      // the first chunk right after the first tiles' DMAs are issued (below), so the
      // row-id chain before them waits for nothing but its own index loads. A head
      // past num_heads or a token out of range reads token 0's first heads: its
      // scores only reach its own softmax column and output row, never stored.
      auto load_q = [&]() {
        const bool ok = tok_ok_w && head_ok;
        const short* qrow =
            (const short*)a.q + ((size_t)(ok ? tok_w : 0) * a.num_heads + (ok ? head : 0)) * DQK;
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
          // (QK8: latent k-step 4 blk + h holds dims 128 blk + 32 g4 + 8 h, the lane's
          // quarter of e4m3 block blk)
          const int dim = (QK8 && ks < NKS_MAIN) ? 128 * (ks >> 2) + 32 * g4 + 8 * (ks & 3)
                                                 : 32 * ks + 8 * g4;
          qf[ks] = *(const i16x8*)(qrow + dim);
        }
      };
      // ---- resolve positions -> cache rows (bit 31: compressed cache) ----
      int cid[PER];
      int tab[PER];
      const int own_lo = max(c0 - g.n_win, 0);
      const int own_hi = min(max(c0 + clen - g.n_win, own_lo), jmax);
      const int n_extra = stop_pending ? jmax - (own_hi - own_lo) : 0;
      constexpr int SCAN_PER = 6;  // first scan round: PER + SCAN_PER loads per thread
      auto extra_slot = [&](int x) { return x < own_lo ? x : x + (own_hi - own_lo); };
      int sv0[SCAN_PER];
      if (scan3) {
        // all loads issued and waited for in one asm statement (gather_dwords_wait)
        const int32_t* src[PER + SCAN_PER];
        int got[PER + SCAN_PER];
#pragma unroll
        for (int e = 0; e < PER; ++e) {
          const int jj = c0 + e * NT + tid - g.n_win;
          src[e] = idx_row + (jj < 0 ? 0 : (jj < a.topk ? jj : a.topk - 1));
        }
#pragma unroll
        for (int e = 0; e < SCAN_PER; ++e) {
          const int x = e * NT + tid;  // clamped into range; unused when n_extra == 0
          const int xc = x < n_extra ? x : (n_extra > 0 ? n_extra - 1 : 0);
          src[PER + e] = idx_row + (n_extra > 0 ? extra_slot(xc) : 0);
        }
        gather_dwords_wait(got, src);
#pragma unroll
        for (int e = 0; e < SCAN_PER; ++e) sv0[e] = got[PER + e];
#pragma unroll
        for (int e = 0; e < PER; ++e) {
          const int r = e * NT + tid;
          const int pos = c0 + r;
          cid[e] = (r < clen && tok_ok && pos >= g.n_win) ? got[e] : -1;
        }
      } else {
#pragma unroll
        for (int e = 0; e < PER; ++e) {
          const int r = e * NT + tid;
          const int pos = c0 + r;
          cid[e] = (r < clen && tok_ok && pos >= g.n_win) ? pos - g.n_win : -1;
        }
      }
      if (stop_pending) {
        int mine = g.n_cmp;
#pragma unroll
        for (int e = 0; e < PER; ++e) {
          const int jj = c0 + e * NT + tid - g.n_win;
          if (jj >= 0 && jj < jmax && e * NT + tid < clen && cid[e] == -1 && jj < mine) mine = jj;
        }
#pragma unroll
        for (int e = 0; e < SCAN_PER; ++e) {
          const int x = e * NT + tid;
          if (x < n_extra && sv0[e] == -1 && extra_slot(x) < mine) mine = extra_slot(x);
        }
        for (int x0 = NT * SCAN_PER; x0 < n_extra; x0 += NT * SCAN_PER) {  // beyond the first round
          int v[SCAN_PER];
#pragma unroll
          for (int e = 0; e < SCAN_PER; ++e) {  // unconditional, clamped: all loads in flight at once
            const int x = x0 + e * NT + tid;
            v[e] = idx_row[extra_slot(x < n_extra ? x : n_extra - 1)];
          }
#pragma unroll
          for (int e = 0; e < SCAN_PER; ++e) {
            const int x = x0 + e * NT + tid;
            if (x < n_extra && v[e] == -1 && extra_slot(x) < mine) mine = extra_slot(x);
          }
        }
        if (mine < g.n_cmp) atomicMin(&first_neg[item_par], mine);
      }
      // block-table words (compiler-visible loads with in-bounds addresses)
#pragma unroll
      for (int e = 0; e < PER; ++e) {
        const int r = e * NT + tid;
        const int pos = c0 + r;
        const bool win = pos < g.n_win;
        const int key = win ? g.win_lo + pos : cid[e];
        const int bsz = win ? a.ori_block_size : a.cmp_block_size;
        const int tlen = win ? a.ori_table_len : a.cmp_table_len;
        const int32_t* tbl = win ? a.ori_block_table : a.cmp_block_table;
        const int bi = key >= 0 ? key / bsz : 0;
        const bool ok = r < clen && tok_ok && key >= 0 && bi < tlen && (win || cid[e] < g.thr);
        const int t = (tbl != nullptr) ? tbl[(size_t)b * tlen + (bi < tlen ? bi : tlen - 1)] : -1;
        tab[e] = ok ? t : -1;
      }
      // every load so far (table words) has landed, as the compiler sees it
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0) expcnt(7) lgkmcnt(15)
      if (c0 == p_lo) m_run = seed_m();
      if (stop_pending) {
        __syncthreads();  // every thread's atomicMin is in
        cmp_stop = min(first_neg[item_par], g.n_cmp);
        if (tid == 0) first_neg[item_par ^ 1] = INT32_MAX;  // the next scan's slot
        item_par ^= 1;
        stop_pending = false;
      }
#pragma unroll
      for (int e = 0; e < PER; ++e) {
        const int r = e * NT + tid;
        const int pos = c0 + r;
        uint32_t id = ROW_INVALID;
        const int phys = tab[e];
        if (r < clen && tok_ok && phys >= 0) {
          if (pos < g.n_win) {
            if (phys < a.ori_block_num)
              id = (uint32_t)(phys * a.ori_block_size + (g.win_lo + pos) % a.ori_block_size);
          } else if (phys < a.cmp_block_num && (!scan3 || pos - g.n_win < cmp_stop)) {
            id = (uint32_t)(phys * a.cmp_block_size + cid[e] % a.cmp_block_size) | 0x80000000u;
          }
        }
        rowid[r] = id;  // masked rows are read from the zero row
        const unsigned long long bal = __ballot(id != ROW_INVALID);
        if (lane == 0) {
          tmask[(r - lane) / TILE] = (uint32_t)bal;
          tmask[(r - lane) / TILE + 1] = (uint32_t)(bal >> 32);
        }
      }
      __syncthreads();

      // ---- DMA issue for one tile into one ring stage ----
      // main part: wave w fills rows w + 8 j (j < 4), one 1 KB row per instruction;
      // rope part: instruction i (wave i < 4) fills slot rows 8 i .. 8 i + 7
      auto row_ptr = [&](uint32_t id) -> const char* {
        const char* base = (id & 0x80000000u) ? cmp_kv : ori_kv;
        const char* p = base + (size_t)(id & 0x7FFFFFFFu) * ROWB;
        return id == ROW_INVALID ? (const char*)g_zero_row : p;
      };
      auto lane_row = [&](uint64_t ptrs, int j) -> const char* {
        const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)ptrs, j);
        const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(ptrs >> 32), j);
        return (const char*)(uintptr_t)(((uint64_t)hi << 32) | lo);
      };
      struct DmaAddrs {
        uint64_t main;     // lane j < RPW: this wave's j-th main row
        const char* rope;  // per lane: its 16-byte rope piece (waves w < NROPE)
        uint32_t sbase;
      };
      // Addresses of the DMAs of tile t. Past the chunk's last tile the
      // instructions read the zero row into the stage they would fill, which
      // nothing reads before the chunk ends (keeps the vmcnt accounting uniform).
      auto next_addrs = [&](int tile) -> DmaAddrs {
        DmaAddrs d;
        const bool real = tile < ntile;
        d.sbase = kv_base + (uint32_t)((tile % NSTG) * STAGE_BYTES);
        const int t0 = real ? tile : 0;
        d.main = (uint64_t)(uintptr_t)row_ptr(rowid[t0 * TILE + w + NW * (lane < RPW ? lane : 0)]);
        d.rope = (const char*)g_zero_row;
        if constexpr (ROPE) {
          const int p = 8 * (w < NROPE ? w : 0) + (lane >> 3);  // slot row of this lane's chunk
          const int c = (lane & 7) ^ ((p >> 1) & 7);            // the chunk slot lane & 7 holds
          d.rope = row_ptr(rowid[t0 * TILE + wide_perm(p)]) + 1024 + c * 16;
        }
        if (!real) {
          d.main = (uint64_t)(uintptr_t)g_zero_row;
          d.rope = (const char*)g_zero_row;
        }
        return d;
      };
      auto dma_one = [&](const DmaAddrs& d, int j) {
        if (j < RPW) {
          dma16_sbase(lane_row(d.main, j), (uint32_t)lane * 16u, d.sbase + wide_row_base(w + NW * j));
        } else if constexpr (ROPE) {
          if (has_rope) dma16_vaddr(d.rope, d.sbase + WMAIN + w * 1024);
        }
      };
      constexpr int DMA_MAX = RPW + (ROPE ? 1 : 0);
      auto issue = [&](const DmaAddrs& d) {
#pragma unroll
        for (int j = 0; j < DMA_MAX; ++j) dma_one(d, j);
      };
      // this wave's DMAs of all but the newest one / two tiles have landed
      auto wait_all_but = [&](auto n_tiles) {
        constexpr int N = decltype(n_tiles)::value;
        if constexpr (FP8) wait_vmcnt<N * RAW_DMA>();
        else if (has_rope) wait_vmcnt<N * (RPW + 1)>();
        else wait_vmcnt<N * RPW>();
      };
      typedef const unsigned char SAS_LDS* lds_p;
      auto stage_of = [&](int tile) -> lds_p {
        return (lds_p)(kv_base + (uint32_t)((tile % NSTG) * STAGE_BYTES));
      };
      // ---- fp8 rows: raw DMA and dequantization ----
      // Raw tile t goes to raw stage t % NRAW as 32 rows of 656 bytes: this wave's
      // instruction j copies row w + 8 j whole, lane i < 41 its 16-byte piece i,
      // from the row's address (lane j of raw_addrs, read into scalars) plus 16 i.
      // Past the chunk's last tile the rows are read from the zero row.
      auto raw_base = [&](int tile) -> uint32_t {
        constexpr int NR = NRAW > 0 ? NRAW : 1;  // (native rows have no raw ring)
        return kv_base + (uint32_t)(NSTG * STAGE_BYTES + (tile % NR) * RAW_STAGE);
      };
      auto raw_addrs = [&](int tile) -> uint64_t {
        const bool real = tile < ntile;
        const int l = lane_id_here();
        const uint32_t id = rowid[(real ? tile : 0) * TILE + w + NW * (l < RAW_DMA ? l : 0)];
        return (uint64_t)(uintptr_t)(real ? row_ptr(id) : (const char*)g_zero_row);
      };
      auto raw_issue = [&](uint64_t ra, uint32_t voff, int tile, int j) {
        dma16_sbase_lanes(lane_row(ra, j), voff,
                          raw_base(tile) + (uint32_t)((w + NW * j) * SAS_FP8_ROW_BYTES),
                          RAW_LANES);
      };
      // Raw tile t (landed and published by a barrier) into bf16 stage t % 2 as
      // bf16(fp32(e4m3) * scale): wave w converts rows w + 8 k (k < 4), lane l dims
      // 8 l .. 8 l + 7 (consecutive lanes read consecutive 8-byte pieces and write
      // consecutive 16-byte chunks: no bank conflicts); the first 256 threads copy
      // the 32 x 8 rope chunks.
      auto convert_row = [&](int tile, int k) {
        typedef int i32x2 __attribute__((ext_vector_type(2)));
        const int l = lane_id_here();  // (recomputed here: no offset stays live across the loop)
        const uint32_t st = kv_base + (uint32_t)((tile % 2) * STAGE_BYTES);
        const int r = w + NW * k;
        const lds_p raw = (lds_p)(raw_base(tile) + (uint32_t)(r * SAS_FP8_ROW_BYTES));
        const i32x2 v = *(const i32x2 SAS_LDS*)(raw + 8 * l);
        const float sc8 = *(const float SAS_LDS*)(raw + LATENT_BYTES + 4 * (l >> 4));
        *(i16x8 SAS_LDS*)(st + (uint32_t)(wide_row_base(r) + 16 * l)) =
            fp8x8_dequant_bf16(make_uint2((uint32_t)v[0], (uint32_t)v[1]), sc8);
        if constexpr (QK8) {
          if ((l & 15) == 0) k8s[tile & 1][l >> 4][r] = sc8;  // block l / 16's scale of row r
        }
      };
      auto convert_rope = [&](int tile) {
        const int x = 64 * w + lane_id_here();
        if (x < TILE * 8) {
          const int r = x >> 3, c = x & 7;
          const i16x8 rp = *(const i16x8 SAS_LDS*)(raw_base(tile) + (uint32_t)(r *
                                                                   SAS_FP8_ROW_BYTES + LATENT_BYTES +
                                                                   16 + 16 * c));
          *(i16x8 SAS_LDS*)(kv_base + (uint32_t)((tile % 2) * STAGE_BYTES + WMAIN +
                                                  16 * wide_rope_slot(wide_perm(r), c))) = rp;
        }
      };
      auto convert = [&](int tile) {
#pragma unroll
        for (int k = 0; k < TILE / NW; ++k) convert_row(tile, k);
        if constexpr (!QK8) convert_rope(tile);
      };

      auto mma16 = [&](i16x8 x, i16x8 y, f32x4 c) -> f32x4 {
        return __is_same(T, __bf16)
                   ? __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(vec8, x),
                                                             __builtin_bit_cast(vec8, y), c, 0, 0, 0)
                   : __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(vec8, x),
                                                            __builtin_bit_cast(vec8, y), c, 0, 0, 0);
      };

      // ---- Q·Kᵀ of one tile: two row blocks (independent accumulators,
      // alternating), K operands KPF MFMAs ahead ----
      auto qk_tile = [&](lds_p sb, f32x4& s0, f32x4& s1, auto&& hook) {
        constexpr int NQK = 2 * NKS;
        constexpr int KPF = SAS_WKPF;
        const lds_p kb_main = sb + wide_k_main(lane_id_here());
        lds_p kb_rope0 = sb, kb_rope1 = sb;
        auto kaddr = [&](int i) -> const i16x8 SAS_LDS* {
          const int ks = i >> 1, rb = i & 1;
          if (ks >= NKS_MAIN && rb == 0) {  // (the rope offsets, first needed here)
            const int l = lane_id_here();
            if (ks == NKS_MAIN) kb_rope0 = sb + wide_rope0(l);
            else kb_rope1 = sb + wide_rope1(l);
          }
          return (const i16x8 SAS_LDS*)(ks < NKS_MAIN ? kb_main + 64 * ks + rb * (16 * WROW)
                                                      : (ks == NKS_MAIN ? kb_rope0 : kb_rope1) +
                                                            rb * (16 * 128));
        };
        i16x8 kb[KPF];
#pragma unroll
        for (int i = 0; i < KPF; ++i) kb[i] = *kaddr(i);
        s0 = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        s1 = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < NQK; ++i) {
          const i16x8 op = kb[i % KPF];
          if (i + KPF < NQK) kb[i % KPF] = *kaddr(i + KPF);
          if (i & 1) s1 = mma16(op, qf[i >> 1], s1);
          else s0 = mma16(op, qf[i >> 1], s0);
          hook(i);
          __builtin_amdgcn_sched_barrier(0);
        }
      };

      // ---- QK8: Q·Kᵀ of one tile from its raw rows. Lane l's A operands: row
      // 16 rb + l % 16, bytes 128 blk + 32 (l / 16) .. + 31 of its e4m3 dims (block
      // blk), and bf16 rope dims 512 + 32 kr + 8 (l / 16) .. + 7. Per 16-row block rb
      // the scores are sq * sum_blk sk[blk][row] * d_blk + d_rope: the block dot
      // products d_blk in fp32 (v_mfma_f32_16x16x128_f8f6f4), folded in block order
      // with fused multiply-adds (block 0 a product), the rope part on two bf16
      // k-steps. The MFMAs alternate between the two row blocks; a block's scale is
      // folded in after the next MFMA is issued. ----
      auto qk8_tile = [&](int tile, f32x4& s0, f32x4& s1, auto&& hook) {
        const int l = lane_id_here();
        const lds_p raw = (lds_p)(raw_base(tile) +
                                  (uint32_t)((l & 15) * SAS_FP8_ROW_BYTES + 32 * (l >> 4)));
        auto k8op = [&](int j) -> i32x8 {  // MFMA j: row block j & 1, e4m3 block j >> 1
          const lds_p p = raw + (uint32_t)((j & 1) * 16 * SAS_FP8_ROW_BYTES + 128 * (j >> 1));
          const i32x4 lo = *(const i32x4 SAS_LDS*)p;
          const i32x4 hi = *(const i32x4 SAS_LDS*)(p + 16);
          return (i32x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        };
        auto kscale = [&](int j) -> f32x4 {  // scales of rows 16 rb + 4 (l / 16) + i
          return *(const f32x4 SAS_LDS*)&k8s[tile & 1][j >> 1][16 * (j & 1) + 4 * (l >> 4)];
        };
        auto mma8 = [&](i32x8 x, i32x8 y) -> f32x4 {
          // e4m3 x e4m3 (format selectors 0), no block scaling
          return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              x, y, (f32x4){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0, 0, 0, 0);
        };
        f32x4 s8[2];
        auto fold = [&](int j, f32x4 d, f32x4 sk) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            s8[j & 1][i] = (j < 2) ? d[i] * sk[i] : __builtin_fmaf(d[i], sk[i], s8[j & 1][i]);
          // (here, not sunk to the end: a product kept for later holds its MFMA's
          // four result registers across the tile)
          asm volatile("" : "+v"(s8[j & 1]));
        };
        constexpr int N8 = 8;
        i32x8 kb[2];
        kb[0] = k8op(0);
        kb[1] = k8op(1);
        // (a block's product is folded two MFMAs after its own, when it has landed;
        // its scales are read when it is issued)
        f32x4 dq[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
        f32x4 skq[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < N8; ++j) {
          const i32x8 op = kb[j & 1];
          if (j + 2 < N8) kb[j & 1] = k8op(j + 2);
          const f32x4 d = mma8(op, q8[j >> 1]);
          if (j > 1) fold(j - 2, dq[j & 1], skq[j & 1]);
          dq[j & 1] = d;
          skq[j & 1] = kscale(j);
          hook(j);
          __builtin_amdgcn_sched_barrier(0);
        }
        // rope: k-steps 16 and 17 of each row block, from the raw rows' bf16 dims
        f32x4 dr[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
        // (row base + 32 (l / 16) + 528 - 16 (l / 16): the rope's chunk l / 16)
        const lds_p rp = raw + (uint32_t)(LATENT_BYTES + 16 - 16 * (l >> 4));
#pragma unroll
        for (int kr = 0; kr < 2; ++kr)
#pragma unroll
          for (int rb = 0; rb < 2; ++rb) {
            const i16x8 ko =
                *(const i16x8 SAS_LDS*)(rp + (uint32_t)(rb * 16 * SAS_FP8_ROW_BYTES + 64 * kr));
            dr[rb] = mma16(ko, qf[NKS_MAIN + kr], dr[rb]);
            if (kr == 0) fold(N8 - 2 + rb, dq[rb], skq[rb]);
            hook(N8 + 2 * kr + rb);
            __builtin_amdgcn_sched_barrier(0);
          }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          s0[i] = __builtin_fmaf(s8[0][i], sq, dr[0][i]);
          s1[i] = __builtin_fmaf(s8[1][i], sq, dr[1][i]);
        }
      };

      // ---- online softmax (exp2 domain) on the lane's 8 rows of its head:
      // returns the tile's Pᵀ operand and the head's rescale factor ----
      auto softmax_tile = [&](int t, f32x4 s0, f32x4 s1, float& alpha) -> i16x8 {
        // (masking only on tiles with invalid rows: tile tails, -1 / out-of-range
        // ids; the empty asm keeps this a branch, so full tiles skip the selects)
        uint32_t tm = tmask[t];
        if constexpr (PAIR) {
          // positions of the tile outside this wave's row's own list
          auto span = [](int lo, int hi, int p0) -> uint32_t {
            const int x = lo - p0 > 0 ? lo - p0 : 0, y = hi - p0 < TILE ? hi - p0 : TILE;
            return y > x ? (uint32_t)(((1ull << y) - 1) & ~((1ull << x) - 1)) : 0u;
          };
          const int p0 = c0 + TILE * t;
          tm &= span(wlo, whi, p0) | span(clo, chi, p0);
        }
        if (__builtin_amdgcn_readfirstlane(tm) != 0xFFFFFFFFu) {
          asm volatile("");
          const uint32_t v0 = tm >> (4 * g4), v1 = tm >> (16 + 4 * g4);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            s0[i] = ((v0 >> i) & 1u) ? s0[i] : -INFINITY;
            s1[i] = ((v1 >> i) & 1u) ? s1[i] : -INFINITY;
          }
        }
        // max of the raw scores, then scaled: rounding is monotonic, so this is
        // the max of the scaled scores
        float mloc = fmaxf(fmaxf(fmaxf(s0[0], s0[1]), fmaxf(s0[2], s0[3])),
                           fmaxf(fmaxf(s1[0], s1[1]), fmaxf(s1[2], s1[3])));
        {
          const auto r1 = __builtin_amdgcn_permlane16_swap(__float_as_uint(mloc),
                                                           __float_as_uint(mloc), false, false);
          mloc = fmaxf(__uint_as_float(r1[0]), __uint_as_float(r1[1]));
        }
        mloc = wave_max_pair(mloc) * sc;
        const bool grow = mloc > m_run;
        const float m_new = grow ? mloc : m_run;
        alpha = grow ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;  // -inf -> 0
        m_run = m_new;
        l_part *= alpha;
        // a head with no key and no sink yet (m_run = -inf) has every score -inf:
        // subtracting 0 instead keeps its P at exactly 0
        const float m_sub = m_run == -INFINITY ? 0.0f : m_run;
        i16x8 pk;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[i], sc, -m_sub));
          l_part += p;
          pk[i] = Ops::from_f32(p);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[i], sc, -m_sub));
          l_part += p;
          pk[4 + i] = Ops::from_f32(p);
        }
        return pk;
      };

      // ---- rescale (skipped when no head of the wave moved its maximum), then
      // P·V with Vᵀ operands VPF MFMAs ahead and the DMA instructions of `dd`
      // (the tile three ahead) between the MFMAs ----
      auto pv_tile = [&](lds_p sb, i16x8 pk, float alpha, const DmaAddrs& dd, int t) {
        if (__ballot(alpha != 1.0f) != 0) {
#pragma unroll
          for (int d = 0; d < NDV; ++d)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[d][j] *= alpha;
        }
        // (fp8: two, making room for the dequantization; row pairs: two, measured
        // faster there, while 128-head items keep three)
        constexpr int VPF = (FP8 || PAIR) ? 2 : SAS_WVPF;
        typedef i16x4 SAS_LDS* lds4;
        const lds_p vbase = sb + wide_v(lane_id_here());
        auto vop = [&](int d) -> i16x8 {
          const i16x4 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds4)(vbase + 32 * d));
          const i16x4 x1 =
              __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds4)(vbase + 16 * WROW + 32 * d));
          return (i16x8){x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
        };
        i16x8 vb[VPF];
#pragma unroll
        for (int i = 0; i < VPF; ++i) vb[i] = vop(i);
        const uint32_t voff = FP8 ? 16u * (uint32_t)lane_id_here() : 0u;
#pragma unroll
        for (int d = 0; d < NDV; ++d) {
          const i16x8 op = vb[d % VPF];
          if (d + VPF < NDV) vb[d % VPF] = vop(d + VPF);
          acc[d] = mma16(op, pk, acc[d]);
          if constexpr (FP8) {
            // the raw DMAs of tile t + 3 (into the raw stage tile t held; dd.main
            // holds their row addresses)
#pragma unroll
            for (int j = 0; j < RAW_DMA; ++j)
              if (d == 3 + 8 * j) raw_issue(dd.main, voff, t + 3, j);
          } else {
#pragma unroll
            for (int j = 0; j < DMA_MAX; ++j)
              if (d == 3 + 6 * j) dma_one(dd, j);
          }
        }
      };

      // ---- prologue: tiles 0, 1, 2 in flight, then the query fragment ----
      if constexpr (FP8) {
        const uint32_t voff = 16u * (uint32_t)lane;
#pragma unroll
        for (int tt = 0; tt < 3; ++tt) {
          const uint64_t ra = raw_addrs(tt);
#pragma unroll
          for (int j = 0; j < RAW_DMA; ++j) raw_issue(ra, voff, tt, j);
        }
      } else {
        issue(next_addrs(0));
        issue(next_addrs(1));
        issue(next_addrs(2));
      }
      if (c0 == p_lo) {
        load_q();
        // (the compiler's wait for the query loads goes here, before the tile loop;
        // it also covers the DMAs issued before them)
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) asm volatile("" ::"v"(qf[ks]));
        if constexpr (QK8) quantize_q(qf, q8, sq);
      }
      if constexpr (FP8) {
        wait_all_but(std::integral_constant<int, 2>{});  // this wave's raw DMAs of tile 0
        __syncthreads();                                  // every wave's
        convert(0);
      }

      // ---- tile loop: before barrier t every wave has waited for its DMAs of tile
      // t (tiles t + 1 and t + 2 may be in flight); after it every wave is done with
      // tile t - 1, whose stage takes the DMAs of tile t + 3, issued between this
      // tile's P·V MFMAs: three tiles in flight under the compute of one. fp8 rows:
      // before barrier t every wave has waited for its raw DMAs of tile t + 1
      // (t + 2 may be in flight), which tile t dequantizes into the bf16 stage of
      // t - 1 while tile t (dequantized during t - 1) is computed, and the raw DMAs
      // of t + 3 go to the raw stage of t ----
      for (int t = 0; t < ntile; ++t) {
        const lds_p sb = stage_of(t);
        if constexpr (FP8) wait_all_but(std::integral_constant<int, 1>{});
        else wait_all_but(std::integral_constant<int, 2>{});  // this wave's share of tile t
        __syncthreads();                                       // barrier t
        f32x4 s0, s1;
        // Q·Kᵀ and the softmax at wave priority 1, P·V at 0: of the SIMD's two
        // waves, one still in the first half of its tile wins issue over one
        // already in P·V, so the slower wave reaches the next barrier sooner
        __builtin_amdgcn_s_setprio(1);
        // (fp8 rows: tile t + 1 is dequantized into the bf16 stage tile t - 1 held,
        // a row at a time between the Q·Kᵀ MFMAs, whose matrix-core time the
        // conversion's VALU work runs beside)
        auto conv_hook = [&](int i) {
          if constexpr (QK8) {
            if (t + 1 < ntile) {
#pragma unroll
              for (int k = 0; k < TILE / NW; ++k)
                if (i == 1 + 3 * k) convert_row(t + 1, k);
            }
          }
        };
        if constexpr (QK8) qk8_tile(t, s0, s1, conv_hook);
        else qk_tile(sb, s0, s1, [&](int i) {
          if constexpr (FP8) {
            if (t + 1 < ntile) {
#pragma unroll
              for (int k = 0; k < TILE / NW; ++k)
                if (i == 4 + 8 * k) convert_row(t + 1, k);
              if (i == 33) convert_rope(t + 1);
            }
          }
        });
        float alpha;
        const i16x8 pk = softmax_tile(t, s0, s1, alpha);
        __builtin_amdgcn_s_setprio(0);
        if constexpr (FP8) {
          DmaAddrs dd;
          dd.main = raw_addrs(t + 3);
          pv_tile(sb, pk, alpha, dd, t);
        } else {
          const DmaAddrs dd = next_addrs(t + 3);
          pv_tile(sb, pk, alpha, dd, t);
        }
      }
      wait_vmcnt<0>();  // the last (zero-row) DMAs have landed ...
      __syncthreads();  // ... for every wave, before LDS is reused
    }

    if (p_lo >= p_hi) m_run = seed_m();  // an item with no rows: the sink alone
    // ---- row sum of the lane's head over its four lanes (identical in all four) ----
    float l_run;
    {
      const auto r1 = __builtin_amdgcn_permlane16_swap(__float_as_uint(l_part),
                                                       __float_as_uint(l_part), false, false);
      l_run = wave_sum_pair(__uint_as_float(r1[0]) + __uint_as_float(r1[1]));
    }

    // ---- epilogue: the item's rows go out through LDS (the ring is free), so
    // every store instruction writes whole rows ----
    __syncthreads();  // (an item without rows: the previous item's staged rows are read out)
    {
      unsigned char* stg = kv_lds;
      const int nh = min(IMB, a.num_heads - hb * IMB);  // heads of this item
      constexpr int SROW = DV * 2 + 16;  // staging row stride (bytes; 16-byte aligned rows)
      constexpr int CPR = DV * 2 / 16;   // 16-byte chunks per row
      int tid_e = tid, hl_e = srow, dv_e = 4 * g4;
      asm volatile("" : "+v"(tid_e), "+v"(hl_e), "+v"(dv_e));
      if (!partial) {
        const float inv = 1.0f / l_run;
#pragma unroll
        for (int d = 0; d < NDV; ++d) {
          const i16x4 v = {Ops::from_f32(acc[d][0] * inv), Ops::from_f32(acc[d][1] * inv),
                           Ops::from_f32(acc[d][2] * inv), Ops::from_f32(acc[d][3] * inv)};
          *(i16x4*)(stg + hl_e * SROW + (16 * d + dv_e) * 2) = v;
        }
        __syncthreads();
        if (tok_ok) {
          if constexpr (PAIR) {
            // staging row h: row s + h / 64, head h % 64
            char* obase = (char*)((T*)a.out + (size_t)tok * a.num_heads * DV);
            for (int c = tid_e; c < (pair ? 2 : 1) * 64 * CPR; c += NT) {
              const int h = c / CPR, c16 = c - h * CPR;
              if ((h & 63) < a.num_heads && tok + (h >> 6) < a.total_tokens)
                *(i16x8*)(obase + ((size_t)(h >> 6) * a.num_heads + (h & 63)) * DV * 2 + c16 * 16) =
                    *(const i16x8*)(stg + h * SROW + c16 * 16);
            }
          } else {
            char* obase = (char*)((T*)a.out + ((size_t)tok * a.num_heads + hb * MB) * DV);
            for (int c = tid_e; c < nh * CPR; c += NT) {
              const int h = c / CPR, c16 = c - h * CPR;
              *(i16x8*)(obase + (size_t)h * DV * 2 + c16 * 16) = *(const i16x8*)(stg + h * SROW + c16 * 16);
            }
          }
          if (g4 == 0 && head_ok && tok_ok_w)
            a.lse[(size_t)tok_w * a.num_heads + head] = (m_run + __log2f(l_run)) * LN2;
        }
      } else if (slot >= 0 && slot < a.num_partial_slots && a.workspace) {
        // (row pairs: a piece of a split item is never paired, so its heads are
        // waves 0..3's, staging rows 0 .. 63)
        // fp16 partials (acc / l, scaled): the head's whole row sits in its four
        // lanes, whose max picks the scale
        const bool empty = !(l_run > 0.0f);
        const float inv = empty ? 0.0f : 1.0f / l_run;
        float amax = 0.0f;
#pragma unroll
        for (int d = 0; d < NDV; ++d)
#pragma unroll
          for (int j = 0; j < 4; ++j) amax = fmaxf(amax, fabsf(acc[d][j]));
        {
          const auto r1 = __builtin_amdgcn_permlane16_swap(__float_as_uint(amax),
                                                           __float_as_uint(amax), false, false);
          amax = fmaxf(__uint_as_float(r1[0]), __uint_as_float(r1[1]));
        }
        // max |acc| times inv is max |acc * inv| (rounding is monotonic)
        amax = wave_max_pair(amax) * inv;
        const PartialScale ps = partial_scale(amax);
#pragma unroll
        for (int d = 0; d < NDV; ++d) {
          i16x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            v[e] = __builtin_bit_cast(short, (_Float16)(acc[d][e] * inv * ps.scale));
          *(i16x4*)(stg + hl_e * SROW + (16 * d + dv_e) * 2) = v;
        }
        __syncthreads();
        const float lse_piece = empty ? -INFINITY : (m_run + __log2f(l_run)) * LN2;
        if (merge_here) {
          // read by another workgroup in this launch: agent-coherent stores
          const __amdgpu_buffer_rsrc_t rs = partial_rsrc(a, IMB, DV);
          const uint32_t base = (uint32_t)slot * IMB * DV * 2;
          for (int c = tid_e; c < nh * CPR; c += NT) {
            const int h = c / CPR, c16 = c - h * CPR;
            partial_store16(rs, base + (uint32_t)(h * DV * 2 + c16 * 16),
                            *(const i32x4*)(stg + h * SROW + c16 * 16));
          }
          if (g4 == 0 && head_ok) {
            const uint32_t lo = (uint32_t)a.num_partial_slots * IMB * DV * 2;
            partial_store4(rs, lo + ((uint32_t)slot * IMB + hl_e) * 4, lse_piece);
            partial_store4(rs, lo + ((uint32_t)(a.num_partial_slots + slot) * IMB + hl_e) * 4,
                           ps.inv);
          }
        } else {
          char* wbase = (char*)a.workspace + (size_t)slot * IMB * DV * 2;
          for (int c = tid_e; c < nh * CPR; c += NT) {
            const int h = c / CPR, c16 = c - h * CPR;
            *(i16x8*)(wbase + (size_t)h * DV * 2 + c16 * 16) =
                *(const i16x8*)(stg + h * SROW + c16 * 16);
          }
          if (g4 == 0 && head_ok) {
            float* wl = partial_lse(a, IMB, DV);
            wl[(size_t)slot * IMB + hl_e] = lse_piece;
            wl[(size_t)(a.num_partial_slots + slot) * IMB + hl_e] = ps.inv;
          }
        }
      }
    }
    if (partial && merge_here) {
      // the piece that completes the item merges it (bit-identical to merge_kernel)
      const int slot0 = (first_item && j_start > 0) ? slot - cont_k : slot;
      if (slot0 >= 0 && slot < a.num_partial_slots && slot0 < SAS_MERGE_SYNC_WORDS) {
        const int npc = split_arrive(a, slot0, slot, bhi - blo, bhi == nblk, nblk, &merge_word);
        if (npc > 0) merge_item_here<DV, T, IMB, NW>(a, tok, hb, slot0, npc);
      }
    }
    if (partial) ++slot;
    if (is_end) break;
    first_item = false;
    if (pair) ++m;
    ++m;
  }
}

}  // namespace sas
