// Sparse shared-KV attention decode for MI355X (gfx950 / CDNA4).
//
// Replaces the reference's fused TileLang kernels (kernel.py:_build_swa /
// _build_cfa / _build_scfa and sparse_flash_mla_kernel.py:_build_swa/_hca/_csa)
// with one metadata-driven HIP kernel plus a split-KV merge kernel.
//
// Work decomposition
//   One workgroup per FA metadata row; it walks its items (query rows) and,
//   inside each, its blocks of the attended list [window rows ++ compressed
//   positions]. All query heads of a token share every gathered KV row
//   (shared KV, N2 = 1): a 32-row tile is loaded once into LDS and read by
//   every wave, as K for Q·Kᵀ and (first head_dim_v columns) as V for P·V.
//
// Waves (NHG head groups of 32 heads x 4 dims quarters = 4*NHG waves, two per
// SIMD for the 64-head items of H > 32; details at attn_kernel):
//   Q·Kᵀ: each wave computes a partial Sᵀ[32 rows x 32 heads] over its quarter
//         of d_qk with v_mfma_f32_32x32x16 (A = K rows from LDS, B = Qᵀ held in
//         VGPRs); the four partials of a head group are summed through LDS.
//   softmax: exp2 domain on 4 rows x 1 head per lane; P shared through LDS;
//         lazy rescaling (the O rescale only runs when some head's max grows
//         by more than 2^8).
//   P·V:  each wave accumulates Oᵀ[its dv quarter x 32 heads] (A = Vᵀ via
//         ds_read_b64_tr_b16 from the row-major tile, B = Pᵀ from LDS).
//   The tile loop is software-pipelined: Q·Kᵀ of the next tile is issued
//   before the softmax of this one, so the two overlap.
//
// Gather: global_load_lds_dwordx4 (16 B per lane straight into LDS, no VGPR
//   staging) into a 3-stage ring; rows of a tile are rotated by 16-byte
//   chunks so both the Kᵀ reads (b128) and the transposed V reads (tr_b16)
//   are bank-conflict free. fp8 cache rows are loaded into VGPRs instead and
//   dequantized into the same bf16 layout.
//
// Numerics follow golden.py:156-200: fp32 scores, P rounded to the input
// dtype before P·V while the running sum uses fp32 P, out = acc / l rounded
// RNE, lse = m + ln(l). Split pieces emit (acc / l, lse) without the sink;
// the merge adds the sink once.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <string>

#include "../../include/sas_mi355x.h"
#include "sas_items.h"

namespace sas {

static thread_local std::string g_last_error;
void set_error(const std::string& msg) { g_last_error = msg; }

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#define SAS_LDS __attribute__((address_space(3)))
#define SAS_GLOBAL __attribute__((address_space(1)))

constexpr int TILE = 32;        // KV rows per pipeline stage
constexpr int NSTAGE = 3;       // LDS ring depth
constexpr int RCHUNK = 1024;    // positions resolved into LDS at a time
constexpr uint32_t ROW_INVALID = 0xFFFFFFFFu;
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;
constexpr float RESCALE_TAU = 8.0f;  // lazy-rescale threshold (log2 units)

template <typename T> struct MfmaOps;
template <> struct MfmaOps<__bf16> {
  typedef bf16x8 vec8;
  static __device__ inline f32x16 mma(i16x8 a, i16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ inline short from_f32(float x) {
    return __builtin_bit_cast(short, (__bf16)x);
  }
};
template <> struct MfmaOps<_Float16> {
  typedef f16x8 vec8;
  static __device__ inline f32x16 mma(i16x8 a, i16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ inline short from_f32(float x) {
    return __builtin_bit_cast(short, (_Float16)x);
  }
};

// LDS stage layout (one 32-row tile).
//   main part, dims 0..511: row r occupies MAIN_SLOTS = 68 sixteen-byte slots
//     (1088 B); its chunk c (dims 8c..8c+7) sits in slot c + rot(r) with
//     rot(r) = (r >> 2) & 3. One DMA instruction (64 lanes x 16 B) fills one
//     row, and every read address is one per-lane base plus an immediate.
//   rope part, dims 512..575 (head_dim 576): 8 slots per row after the main
//     part; chunk 64 + c' of row r sits in slot 8 r + ((c' + (r >> 1)) & 7), so
//     one DMA instruction fills 8 rows.
// With 64 banks x 4 B (16 sixteen-byte bank groups):
//   * Kᵀ reads (ds_read_b128, 16 lanes = rows r..r+15 at one chunk) hit bank
//     groups (4 r + rot(r) + c) mod 16 (main) or (8 r + ((c' + r/2) & 7)) mod 16
//     (rope), all distinct;
//   * Vᵀ reads (ds_read_b64_tr_b16, 32 lanes = 4 consecutive rows x 4 chunks)
//     start at 4 (r % 4) + rot(r) = {0, 4, 8, 12} + const, four disjoint spans.
constexpr int MAIN_SLOTS = 68;
constexpr int MAIN_ROW_BYTES = MAIN_SLOTS * 16;
constexpr int MAIN_BYTES = TILE * MAIN_ROW_BYTES;      // 34816
constexpr int ROPE_BYTES = TILE * 8 * 16;              // 4096
__device__ __host__ inline int row_rot(int r) { return (r >> 2) & 3; }
__device__ __host__ inline int main_row_base(int r) { return r * MAIN_ROW_BYTES + row_rot(r) * 16; }
__device__ __host__ inline int rope_slot(int r, int cr) { return 8 * r + ((cr + (r >> 1)) & 7); }

// Combine lane l with lane l ^ 32 in registers (v_permlane32_swap): both
// halves end up with the identical result.
__device__ inline float wave_max_pair(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float wave_sum_pair(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);  // lower half + upper half
}

// Direct-to-LDS 16-byte loads: lane's data lands at M0 + lane * 16.
// Issued through inline asm so the compiler does not serialise them against
// unrelated LDS reads; completion is tracked by hand with s_waitcnt vmcnt.
// An LDS DMA that reads M0 needs one wait state after the SALU write of M0
// (the compiler's hazard pass cannot see inside the asm), hence the s_nop.
// Rows are fetched with the streaming cache policy (sc0 nt): each row is read
// once per workgroup (the second 64-head m-block of a token reads it on the
// same XCD shortly after), and the non-temporal fills shortened the stalls of
// the DMA issue on every tile (measured about 3.5 us of 66 at B = 64, H = 128).
__device__ inline void dma16_sbase(const void* sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1 sc0 nt\n\t" ::"v"(voff),
      "s"(sbase), "s"(lds_base)
      : "memory");
}
__device__ inline void dma16_vaddr(const void* gptr, uint32_t lds_base) {
  asm volatile(
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, off sc0 nt\n\t" ::"v"(gptr),
      "s"(lds_base)
      : "memory");
}

// A read-only kernel input at a wave-uniform address, as a scalar load (through
// the constant address space: the compiler cannot prove on its own that the
// kernel's stores leave these arrays alone, and would use a vector load).
__device__ inline int32_t ld_uniform(const int32_t* p) {
  return *(const __attribute__((address_space(4))) int32_t*)p;
}

// Materialise a value at this point of the program: the empty asm (ordered
// with the barriers and the DMA asm) consumes it, so its computation cannot be
// sunk past the next barrier towards its use.
__device__ inline void pin_u64(uint64_t& v) {
  uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
  asm volatile("" : "+v"(lo), "+v"(hi));
  v = ((uint64_t)hi << 32) | lo;
}

template <int N>
__device__ inline void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// ds_read_b64_tr_b16 with an immediate offset (the builtin does not fold
// offsets, which costs one address VGPR per read). The result is not tracked
// by the compiler's lgkmcnt bookkeeping: consume it only after lds_wait_pv.
template <int OFF>
__device__ inline i16x4 ds_read_tr16(uint32_t addr) {
  i16x4 v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF) : "memory");
  return v;
}

template <int OFF>
__device__ inline i16x8 ds_read_b128_asm(uint32_t addr) {
  i16x8 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF) : "memory");
  return v;
}
__device__ inline uint32_t ds_read_b32_asm(uint32_t addr) {
  uint32_t v;
  asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(addr) : "memory");
  return v;
}
__device__ inline uint64_t ds_read_b64_asm(uint32_t addr) {
  uint64_t v;
  asm volatile("ds_read_b64 %0, %1" : "=v"(v) : "v"(addr) : "memory");
  return v;
}

// Wait for every LDS operation of this wave; all registers written by the
// untracked asm reads pass through the asm, so no consumer (and no copy) of
// them can be placed above the wait.
__device__ inline void lds_wait_pv(uint64_t& votes, i16x8 (&p)[2], i16x4 (&g0)[8],
                                   i16x4 (&g1)[8]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(votes), "+v"(p[0]), "+v"(p[1]), "+v"(g0[0]), "+v"(g0[1]), "+v"(g0[2]),
                 "+v"(g0[3]), "+v"(g0[4]), "+v"(g0[5]), "+v"(g0[6]), "+v"(g0[7]), "+v"(g1[0]),
                 "+v"(g1[1]), "+v"(g1[2]), "+v"(g1[3]), "+v"(g1[4]), "+v"(g1[5]), "+v"(g1[6]),
                 "+v"(g1[7])
               :
               : "memory");
}

// Cache rows that a tile holds but the softmax masks (tile tails, -1 and
// out-of-range top-k ids) are read from this all-zero row instead of the
// pool: their P is 0, and 0 * V is only 0 when V is finite, which an
// unwritten pool row need not be. Large enough for every row format.
__device__ __attribute__((aligned(256))) unsigned char g_zero_row[1152];

// Device-built schedules (num_fd == SAS_SCHED_DEVICE): the summary is read from
// the metadata config row; num_fa and num_partial_slots are the launch and
// workspace capacities it must fit.
__device__ inline bool dev_sched_ok(const SasAttnArgs& a, int mb) {
  const int32_t* cfg = a.metadata + SAS_CFG_OFFSET;
  return cfg[0] == SAS_META_MAGIC && cfg[5] == a.num_heads && cfg[6] == mb &&
         cfg[2] >= 1 && cfg[2] <= a.num_fa && cfg[4] <= a.num_partial_slots &&
         cfg[3] >= 0 && cfg[3] <= SAS_AIV_CORE_NUM && cfg[1] >= 32 && cfg[1] % 32 == 0;
}
// An unusable device-built schedule: every output becomes NaN (one workgroup).
template <typename T>
__device__ void nan_fill(const SasAttnArgs& a, int tid, int nthreads) {
  const short qnan = __is_same(T, __bf16) ? (short)0x7FC0 : (short)0x7E00;
  const size_t rows = (size_t)a.total_tokens * a.num_heads;
  short* out = (short*)a.out;
  for (size_t k = tid; k < rows * a.head_dim_v; k += nthreads) out[k] = qnan;
  for (size_t k = tid; k < rows; k += nthreads) a.lse[k] = __builtin_nanf("");
}

// fp8 cache rows (SAS_KV_FP8_DS_MLA): eight e4m3 values (one 8-byte word) times
// their block scale, each product rounded to bf16 (v_cvt_pk_f32_fp8 decodes OCP
// e4m3 exactly; v_mul_f32 and v_cvt_pk_bf16_f32 round to nearest even).
__device__ inline i16x8 fp8x8_dequant_bf16(uint2 v, float s) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const f32x2 f0 = __builtin_amdgcn_cvt_pk_f32_fp8(v.x, false);
  const f32x2 f1 = __builtin_amdgcn_cvt_pk_f32_fp8(v.x, true);
  const f32x2 f2 = __builtin_amdgcn_cvt_pk_f32_fp8(v.y, false);
  const f32x2 f3 = __builtin_amdgcn_cvt_pk_f32_fp8(v.y, true);
  const bf16x2 b0 = __builtin_convertvector((f32x2){f0[0] * s, f0[1] * s}, bf16x2);
  const bf16x2 b1 = __builtin_convertvector((f32x2){f1[0] * s, f1[1] * s}, bf16x2);
  const bf16x2 b2 = __builtin_convertvector((f32x2){f2[0] * s, f2[1] * s}, bf16x2);
  const bf16x2 b3 = __builtin_convertvector((f32x2){f3[0] * s, f3[1] * s}, bf16x2);
  typedef short s2 __attribute__((ext_vector_type(2)));
  const s2 w0 = __builtin_bit_cast(s2, b0), w1 = __builtin_bit_cast(s2, b1);
  const s2 w2 = __builtin_bit_cast(s2, b2), w3 = __builtin_bit_cast(s2, b3);
  return (i16x8){w0[0], w0[1], w1[0], w1[1], w2[0], w2[1], w3[0], w3[1]};
}

// ---------------------------------------------------------------------------
// Attention kernel
// ---------------------------------------------------------------------------
// Waves: NHG head groups of 32 heads x 4 quarters = 4*NHG waves (two per SIMD
// for NHG = 2). Wave w -> head group hg = w % NHG, quarter q = w / NHG.
//   Q·Kᵀ: wave q computes a partial Sᵀ[32 rows x 32 heads] over dims quarter q
//         (main dims 128q..128q+127 and, for d_qk 576, rope dims 512+16q..+15).
//   reduce-scatter: the partials of a head group are summed through LDS; wave q
//         owns the 8 rows {8q + 4*hl + 0..3} (hl = lane / 32) of the sum.
//   softmax: on the 4 rows x 1 head a lane owns; P (rounded to the input type)
//         is shared through LDS, so every wave of the head group sees all 32
//         rows of P. Running max m is shared by the four waves; each keeps a
//         partial row sum (fp32 P) that is combined once per item.
//   P·V:  wave q accumulates Oᵀ[dv quarter q (128) x 32 heads] over all rows.
// Per tile: barrier A (partials written; the oldest stage is free for the
// next DMA) and barrier B (P written). A rescale (some head's max grew by more
// than 2^8) is decided workgroup-wide after B and costs one more barrier.
// fp8 rows (KVF = SAS_KV_FP8_DS_MLA): the main dims are loaded into VGPRs,
// dequantized to bf16 and written to the same LDS layout, so every read of a
// stage is the same as for a bf16 cache. Tile it + 2 is converted while tile
// it's P·V runs, and tile it + 3's loads are issued right after.
template <int DQK, int DV, int NHG, typename T, int KVF>
__global__ __launch_bounds__(256 * NHG) void attn_kernel(const SasAttnArgs a) {
  constexpr int NQ = 4;                  // dims / dv quarters per head group
  constexpr int NW = NQ * NHG;           // waves per workgroup
  constexpr int MB = 32 * NHG;           // heads per item (m-block)
  constexpr int NT = 64 * NW;            // threads
  constexpr bool ROPE = DQK == 576;      // 64 extra rope dims after the 512 main dims
  constexpr bool FP8 = KVF == SAS_KV_FP8_DS_MLA;
  constexpr int ROWB = FP8 ? SAS_FP8_ROW_BYTES : DQK * 2;  // bytes per cache row in HBM
  constexpr int ROPE_OFF = FP8 ? 528 : 1024;               // byte offset of the rope dims
  constexpr int NKS_MAIN = 8;            // k-steps over 128 main dims
  constexpr int NKS = NKS_MAIN + (ROPE ? 1 : 0);
  constexpr int DVB = DV / 32 / NQ;      // 32-wide dv blocks per wave (4)
  constexpr int STAGE_BYTES = MAIN_BYTES + (ROPE ? ROPE_BYTES : 0);
  constexpr int ROWS_PER_WAVE = TILE / NW;            // main-part DMA instructions per wave
  constexpr int NROPE = ROPE ? TILE / 8 : 0;          // rope DMA instructions per tile
  constexpr int PSTRIDE = 80;            // bytes per head in the P buffer (64 + pad)
  static_assert(DQK == 512 || DQK == 576, "head_dim");
  static_assert(DV == 512, "head_dim_v");
  static_assert((STAGE_BYTES % 1024) == 0, "stage alignment");
  static_assert(TILE % NW == 0, "rows per wave");
  static_assert(DVB == 4, "two groups of four dv blocks per wave");
  static_assert(NROPE <= NW, "at most one rope DMA instruction per wave");
  static_assert(!FP8 || (ROPE && __is_same(T, __bf16)), "fp8 rows: head_dim 576, bf16");
  constexpr int RPL = 2 * ROWS_PER_WAVE;  // fp8 path: rope bytes per lane per tile (8 or 16)
  typedef uint32_t ropev __attribute__((ext_vector_type(RPL / 4)));
  typedef MfmaOps<T> Ops;

  __shared__ __attribute__((aligned(1024))) unsigned char kv_lds[NSTAGE * STAGE_BYTES];
  __shared__ __attribute__((aligned(16))) f32x4 xpart[NHG][NQ][NQ][64];  // partial Sᵀ [dest][src]
  __shared__ __attribute__((aligned(16))) unsigned char pbuf[NHG][32 * PSTRIDE];
  __shared__ float mbuf[NHG][NQ][32];   // per-quarter row max (also the l combine)
  __shared__ __attribute__((aligned(8))) unsigned char flags[8];  // per-wave rescale votes
  __shared__ uint32_t rowid[RCHUNK];
  __shared__ uint32_t tmask[RCHUNK / TILE];
  __shared__ int first_neg[2];  // first -1 of the top-k scan (the slots alternate between scans)

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hg = w % NHG;
  const int q = w / NHG;
  const int hlocal = hg * 32 + (lane & 31);  // head within the item's m-block
  const int hblocks = (a.num_heads + MB - 1) / MB;
  const int hl = lane >> 5;
  // Kᵀ operand: row lane%32, main chunk 16q + 2ks + hl, rope chunk 64 + 2q + hl
  const int r_qk = lane & 31;
  const int qk_base = main_row_base(r_qk) + (16 * q + hl) * 16;
  const int rope_off = MAIN_BYTES + rope_slot(r_qk, 2 * q + hl) * 16;
  // Vᵀ operand (ds_read_b64_tr_b16): 16-lane group (lane>>4) reads rows
  // 4*hl + (lane&15)/4 (+16k, +8) at dv 128q + 16*((lane>>4)&1) + 4*(lane&3) (+32d).
  // Row r+16 has the same rotation as r; row r+8 (r%8 < 4) has rotation +2.
  const int tr_base = main_row_base(4 * hl + ((lane & 15) >> 2)) + q * (DV / NQ) * 2 +
                      ((lane >> 4) & 1) * 32 + (lane & 3) * 8;
  // P buffer: per head 32 bf16 in k-operand order. Position 16k + 8h + i holds
  // row 16k + 4h + i (i < 4) or 16k + 8 + 4h + (i - 4), matching the Vᵀ reads.
  // Wave q's rows 8q + 4hl + jj sit at 16(q/2) + 8hl + 4(q%2) + jj.
  unsigned char* prow = &pbuf[hg][(lane & 31) * PSTRIDE];
  const int pwr_off = (16 * (q >> 1) + 8 * hl + 4 * (q & 1)) * 2;

  int s2b = a.s2_base;
  int nfa = a.num_fa;
  if (a.num_fd == SAS_SCHED_DEVICE) {
    if (!dev_sched_ok(a, MB)) {
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

  const char* ori_kv = (const char*)a.ori_kv;
  const char* cmp_kv = (const char*)(a.cmp_kv ? a.cmp_kv : a.ori_kv);
  const float sc = a.softmax_scale * LOG2E;
  if (tid < 8) flags[tid] = 0;  // bytes of absent waves stay 0
  if (tid < 2) first_neg[tid] = INT32_MAX;
  __syncthreads();

  // Sinks of this lane's head in the (at most two: num_heads <= 128, 64-head
  // items above 32 heads) head blocks of an item, loaded once: a load per
  // item would also wait for the previous item's output stores (one in-order
  // counter covers loads and stores). The wait the compiler can see keeps
  // it from re-waiting at every use inside the item loop.
  const float sink_hb0 = hlocal < a.num_heads ? a.sinks[hlocal] : -INFINITY;
  const float sink_hb1 = MB + hlocal < a.num_heads ? a.sinks[MB + hlocal] : -INFINITY;
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0) expcnt(7) lgkmcnt(15)
  int item_par = 0;  // which first_neg slot the next top-k scan uses
  bool first_item = true;
  for (;;) {
    // the cursor is uniform: keep it in SGPRs so the per-item length and
    // prefix reads are scalar loads (a vector load here would wait for the
    // previous item's output stores, which share its in-order counter)
    b = __builtin_amdgcn_readfirstlane(b);
    m = __builtin_amdgcn_readfirstlane(m);
    // normalise the cursor: skip batches with no (more) query rows
    while (b < a.batch && b <= b_end && m >= ld_uniform(a.act_q_lens + b) * hblocks) {
      ++b;
      m = 0;
    }
    if (b >= a.batch || b > b_end || (b == b_end && m > s_end)) break;
    const bool is_end = (b == b_end && m == s_end);
    const int s = m / hblocks;
    const int head = (m - s * hblocks) * MB + hlocal;
    const bool head_ok = head < a.num_heads;
    if (is_end && j_end == 0) break;

    const int act_q = ld_uniform(a.act_q_lens + b);
    const int act_kv = ld_uniform(a.seqused_kv + b);
    const int tok = ld_uniform(a.q_prefix + b) + s;
    const ItemGeom g =
        item_geom(act_q, act_kv, s, a.ori_win_left, a.scenario, a.cmp_ratio, a.topk);
    const int L = g.n_win + g.n_cmp;
    const int nblk = (L + s2b - 1) / s2b;
    const int blo = first_item ? j_start : 0;
    int bhi = is_end ? j_end : nblk;
    if (bhi > nblk) bhi = nblk;
    const bool partial = (first_item && j_start > 0) || is_end;
    const int p_lo = blo * s2b;
    const int p_hi = bhi * s2b < L ? bhi * s2b : L;
    const bool tok_ok = tok >= 0 && tok < a.total_tokens;

    // query fragment for this wave's dims (B operand of Sᵀ = K·Qᵀ)
    i16x8 qf[NKS];
    // ---- online-softmax state: m shared by the head group, l partial per wave ----
    // (golden.py:156-160 seeds m = sink, l = 1: the 1 goes to one lane of quarter 0;
    // the row sums of lanes l and l ^ 32 (same head) are added at the end)
    const int hb = m - s * hblocks;
    const float sink_v = hb == 0 ? sink_hb0 : sink_hb1;
    float m_run = partial ? -INFINITY : (head_ok ? sink_v * LOG2E : -INFINITY);
    float l_part = (partial || q != 0 || hl != 0) ? 0.0f : 1.0f;
    f32x16 acc[DVB];
#pragma unroll
    for (int d = 0; d < DVB; ++d)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[d][j] = 0.0f;

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

    for (int c0 = p_lo; c0 < p_hi; c0 += RCHUNK) {
      const int clen = (p_hi - c0) < RCHUNK ? (p_hi - c0) : RCHUNK;
      const int ntile = (clen + TILE - 1) / TILE;
      // ---- resolve positions -> cache rows (bit 31: compressed cache) ----
      // Thread tid owns positions c0 + e*NT + tid. Phase 1 issues the top-k
      // loads, phase 2 the block-table loads, phase 3 packs and publishes.
      constexpr int PER = RCHUNK / NT;
      int cid[PER];
      int tab[PER];  // block-table word to read, or -1
      // Loads are unconditional with clamped, always in-bounds indices (so all
      // of a phase's loads are in flight together); results are masked after.
      // (two branches: a load-free path must not inherit the top-k path's wait,
      // which would also wait for the previous item's output stores)
      // The -1 scan of the top-k slots [0, jmax) outside this chunk's own
      // [own_lo, own_hi) (first chunk of a scanned item only): its first
      // NT * SCAN_PER slots are loaded together with the chunk's own ids.
      const int own_lo = max(c0 - g.n_win, 0);
      const int own_hi = min(max(c0 + clen - g.n_win, own_lo), jmax);
      const int n_extra = stop_pending ? jmax - (own_hi - own_lo) : 0;
      constexpr int SCAN_PER = 4;
      auto extra_slot = [&](int x) {  // x-th slot outside the own range
        return x < own_lo ? x : x + (own_hi - own_lo);
      };
      int sv0[SCAN_PER];
      if (scan3) {
        // all loads issued, then one wait (as asm: the compiler gives such loads
        // one destination register and a wait each)
        int v[PER];
#pragma unroll
        for (int e = 0; e < PER; ++e) {
          const int jj = c0 + e * NT + tid - g.n_win;
          const int32_t* src = idx_row + (jj < 0 ? 0 : (jj < a.topk ? jj : a.topk - 1));
          asm volatile("global_load_dword %0, %1, off" : "=v"(v[e]) : "v"(src) : "memory");
        }
#pragma unroll
        for (int e = 0; e < SCAN_PER; ++e) {
          const int x = e * NT + tid;  // clamped into range; unused when n_extra == 0
          const int xc = x < n_extra ? x : (n_extra > 0 ? n_extra - 1 : 0);
          const int32_t* src = idx_row + (n_extra > 0 ? extra_slot(xc) : 0);
          asm volatile("global_load_dword %0, %1, off" : "=v"(sv0[e]) : "v"(src) : "memory");
        }
        static_assert(PER == 2 || PER == 4, "resolution positions per thread");
        static_assert(SCAN_PER == 4, "scan loads tied below");
        if constexpr (PER == 2)
          asm volatile("s_waitcnt vmcnt(0)"
                       : "+v"(v[0]), "+v"(v[1]), "+v"(sv0[0]), "+v"(sv0[1]), "+v"(sv0[2]),
                         "+v"(sv0[3])
                       :
                       : "memory");
        else
          asm volatile("s_waitcnt vmcnt(0)"
                       : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(sv0[0]),
                         "+v"(sv0[1]), "+v"(sv0[2]), "+v"(sv0[3])
                       :
                       : "memory");
#pragma unroll
        for (int e = 0; e < PER; ++e) {
          const int r = e * NT + tid;
          const int pos = c0 + r;
          cid[e] = (r < clen && tok_ok && pos >= g.n_win) ? v[e] : -1;
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
      // Block-table words (the query fragment is loaded after the resolution).
      // d_qk 512: as asm loads with one wait, the wait and the tie of their
      // destination registers being one statement (no copy of a register can be
      // placed between an asm load and its wait); every load has an in-bounds
      // address (masked lanes read word 0 of the window table).
      const bool load_q = c0 == p_lo;
      if constexpr (!ROPE) {
        bool tab_ok[PER];
        int tword[PER];
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
          tab_ok[e] = r < clen && tok_ok && key >= 0 && bi < tlen && (win || cid[e] < g.thr) &&
                      tbl != nullptr;
          const int32_t* src = tab_ok[e] ? tbl + (size_t)b * tlen + bi : a.ori_block_table;
          asm volatile("global_load_dword %0, %1, off" : "=v"(tword[e]) : "v"(src) : "memory");
        }
        static_assert(PER == 2 || PER == 4, "resolution positions per thread");
        if constexpr (PER == 2)
          asm volatile("s_waitcnt vmcnt(0)" : "+v"(tword[0]), "+v"(tword[1]) : : "memory");
        else
          asm volatile("s_waitcnt vmcnt(0)"
                       : "+v"(tword[0]), "+v"(tword[1]), "+v"(tword[2]), "+v"(tword[3])
                       : : "memory");
#pragma unroll
        for (int e = 0; e < PER; ++e) tab[e] = tab_ok[e] ? tword[e] : -1;
      } else {
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
      }
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
      // main part: wave w fills rows w, w + NW, ...; one 1 KB row per instruction
      // rope part: instruction i fills rows 8i..8i+7 (8 lanes per row)
      // branch-free row address (bit 31 of the id selects the compressed cache)
      auto row_ptr = [&](uint32_t id) -> const char* {
        const char* base = (id & 0x80000000u) ? cmp_kv : ori_kv;
        const char* p = base + (size_t)(id & 0x7FFFFFFFu) * ROWB;
        return id == ROW_INVALID ? (const char*)g_zero_row : p;
      };
      // row addresses a wave needs to issue one tile, computed per lane ahead of
      // use (off the path between barrier A and the DMA issue): lane j <
      // ROWS_PER_WAVE holds the address of its j-th main row; for the rope
      // instruction (waves w < NROPE) lane l holds that of row 8w + l/8.
      auto main_ptrs = [&](int tile) -> uint64_t {
        return (uint64_t)(uintptr_t)row_ptr(
            rowid[tile * TILE + w + NW * (lane < ROWS_PER_WAVE ? lane : 0)]);
      };
      // (computed by every wave, without a branch; only waves w < NROPE use it)
      auto rope_ptr = [&](int tile) -> uint64_t {
        const int wr = ROPE && w < NROPE ? w : 0;
        return (uint64_t)(uintptr_t)row_ptr(rowid[tile * TILE + 8 * wr + (lane >> 3)]);
      };
      // address of main row j from lane j (two v_readlane, no scalar arithmetic)
      auto lane_row = [&](uint64_t ptrs, int j) -> const char* {
        const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)ptrs, j);
        const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(ptrs >> 32), j);
        return (const char*)(uintptr_t)(((uint64_t)hi << 32) | lo);
      };
      auto issue = [&](int stage, uint64_t my_ptrs, uint64_t rope_row) {
        const uint32_t sbase = kv_base + stage * STAGE_BYTES;
#pragma unroll
        for (int j = 0; j < ROWS_PER_WAVE; ++j) {
          const int r = w + NW * j;
          dma16_sbase(lane_row(my_ptrs, j), (uint32_t)lane * 16u, sbase + main_row_base(r));
        }
        if (ROPE && w < NROPE) {
          const int r = 8 * w + (lane >> 3);
          const int cr = ((lane & 7) - (r >> 1)) & 7;
          const char* src = (const char*)(uintptr_t)rope_row + 1024 + cr * 16;
          dma16_vaddr(src, sbase + MAIN_BYTES + w * 1024);
        }
      };
      // ---- fp8 rows: VGPR loads, then dequantize into one ring stage ----
      // wave w takes rows w + NW j (j < ROWS_PER_WAVE): lane l loads bytes 8l..8l+7
      // (dims 8l..8l+7, scale l / 16) of each, and RPL rope bytes of row
      // w + NW (l / (128 / RPL)).
      struct Fp8Tile {
        uint2 v[ROWS_PER_WAVE];
        float s[ROWS_PER_WAVE];
        ropev rope;
      };
      constexpr int ROPE_LPR = 128 / RPL;  // lanes per row for the rope bytes
      // (global, non-temporal loads: the rows stream through once, as the
      // native rows' DMAs do)
      typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
      auto fp8_load = [&](Fp8Tile& f, uint64_t my_ptrs) {
        const char* rp = nullptr;
#pragma unroll
        for (int j = 0; j < ROWS_PER_WAVE; ++j) {
          const char* p = lane_row(my_ptrs, j);
          const u32x2 t = __builtin_nontemporal_load((const SAS_GLOBAL u32x2*)(p + 8 * lane));
          f.v[j] = make_uint2(t[0], t[1]);
          f.s[j] = __builtin_nontemporal_load((const SAS_GLOBAL float*)(p + 512 + 4 * (lane >> 4)));
          rp = (lane / ROPE_LPR == j) ? p : rp;
        }
        f.rope = __builtin_nontemporal_load(
            (const SAS_GLOBAL ropev*)(rp + ROPE_OFF + (lane % ROPE_LPR) * RPL));
      };
      auto fp8_store = [&](const Fp8Tile& f, int stage) {
        unsigned char* sb = kv_lds + stage * STAGE_BYTES;
#pragma unroll
        for (int j = 0; j < ROWS_PER_WAVE; ++j) {
          const int r = w + NW * j;
          *(i16x8*)(sb + main_row_base(r) + 16 * lane) = fp8x8_dequant_bf16(f.v[j], f.s[j]);
        }
        const int r = w + NW * (lane / ROPE_LPR);
        const int byte = (lane % ROPE_LPR) * RPL;
        *(ropev*)(sb + MAIN_BYTES + rope_slot(r, byte >> 4) * 16 + (byte & 15)) = f.rope;
      };
      Fp8Tile fpt;


      if constexpr (FP8) {
        Fp8Tile f1;
        fp8_load(fpt, main_ptrs(0));
        if (ntile > 1) fp8_load(f1, main_ptrs(1));
        fp8_store(fpt, 0);
        if (ntile > 1) fp8_store(f1, 1);
      } else {
        issue(0, main_ptrs(0), rope_ptr(0));
        if (ntile > 1) issue(1, main_ptrs(1), rope_ptr(1));
      }
      // query fragment (compiler-visible loads, in flight with tiles 0 and 1)
      if (load_q) {
        const short* qrow = (const short*)a.q + ((size_t)(tok_ok ? tok : 0) * a.num_heads +
                                                 (head_ok ? head : 0)) * DQK;
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
          const int dim = ks < NKS_MAIN ? (128 * q + 16 * ks + 8 * hl) : (512 + 16 * q + 8 * hl);
          i16x8 v = *(const i16x8*)(qrow + dim);
          qf[ks] = (head_ok && tok_ok) ? v : (i16x8){0, 0, 0, 0, 0, 0, 0, 0};
        }
      }
      // A wait the compiler can see: it clears its pending-load state here, so it
      // puts no vmcnt wait for qf inside the tile loop (that wait would also drain
      // the row DMAs in flight on every tile). Also lands tiles 0 and 1.
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0) expcnt(7) lgkmcnt(15)
      if (FP8 && ntile > 2) fp8_load(fpt, main_ptrs(2));
      __syncthreads();

      // ---- Sᵀ partial of one tile over this wave's dims quarter (K operands 3 deep) ----
      auto qk = [&](int stg) -> f32x16 {
        const unsigned char* kb = kv_lds + stg * STAGE_BYTES;
        auto kaddr = [&](int ks) -> const i16x8* {
          return (const i16x8*)(ks < NKS_MAIN ? kb + qk_base + ks * 32 : kb + rope_off);
        };
        f32x16 r;
#pragma unroll
        for (int j = 0; j < 16; ++j) r[j] = 0.0f;
        constexpr int PF = 3;
        i16x8 kbuf[PF];
#pragma unroll
        for (int i = 0; i < PF; ++i) kbuf[i] = *kaddr(i);
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
          const i16x8 kop = kbuf[ks % PF];
          if (ks + PF < NKS) kbuf[ks % PF] = *kaddr(ks + PF);
          r = Ops::mma(kop, qf[ks], r);
        }
        return r;
      };
      // ---- reduce-scatter of the partials: quarter G's rows go to wave G ----
      auto write_partials = [&](const f32x16& r) {
#pragma unroll
        for (int G = 0; G < NQ; ++G)
          xpart[hg][G][q][lane] = (f32x4){r[4 * G], r[4 * G + 1], r[4 * G + 2], r[4 * G + 3]};
      };

      // Software pipeline over tiles. Iteration it runs Q·Kᵀ of tile it + 1 (its
      // MFMAs execute under the softmax of tile it), the softmax and P·V of tile
      // it, and publishes the partials of tile it + 1:
      //   barrier A(it): partials of tile it visible; stage (it + 2) % 3 (tile
      //                  it - 1's) free
      //   barrier B(it): P of tile it visible
      // Tile it + 2 is issued at the head of iteration it, into the stage that
      // barrier A(it) has released (tile it - 1's), and must have landed before
      // barrier A(it + 1).
      write_partials(qk(0));
      __syncthreads();  // barrier A(0)
      // row addresses of the next tile to issue (tile it + 2 at the head of
      // iteration it; garbage and unused when there is no such tile)
      uint64_t pend_main = 0, pend_rope = 0;
      if constexpr (!FP8) {
        pend_main = main_ptrs(2);
        pend_rope = rope_ptr(2);
      }

      for (int it = 0; it < ntile; ++it) {
        const int stage = it % NSTAGE;
        const unsigned char* sb = kv_lds + stage * STAGE_BYTES;
        const bool has_next = it + 1 < ntile;
        const bool more = it + 2 < ntile;
        const int nx_tile = it + 3 < ntile ? it + 3 : it;
        // Vᵀ operands of this tile (the A operand of P·V)
        const uint32_t trb = (uint32_t)(uintptr_t)(sb + tr_base);
        i16x4 gbuf[2][8];
        auto read_vt = [&]() {
#define SAS_TR_GROUP(GI, DST)                                                              \
  {                                                                                        \
    constexpr int q_ = (GI);                                                               \
    DST[0] = ds_read_tr16<(16 * q_) * MAIN_ROW_BYTES + 0 * 64>(trb);                       \
    DST[1] = ds_read_tr16<(16 * q_ + 8) * MAIN_ROW_BYTES + 32 + 0 * 64>(trb);              \
    DST[2] = ds_read_tr16<(16 * q_) * MAIN_ROW_BYTES + 1 * 64>(trb);                       \
    DST[3] = ds_read_tr16<(16 * q_ + 8) * MAIN_ROW_BYTES + 32 + 1 * 64>(trb);              \
    DST[4] = ds_read_tr16<(16 * q_) * MAIN_ROW_BYTES + 2 * 64>(trb);                       \
    DST[5] = ds_read_tr16<(16 * q_ + 8) * MAIN_ROW_BYTES + 32 + 2 * 64>(trb);              \
    DST[6] = ds_read_tr16<(16 * q_) * MAIN_ROW_BYTES + 3 * 64>(trb);                       \
    DST[7] = ds_read_tr16<(16 * q_ + 8) * MAIN_ROW_BYTES + 32 + 3 * 64>(trb);              \
  }
          SAS_TR_GROUP(0, gbuf[0]);
          SAS_TR_GROUP(1, gbuf[1]);
#undef SAS_TR_GROUP
        };
        uint32_t vm_tile;
        uint64_t nx_main, nx_rope = 0;
        f32x16 st_next;
        f32x4 sred;
        if constexpr (!FP8) {
          // Every LDS read of the Q·Kᵀ / softmax phase is one ordered asm group,
          // waited for by count: the tile mask and next-DMA row ids, Kᵀ of tile
          // it + 1 and the partials of tile it; then the Vᵀ operands of tile it,
          // so they stream in under the Q·Kᵀ MFMAs instead of between barrier B
          // and P·V. (The fp8 form keeps the reads in source order: the extra
          // live registers would spill there.)
          vm_tile = ds_read_b32_asm((uint32_t)(uintptr_t)&tmask[it]);
          uint32_t rid_main = ds_read_b32_asm((uint32_t)(uintptr_t)&rowid[
              nx_tile * TILE + w + NW * (lane < ROWS_PER_WAVE ? lane : 0)]);
          const int wr = ROPE && w < NROPE ? w : 0;
          uint32_t rid_rope =
              ds_read_b32_asm((uint32_t)(uintptr_t)&rowid[nx_tile * TILE + 8 * wr + (lane >> 3)]);
          const unsigned char* kbn = kv_lds + ((it + 1) % NSTAGE) * STAGE_BYTES;
          const uint32_t ka = (uint32_t)(uintptr_t)(kbn + qk_base);
          i16x8 kq[NKS];
          kq[0] = ds_read_b128_asm<0>(ka);
          kq[1] = ds_read_b128_asm<32>(ka);
          kq[2] = ds_read_b128_asm<64>(ka);
          kq[3] = ds_read_b128_asm<96>(ka);
          kq[4] = ds_read_b128_asm<128>(ka);
          kq[5] = ds_read_b128_asm<160>(ka);
          kq[6] = ds_read_b128_asm<192>(ka);
          kq[7] = ds_read_b128_asm<224>(ka);
          if constexpr (ROPE) kq[8] = ds_read_b128_asm<0>((uint32_t)(uintptr_t)(kbn + rope_off));
          const uint32_t xa = (uint32_t)(uintptr_t)&xpart[hg][q][0][lane];
          i16x8 xp[NQ];
          xp[0] = ds_read_b128_asm<0>(xa);
          xp[1] = ds_read_b128_asm<1024>(xa);
          xp[2] = ds_read_b128_asm<2048>(xa);
          xp[3] = ds_read_b128_asm<3072>(xa);
          // Tile it + 2 into the stage tile it - 1 has released (barrier A(it)),
          // issued behind this phase's first LDS reads so that their latency runs
          // under the DMA issue's memory-pipeline back-pressure. The LDS DMA
          // counts in vmcnt only: the lgkmcnt waits below are unchanged.
          if (it + 2 < ntile) issue((it + 2) % NSTAGE, pend_main, pend_rope);
          // mask, row ids and Kᵀ have landed (only the four partial reads may be
          // pending; LDS reads of a wave complete in order). Each asm output
          // register appears once: a duplicated operand makes the compiler copy
          // the register before the wait, i.e. before the data has arrived.
          if constexpr (ROPE)
            asm volatile("s_waitcnt lgkmcnt(4)"
                         : "+v"(vm_tile), "+v"(rid_main), "+v"(rid_rope), "+v"(kq[0]), "+v"(kq[1]),
                           "+v"(kq[2]), "+v"(kq[3]), "+v"(kq[4]), "+v"(kq[5]), "+v"(kq[6]),
                           "+v"(kq[7]), "+v"(kq[8])
                         :
                         : "memory");
          else
            asm volatile("s_waitcnt lgkmcnt(4)"
                         : "+v"(vm_tile), "+v"(rid_main), "+v"(rid_rope), "+v"(kq[0]), "+v"(kq[1]),
                           "+v"(kq[2]), "+v"(kq[3]), "+v"(kq[4]), "+v"(kq[5]), "+v"(kq[6]),
                           "+v"(kq[7])
                         :
                         : "memory");
          read_vt();
          nx_main = (uint64_t)(uintptr_t)row_ptr(rid_main);
          nx_rope = (uint64_t)(uintptr_t)row_ptr(rid_rope);
          // ---- Q·Kᵀ of the next tile (results needed only after P·V; on the
          // last tile it reads a stale stage and is discarded) ----
#pragma unroll
          for (int j = 0; j < 16; ++j) st_next[j] = 0.0f;
#pragma unroll
          for (int ks = 0; ks < NKS; ++ks) st_next = Ops::mma(kq[ks], qf[ks], st_next);
          // the partials have landed (at most 15 of the 16 Vᵀ reads pending)
          asm volatile("s_waitcnt lgkmcnt(15)"
                       : "+v"(xp[0]), "+v"(xp[1]), "+v"(xp[2]), "+v"(xp[3])
                       :
                       : "memory");
          // fixed summation order over source quarters 0, 1, 2, 3
          sred = ((__builtin_bit_cast(f32x4, xp[0]) + __builtin_bit_cast(f32x4, xp[1])) +
                  __builtin_bit_cast(f32x4, xp[2])) + __builtin_bit_cast(f32x4, xp[3]);
        } else {
          vm_tile = tmask[it];
          nx_main = main_ptrs(nx_tile);
          st_next = qk((it + 1) % NSTAGE);
          sred = ((xpart[hg][q][0][lane] + xpart[hg][q][1][lane]) + xpart[hg][q][2][lane]) +
                 xpart[hg][q][3][lane];
        }

        // ---- online softmax (exp2 domain) on rows 8q + 4hl + jj ----
        const uint32_t vm = vm_tile >> (8 * q + 4 * hl);
        float sv[4];
        float mloc = -INFINITY;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sv[e] = ((vm >> e) & 1u) ? sred[e] * sc : -INFINITY;
          mloc = fmaxf(mloc, sv[e]);
        }
        mloc = wave_max_pair(mloc);
        // lanes l and l ^ 32 store the same value to the same word (no branch)
        mbuf[hg][q][lane & 31] = mloc;
        const bool need_any = __any(mloc > m_run + RESCALE_TAU);
        flags[w] = need_any ? 1 : 0;
        float pv[4];
        auto make_p = [&]() {
          i16x4 pk4;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            pv[e] = (sv[e] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(sv[e] - m_run);
            pk4[e] = Ops::from_f32(pv[e]);
          }
          *(i16x4*)(prow + pwr_off) = pk4;
        };
        make_p();
        // next DMA addresses, computed before barrier B
        pin_u64(nx_main);
        if (!FP8) pin_u64(nx_rope);
        __syncthreads();  // barrier B(it)
        // fp8 rows: partials of tile it + 1 published here, so the Sᵀ registers are
        // free during P·V (every wave has read tile it's partials before barrier
        // B; on the last tile they are garbage and never read)
        if (FP8) write_partials(st_next);

        // rescale votes and the P operand of both k-steps (and, for fp8 rows,
        // Vᵀ of the whole tile): issued together, then one wait (none of the
        // asm outputs is touched before it)
        const uint32_t pka = (uint32_t)(uintptr_t)(prow + 16 * hl);
        uint64_t votes = ds_read_b64_asm((uint32_t)(uintptr_t)flags);
        i16x8 pk[2];
        pk[0] = ds_read_b128_asm<0>(pka);
        pk[1] = ds_read_b128_asm<32>(pka);
        if constexpr (FP8) read_vt();
        lds_wait_pv(votes, pk, gbuf[0], gbuf[1]);
        if (__builtin_amdgcn_readfirstlane((uint32_t)(votes | (votes >> 32)))) {
          // rescale: every wave of the head group derives the same new max
          float mt = mbuf[hg][0][lane & 31];
#pragma unroll
          for (int i = 1; i < NQ; ++i) mt = fmaxf(mt, mbuf[hg][i][lane & 31]);
          if (mt > m_run + RESCALE_TAU) {
            const float m2 = fmaxf(m_run, mt);
            const float alpha = __builtin_amdgcn_exp2f(m_run - m2);  // m_run = -inf -> 0
            l_part *= alpha;
#pragma unroll
            for (int d = 0; d < DVB; ++d)
#pragma unroll
              for (int j = 0; j < 16; ++j) acc[d][j] *= alpha;
            m_run = m2;
          }
          make_p();         // rewrite this wave's rows with the new max (the P
          __syncthreads();  // read above is void and is repeated after barrier C)
          pk[0] = *(const i16x8*)(prow + 16 * hl);
          pk[1] = *(const i16x8*)(prow + 32 + 16 * hl);
        }
        l_part += (pv[0] + pv[1]) + (pv[2] + pv[3]);

        // ---- Oᵀ += Vᵀ · Pᵀ over both 16-row k-steps ----
        // (issue priority to this wave's MFMA chain while its SIMD partner runs
        // VALU / LDS work)
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int kq = 0; kq < 2; ++kq)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const i16x4* g = gbuf[kq];
            const i16x8 aop = {g[2 * e][0],     g[2 * e][1],     g[2 * e][2],     g[2 * e][3],
                               g[2 * e + 1][0], g[2 * e + 1][1], g[2 * e + 1][2], g[2 * e + 1][3]};
            acc[e] = Ops::mma(aop, pk[kq], acc[e]);
          }
        __builtin_amdgcn_s_setprio(0);
        // fp8 rows: stage (it + 2) % 3 last held tile it - 1, read before barrier A(it)
        if constexpr (FP8) {
          if (more) fp8_store(fpt, (it + 2) % NSTAGE);
          if (it + 3 < ntile) fp8_load(fpt, nx_main);
        }
        if (has_next) {
          if (!FP8) write_partials(st_next);
          if (!FP8) wait_vmcnt<0>();  // this wave's share of tile it + 2 has landed
          __syncthreads();            // barrier A(it + 1)
          if constexpr (!FP8) {       // tile it + 3 is issued at the next loop head
            pend_main = nx_main;
            pend_rope = nx_rope;
          }
        }
      }
      __syncthreads();  // rowid / tmask / ring are rewritten by the next chunk or item
    }

    // ---- combine the row sums of the four quarters (fixed order) ----
    l_part = wave_sum_pair(l_part);
    if (hl == 0) mbuf[hg][q][lane & 31] = l_part;
    __syncthreads();
    const float l_run = ((mbuf[hg][0][lane & 31] + mbuf[hg][1][lane & 31]) +
                         mbuf[hg][2][lane & 31]) + mbuf[hg][3][lane & 31];
    __syncthreads();  // mbuf is reused by the next item

    // ---- epilogue: the item's rows go out through LDS (the ring is free), so
    // every store instruction writes whole rows (1 KB per wave) instead of
    // 16- or 32-byte pieces of 32 rows ----
    {
      unsigned char* stg = kv_lds;
      const int nh = min(MB, a.num_heads - hb * MB);  // heads of this item
      // opaque copies of the thread indices: the addresses below are then
      // computed here, not hoisted out of the item loop (where they would
      // occupy registers across the tile loop)
      int tid_e = tid, hl_e = hlocal, dv_e = q * (DV / NQ) + 4 * hl;
      asm volatile("" : "+v"(tid_e), "+v"(hl_e), "+v"(dv_e));
      if (!partial) {
        constexpr int SROW = DV * 2 + 8;   // staging row stride (bytes)
        constexpr int CPR = DV * 2 / 16;   // 16-byte chunks per row
        static_assert(MB * SROW <= NSTAGE * STAGE_BYTES, "output staging");
        const float inv = 1.0f / l_run;
#pragma unroll
        for (int d = 0; d < DVB; ++d)
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            const int dv = dv_e + 32 * d + 8 * g4;
            const i16x4 v = {Ops::from_f32(acc[d][4 * g4] * inv),
                             Ops::from_f32(acc[d][4 * g4 + 1] * inv),
                             Ops::from_f32(acc[d][4 * g4 + 2] * inv),
                             Ops::from_f32(acc[d][4 * g4 + 3] * inv)};
            *(i16x4*)(stg + hl_e * SROW + dv * 2) = v;
          }
        __syncthreads();
        if (tok_ok) {
          char* obase = (char*)((T*)a.out + ((size_t)tok * a.num_heads + hb * MB) * DV);
          for (int c = tid_e; c < nh * CPR; c += NT) {
            const int h = c / CPR, c16 = c - h * CPR;
            *(i16x8*)(obase + (size_t)h * DV * 2 + c16 * 16) = *(const i16x8*)(stg + h * SROW + c16 * 16);
          }
          if (q == 0 && hl == 0 && head_ok)
            a.lse[(size_t)tok * a.num_heads + hb * MB + hl_e] = (m_run + __log2f(l_run)) * LN2;
        }
      } else if (slot >= 0 && slot < a.num_partial_slots && a.workspace) {
        // fp32 partials (acc / l), staged in two halves of the dv range
        constexpr int HALF = DV / 2;
        constexpr int SROW = HALF * 4 + 16;
        constexpr int CPR = HALF * 4 / 16;
        static_assert(MB * SROW <= NSTAGE * STAGE_BYTES, "partial staging");
        const bool empty = !(l_run > 0.0f);
        const float inv = empty ? 0.0f : 1.0f / l_run;
        char* wbase = (char*)(a.workspace + (size_t)slot * MB * DV);
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          if (half) __syncthreads();  // the first half has been read out
          if ((q >> 1) == half) {  // waves whose dv quarter lies in this half
#pragma unroll
            for (int d = 0; d < DVB; ++d)
#pragma unroll
              for (int g4 = 0; g4 < 4; ++g4) {
                const int dv = dv_e - half * HALF + 32 * d + 8 * g4;  // within the half
                f32x4 v;
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = acc[d][4 * g4 + e] * inv;
                *(f32x4*)(stg + hl_e * SROW + dv * 4) = v;
              }
          }
          __syncthreads();
          for (int c = tid_e; c < nh * CPR; c += NT) {
            const int h = c / CPR, c16 = c - h * CPR;
            *(f32x4*)(wbase + ((size_t)h * DV + half * HALF) * 4 + c16 * 16) =
                *(const f32x4*)(stg + h * SROW + c16 * 16);
          }
        }
        if (q == 0 && hl == 0 && head_ok) {
          float* wl = a.workspace + (size_t)a.num_partial_slots * MB * DV;
          wl[(size_t)slot * MB + hl_e] =
              empty ? -INFINITY : (m_run + __log2f(l_run)) * LN2;
        }
      }
    }
    if (partial) ++slot;
    if (is_end) break;
    first_item = false;
    ++m;
  }
}

// ---------------------------------------------------------------------------
// Split-KV merge: lse = log(e^sink + Σ e^lse_i), out = Σ e^(lse_i - lse) o_i
// ---------------------------------------------------------------------------
// Grid: (merge task, group of MERGE_HPB heads). Thread t owns head t / 32 of
// the group and float4 columns (t % 32) + 32 k: a half-wave reads 512
// contiguous bytes per load. Each thread derives its head's weights itself
// (the piece lse values are the same words for its 32 lanes), so there is no
// LDS and no barrier, and the first two pieces' loads are in flight with the
// lse, sink and token loads.
constexpr int MERGE_HPB = 8;          // heads per workgroup
constexpr int MERGE_THREADS = 256;

template <int DV, typename T>
__device__ __forceinline__ void merge_task(const SasAttnArgs& a, int task) {
  constexpr int V4 = DV / 4;                              // float4 per head row
  constexpr int TPH = MERGE_THREADS / MERGE_HPB;          // threads per head (32)
  constexpr int PER = V4 / TPH;                           // float4 per thread (4)
  static_assert(V4 % TPH == 0 && TPH <= 64 && 64 % TPH == 0, "merge tiling");
  const int32_t* fd = a.metadata + SAS_FD_OFFSET + task * SAS_FD_METADATA_SIZE;
  if (fd[0] == 0) return;
  const int mb = a.m_base;
  const int hblocks = (a.num_heads + mb - 1) / mb;
  const int b = fd[1], m = fd[2], slot0 = fd[3], npc = fd[4], h0 = fd[5], hn = fd[6];
  if (b < 0 || b >= a.batch || m < 0 || slot0 < 0 || npc < 1 ||
      slot0 + npc > a.num_partial_slots || h0 < 0 || hn < 1 || h0 + hn > mb)
    return;
  const int g0 = (int)blockIdx.y * MERGE_HPB;  // first head of this group within the task
  if (g0 >= hn) return;
  const int tid = threadIdx.x;
  const int hh = tid / TPH;
  const int c0 = tid % TPH;
  // rows past the task's last head (never stored) read that head's row instead
  const int hr = g0 + hh < hn ? g0 + hh : hn - 1;
  const int hloc = h0 + hr;                            // m-block slot of this thread's row
  const float* wo = a.workspace;
  const float* wl = a.workspace + (size_t)a.num_partial_slots * mb * DV;
  auto piece = [&](int i, f32x4 (&v)[PER]) {
    const float* src = wo + ((size_t)(slot0 + i) * mb + hloc) * DV + 4 * c0;
#pragma unroll
    for (int k = 0; k < PER; ++k)  // all of one piece's loads in flight together
      v[k] = *(const f32x4*)(src + 4 * TPH * k);
  };
  auto plse = [&](int i) -> float { return wl[(size_t)(slot0 + i) * mb + hloc]; };
  const int s = m / hblocks;
  const int h = (m - s * hblocks) * mb + hloc;  // query head
  const bool store = g0 + hh < hn && h < a.num_heads;
  const float sink = a.sinks[h < a.num_heads ? h : a.num_heads - 1];
  const int tok = a.q_prefix[b] + s;
  // lse = log(e^sink + Σ_i e^lse_i); weights e^(lse_i - lse); the sums keep the
  // piece order 0, 1, 2, ...
  f32x4 o[PER];
  float l = -INFINITY;
  auto weight = [&](float li) -> float {
    return (l == -INFINITY || li == -INFINITY) ? 0.0f : __expf(li - l);
  };
  if (npc <= 2) {
    // one or two pieces: both fetched before the weights are known
    f32x4 v0[PER], v1[PER];
    piece(0, v0);
    if (npc > 1) piece(1, v1);
    const float l0 = plse(0);
    const float l1 = npc > 1 ? plse(1) : -INFINITY;
    float mx = fmaxf(sink, l0);
    if (npc > 1) mx = fmaxf(mx, l1);
    if (mx != -INFINITY) {  // else no key and no sink: lse -inf, every weight 0
      float tot = __expf(sink - mx) + __expf(l0 - mx);
      if (npc > 1) tot += __expf(l1 - mx);
      l = mx + __logf(tot);
    }
    const float w0 = weight(l0);
#pragma unroll
    for (int k = 0; k < PER; ++k)
      o[k] = (f32x4){w0 * v0[k][0], w0 * v0[k][1], w0 * v0[k][2], w0 * v0[k][3]};
    if (npc > 1) {
      const float w1 = weight(l1);
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        o[k][0] += w1 * v1[k][0]; o[k][1] += w1 * v1[k][1];
        o[k][2] += w1 * v1[k][2]; o[k][3] += w1 * v1[k][3];
      }
    }
  } else {
    // more pieces: their data in batches of PB with all loads of a batch in
    // flight together, the first MAXL lse values in one batch (a loop of one
    // piece per round trip costs a memory latency per piece)
    constexpr int PB = 4;
    constexpr int MAXL = 16;
    f32x4 vb[PB][PER];
#pragma unroll
    for (int i = 0; i < PB; ++i) piece(i < npc ? i : npc - 1, vb[i]);
    float lv[MAXL];
#pragma unroll
    for (int i = 0; i < MAXL; ++i) lv[i] = plse(i < npc ? i : npc - 1);
    auto lse_of = [&](int i) -> float { return i < MAXL ? lv[i] : plse(i); };
    float mx = fmaxf(sink, lv[0]);
#pragma unroll
    for (int i = 1; i < MAXL; ++i)
      if (i < npc) mx = fmaxf(mx, lv[i]);
    for (int i = MAXL; i < npc; ++i) mx = fmaxf(mx, plse(i));
    if (mx != -INFINITY) {
      float tot = __expf(sink - mx) + __expf(lv[0] - mx);
#pragma unroll
      for (int i = 1; i < MAXL; ++i)
        if (i < npc) tot += __expf(lv[i] - mx);
      for (int i = MAXL; i < npc; ++i) tot += __expf(plse(i) - mx);
      l = mx + __logf(tot);
    }
    for (int i0 = 0; i0 < npc; i0 += PB) {
      if (i0 > 0) {
#pragma unroll
        for (int i = 0; i < PB; ++i) piece(i0 + i < npc ? i0 + i : npc - 1, vb[i]);
      }
#pragma unroll
      for (int i = 0; i < PB; ++i) {
        if (i0 + i >= npc) break;
        const float wi = weight(lse_of(i0 + i));
#pragma unroll
        for (int k = 0; k < PER; ++k) {
          if (i0 + i == 0) {
            o[k] = (f32x4){wi * vb[i][k][0], wi * vb[i][k][1], wi * vb[i][k][2], wi * vb[i][k][3]};
          } else {
            o[k][0] += wi * vb[i][k][0]; o[k][1] += wi * vb[i][k][1];
            o[k][2] += wi * vb[i][k][2]; o[k][3] += wi * vb[i][k][3];
          }
        }
      }
    }
  }
  if (!store || tok < 0 || tok >= a.total_tokens) return;
  T* orow = (T*)a.out + ((size_t)tok * a.num_heads + h) * DV + 4 * c0;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const i16x4 pk = {MfmaOps<T>::from_f32(o[k][0]), MfmaOps<T>::from_f32(o[k][1]),
                      MfmaOps<T>::from_f32(o[k][2]), MfmaOps<T>::from_f32(o[k][3])};
    *(i16x4*)(orow + 4 * TPH * k) = pk;
  }
  if (c0 == 0) a.lse[(size_t)tok * a.num_heads + h] = l;
}

// Tasks t = blockIdx.x, + gridDim.x, ... (one per workgroup column when the grid
// matches the task count; device-built schedules launch for the capacity).
template <int DV, typename T>
__global__ __launch_bounds__(MERGE_THREADS) void merge_kernel(const SasAttnArgs a) {
  int nfd = a.num_fd;
  if (nfd == SAS_SCHED_DEVICE) {
    if (!dev_sched_ok(a, a.m_base)) return;  // the attention kernel wrote NaN
    nfd = a.metadata[SAS_CFG_OFFSET + 3];
  }
  // Tasks in eight slices: column bx runs on XCD bx % 8 (workgroups go round-
  // robin over the 8 XCDs and the grid width is a multiple of 8) and takes the
  // tasks of slice bx % 8. The attention kernel keeps consecutive FA rows on
  // one XCD, so an evenly spread schedule leaves each slice's partials in that
  // XCD's L2.
  const int per = (nfd + 7) >> 3;
  const int cols = (int)gridDim.x >> 3;
  const int x = (int)blockIdx.x & 7;
  for (int j = (int)blockIdx.x >> 3; j < per; j += cols) {
    const int t = x * per + j;
    if (t < nfd) merge_task<DV, T>(a, t);
  }
}

template <int DQK, int NHG, typename T, int KVF>
static hipError_t launch_attn(const SasAttnArgs& a, hipStream_t st) {
  const int phases = a.phases == 0 ? 3 : a.phases;
  if (phases & 1) {
    const int per_xcd = (a.num_fa + 7) / 8;
    hipLaunchKernelGGL((attn_kernel<DQK, 512, NHG, T, KVF>), dim3(8 * per_xcd), dim3(256 * NHG),
                       0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const bool dev = a.num_fd == SAS_SCHED_DEVICE;
  if ((phases & 2) && (a.num_fd > 0 || dev)) {
    const int groups = (a.m_base + MERGE_HPB - 1) / MERGE_HPB;  // head groups per task (upper bound)
    const int tasks = dev ? (a.num_fa < 256 ? a.num_fa : 256) : a.num_fd;  // columns; tasks strided
    const int cols = (tasks + 7) / 8 * 8;  // a multiple of the 8 XCDs
    hipLaunchKernelGGL((merge_kernel<512, T>), dim3(cols, groups), dim3(MERGE_THREADS), 0, st, a);
    return hipGetLastError();
  }
  return hipSuccess;
}

// Items carry m_base = 32 or 64 heads (one or two 32-head groups of four
// dims-quarter waves): 4 or 8 waves, one or two per SIMD.
template <typename T>
static hipError_t dispatch_heads(const SasAttnArgs& a, hipStream_t st) {
  constexpr int NAT = SAS_KV_NATIVE;
  if (a.head_dim == 576)
    return a.m_base == 32 ? launch_attn<576, 1, T, NAT>(a, st) : launch_attn<576, 2, T, NAT>(a, st);
  return a.m_base == 32 ? launch_attn<512, 1, T, NAT>(a, st) : launch_attn<512, 2, T, NAT>(a, st);
}

// fp8 rows: head_dim 576, bf16 queries and outputs
static hipError_t dispatch_fp8(const SasAttnArgs& a, hipStream_t st) {
  constexpr int F8 = SAS_KV_FP8_DS_MLA;
  return a.m_base == 32 ? launch_attn<576, 1, __bf16, F8>(a, st)
                        : launch_attn<576, 2, __bf16, F8>(a, st);
}

}  // namespace sas

extern "C" int sas_attention_launch(const SasAttnArgs* a, void* stream) {
  using sas::set_error;
  if (!a) {
    set_error("sas_attention_launch: null args");
    return SAS_E_INVALID;
  }
  if (!a->q || !a->ori_kv || !a->ori_block_table || !a->q_prefix || !a->act_q_lens ||
      !a->seqused_kv || !a->sinks || !a->metadata || !a->out || !a->lse) {
    set_error("sas_attention_launch: null tensor pointer");
    return SAS_E_INVALID;
  }
  if (a->head_dim != 512 && a->head_dim != 576) {
    set_error("sas_attention_launch: head_dim must be 512 or 576");
    return SAS_E_UNSUPPORTED;
  }
  if (a->head_dim_v != 512) {
    set_error("sas_attention_launch: head_dim_v must be 512");
    return SAS_E_UNSUPPORTED;
  }
  if (a->num_heads < 1 || a->num_heads > 128 || (a->num_heads % 16) != 0) {
    set_error("sas_attention_launch: num_heads must be a multiple of 16 in [16, 128]");
    return SAS_E_UNSUPPORTED;
  }
  if ((a->m_base != 32 && a->m_base != 64) || (a->num_heads <= 32 && a->m_base != 32) ||
      (a->num_heads > 32 && a->m_base != 64)) {
    set_error("sas_attention_launch: m_base must be 32 for <= 32 heads, else 64");
    return SAS_E_INVALID;
  }
  if (a->scenario < 1 || a->scenario > 3 || (a->scenario >= 2 && (!a->cmp_kv ||
      !a->cmp_block_table || a->cmp_ratio < 1)) || (a->scenario == 3 && (!a->cmp_indices ||
      a->topk < 0))) {
    set_error("sas_attention_launch: scenario inputs missing");
    return SAS_E_INVALID;
  }
  if (a->phases < 0 || a->phases > 3) {
    set_error("sas_attention_launch: phases must be 0..3");
    return SAS_E_INVALID;
  }
  const bool dev_sched = a->num_fd == SAS_SCHED_DEVICE;
  if (a->num_fa < 1 || a->num_fa > SAS_AIC_CORE_NUM || (a->num_fd < 0 && !dev_sched) ||
      a->num_fd > SAS_AIV_CORE_NUM || a->s2_base < 32 || (a->s2_base % 32) != 0 ||
      ((a->num_fd > 0 || dev_sched) && (!a->workspace || a->num_partial_slots < 1))) {
    set_error("sas_attention_launch: inconsistent schedule");
    return SAS_E_INVALID;
  }
  if (a->ori_block_num < 1 || a->ori_block_size < 1 || a->ori_table_len < 1 || a->batch < 0 ||
      a->total_tokens < 0 || (a->scenario >= 2 && (a->cmp_block_num < 1 ||
      a->cmp_block_size < 1 || a->cmp_table_len < 1))) {
    set_error("sas_attention_launch: bad cache geometry");
    return SAS_E_INVALID;
  }
  if ((int64_t)a->ori_block_num * a->ori_block_size >= (1ll << 31) ||
      (int64_t)a->cmp_block_num * a->cmp_block_size >= (1ll << 31)) {
    set_error("sas_attention_launch: more than 2^31 cache rows");
    return SAS_E_UNSUPPORTED;
  }
  if (a->kv_format != SAS_KV_NATIVE && a->kv_format != SAS_KV_FP8_DS_MLA) {
    set_error("sas_attention_launch: unknown kv_format");
    return SAS_E_INVALID;
  }
  if (a->kv_format == SAS_KV_FP8_DS_MLA && (a->head_dim != 576 || a->dtype != SAS_DTYPE_BF16)) {
    set_error("sas_attention_launch: fp8 cache rows need head_dim 576 and bf16 queries");
    return SAS_E_UNSUPPORTED;
  }
  if (a->batch == 0 || a->total_tokens == 0) return SAS_OK;
  hipStream_t st = (hipStream_t)stream;
  hipError_t e = a->kv_format == SAS_KV_FP8_DS_MLA ? sas::dispatch_fp8(*a, st)
                 : a->dtype == SAS_DTYPE_FP16      ? sas::dispatch_heads<_Float16>(*a, st)
                                                   : sas::dispatch_heads<__bf16>(*a, st);
  if (e != hipSuccess) {
    set_error(std::string("sas_attention_launch: ") + hipGetErrorString(e));
    return SAS_E_HIP;
  }
  return SAS_OK;
}

extern "C" int sas_version(void) { return 110; }

extern "C" int sas_args_struct_size(void) { return (int)sizeof(SasAttnArgs); }

extern "C" const char* sas_last_error(void) { return sas::g_last_error.c_str(); }
