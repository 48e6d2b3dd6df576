// Causal varlen prefill attention for gfx950 on bf16/f16 MFMA.
//
// Reference semantics: layers/attention.py:64-70 calls
// flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
// max_seqlen_k, softmax_scale, causal=True, block_table): sequence s owns query
// rows [cu_q[s], cu_q[s+1]) and Lk = cu_k[s+1]-cu_k[s] keys; query row i sees
// keys j <= i + (Lk - Lq) (causal mask aligned to the bottom-right corner, so
// a prefix-cache hit of P = Lk - Lq tokens is visible to every row).  With a
// block table (any prefix hit in the batch, engine/model_runner.py:275-276)
// K/V are the whole paged cache (layers/attention.py:65-66).
//
// One kernel, varlen_prefill_dma_kernel, for 16-bit and fp8 K/V at head_dim
// 128 and 256:
//  * Persistent workgroups (G4 <= 4 query heads of one kv head x row
//    blocks), resident on every CU and pulling work items from per-XCD
//    queues; K/V tiles of 32 keys are copied HBM -> LDS by the LDS DMA into
//    a ring (no VGPRs), the QK products of tile j+1 overlap the softmax of
//    tile j.  fp8 K/V stay codes in the ring: the operand reads take 8
//    codes per lane (ds_read_b64, ds_read_b64_tr_b8) and widen them in
//    registers.
//  * GQA sharing in LDS: the waves of a workgroup are query heads of the SAME
//    kv head, so every K/V tile staged in LDS serves all of them.
//  * A tile never crosses a cache block (block_size % 32 == 0), so one buffer
//    descriptor covers it and keys past the causal limit read as zeros.
//  * S^T = K . Q^T and O^T += V^T . P^T on v_mfma_f32_16x16x32 with Q in
//    registers; P stays in registers (the S^T accumulator layout is the PV
//    B-operand layout); V^T comes from the row-major tile through
//    ds_read_b64_tr_b16.  Chunks of a tile row are XOR-swizzled so the
//    operand reads are bank-conflict free.
//  * Online softmax in the log2 domain with lazy rescaling: O and l are only
//    rescaled when a row maximum grows by more than 2^8, so P <= 256.
#include <type_traits>

#include "nq_device.hpp"

namespace nq {
namespace {

constexpr int kKeys = 32;    // keys per LDS tile
constexpr float kRescale = 8.0f;  // log2 growth of a row max that forces a rescale
// Cost levels of the queue: key tiles per item, coarsened to at most this
// many.  Within a level the items of one sequence run together, so its K/V
// stays in the XCD's L2 for all of them; 16 levels keep the queue longest
// first in steps of 1/16 of the longest item.
constexpr int kQueueLevels = 16;
constexpr int kMaxSeqs = 1024;    // sequences whose bounds the persistent kernel keeps in LDS
constexpr int kQueueWords = 16;   // prefill workspace: 8 per-XCD counters + 1 finish counter (+ pad)

struct PrefillArgs {
  const uint8_t *q;
  int64_t q_rs, q_hs;  // bytes
  const uint8_t *k;
  const uint8_t *v;
  int64_t kv_rs;  // bytes per K/V row (token)
  const int32_t *cu_q;
  const int32_t *cu_k;
  const int32_t *block_tables;  // null: packed K/V
  int64_t bt_stride;
  int max_blocks;  // table width: entries past it are never read
  int num_blocks;  // clamped to INT32_MAX: block ids are int32
  uint8_t *out;
  int64_t o_rs, o_hs;  // bytes
  int Hq, Hkv, G, G4, quads, block_size, num_seqs, n_qtiles, max_seqlen_q, max_seqlen_k;
  int causal;
  float scale_log2;
  const float *k_scale;
  const float *v_scale;
  uint32_t *queue;  // persistent kernel: kQueueWords work counters (zero between calls)
  int pin;          // work groups pinned to XCDs (>= 8 groups)
  int by_cost;      // persistent kernel: 0 query-tile order; cost order over live items (num_seqs <= kMaxSeqs),
                    // 1 each item derived when taken, 2 read from a list built at launch
  int level_shift;  // cost level of an item: its key tiles >> level_shift (< n_levels)
  int n_levels;
  const uint8_t *gate;  // null, or Qwen3.5's output gate [total_q, Hq, D] (type of out)
  int64_t g_rs, g_hs;   // bytes
};

// Chunk swizzles of the 16-bit DMA kernel's LDS tiles (16-byte chunk c of
// key row r is stored at chunk c ^ swz(r)), one per tile because the two
// operand reads want different ones.  Measured with SQ_LDS_BANK_CONFLICT on
// gfx950 over all bit permutations of r: the K operand's ds_read_b128 (16
// rows x one chunk per 16 lanes) is conflict-free exactly when swizzle bit 0
// comes from row bit 0 or 1, the V^T operand's ds_read_b64_tr_b16 (rows
// 4vg..4vg+3 x 32 bytes) exactly when it comes from row bit 3; both halve
// the LDS throughput (2-way conflicts) otherwise.
__device__ inline int swz_k(int row) { return row & 15; }
__device__ inline int swz_v(int row) { return ((row & 7) << 1) | ((row >> 3) & 1); }
// fp8 code tiles (rows of D bytes): 8-byte piece c of key row r is stored at
// piece c ^ 2 swz8(r), i.e. 16-byte unit u at u ^ swz8(r).  Conflict-free
// (64 banks, 32 lanes a pass) for the K operand reads (rows m and m + 16 x
// pieces 4 kk + g) and for the V^T reads, whose 16-lane groups g address
// rows 4 g .. +3 and 16 + 4 g .. +3 (the key order of the P operand).  Row
// bit 4 enters only through b = bit 3 ^ bit 4, so row m + 16's pieces are
// row m's with bit 2 (D = 128) or bit 3 (D = 256) of the piece flipped.
template <int D>
__device__ inline int swz8(int row) {
  const int b = ((row >> 3) ^ (row >> 4)) & 1;
  return D == 128 ? (((row >> 1) & 3) | (b << 2)) : ((row & 7) | (b << 3));
}

// Groups u = s * n_y + y (kv-head slot y of sequence s) -- the work items
// that read the same K/V -- are pinned to XCD u % 8 (the hardware places
// workgroup L on XCD L % 8), so they share that XCD's L2; y varies fastest in
// u, so every XCD gets a share of every sequence and the XCDs stay balanced
// however the lengths vary.  Fewer than 8 groups: no pinning.
// Work items of the queues: n_x query tiles of each group, 8 equal queues
// when pinned.
inline int64_t work_grid(int64_t n_x, int64_t U) { return U >= 8 ? 8 * ((U + 7) / 8) * n_x : U * n_x; }

// 16-bit K/V: persistent workgroups fed by an LDS DMA ring.
//
// K/V tiles of 32 keys go HBM/L2 -> LDS directly (buffer loads to LDS, no
// VGPRs), into a ring of kSlots slots; copies run kAhead tiles ahead of the
// tile being computed.  Each of the NW waves copies 32/NW rows of K and of V
// per tile (1 KiB = 4 rows per load); it waits for its own copies (vmcnt)
// and one raw workgroup barrier per tile makes the whole tile visible.  The
// chunk swizzle of the LDS tile is produced by the source offset each lane
// fetches.
//
// Shapes (PShape): NW waves per workgroup, each wave QS x 16 query rows of
// one head, WPE waves per SIMD.  C = two independent 4-wave workgroups per
// CU, whose barriers, prologues and epilogues do not line up, so one's
// stalls overlap the other's work (measured faster than one 8-wave
// workgroup per CU); D = head_dim 256.
template <class T, int D>
struct DTile {
  static_assert(D == 128 || D == 256, "head_dim 128 or 256");
  static constexpr int NKK = D / 32;  // 32-dim slices of a QK product
  static constexpr int NJ = D / 16;   // 16-dim blocks of O
  static constexpr int ROWB = D * 2;
  static constexpr int TILE_B = kKeys * ROWB;   // 8 (16) KiB per K (or V) tile at head_dim 128 (256)
  static constexpr int SLOT_B = 2 * TILE_B;     // K + V
};

// Launch shape of the 16-bit kernel: NW waves per workgroup, each QS x 16
// query rows of one head; WPE waves per SIMD (so WPE * 4 / NW resident
// workgroups per CU); a ring of SLOTS K/V tiles, copies SLOTS - 1 ahead.
// Two waves per SIMD: a wave owns at most 256 VGPRs.
template <int NW_, int QS_, int WPE_, int SLOTS_, int D_ = 128>
struct PShape {
  static constexpr int NW = NW_, QS = QS_, WPE = WPE_, SLOTS = SLOTS_, AHEAD = SLOTS_ - 1, D = D_;
  static constexpr int WG_PER_CU = WPE * 4 / NW;
  static constexpr int ITEM_ROWS = 16 * QS * NW;  // query rows x heads of one work item
  static constexpr int RING_BYTES = SLOTS * 2 * kKeys * 2 * D;
  // ring, queue item slots (4 words), queue size (4 words), cost-level
  // starts, sequence bounds (cu_q, cu_k), then the items of the queue listed
  // at launch (one packed word each: sequence << 22 | kv-head slot << 14 |
  // query tile) in what the CU's LDS has left, at most 4096
  static constexpr int FIXED_BYTES = RING_BYTES + 32 + 4 * kQueueLevels + 8 * (kMaxSeqs + 1);
  static constexpr int MAX_ITEMS = (160 * 1024 / WG_PER_CU - FIXED_BYTES) / 4 > 4096
                                       ? 4096
                                       : ((160 * 1024 / WG_PER_CU - FIXED_BYTES) / 4) & ~63;
  static constexpr int LDS_BYTES = FIXED_BYTES + 4 * MAX_ITEMS;
  static_assert(WPE == 2, "two waves per SIMD");
  static_assert(WG_PER_CU * LDS_BYTES <= 160 * 1024, "LDS of the resident workgroups");
};
using ShapeC = PShape<4, 2, 2, 4>;  // two independent workgroups per CU, 32-row waves
// head_dim 256: one workgroup per CU, two 16-row waves per SIMD (a 32 KiB
// ring slot; the 16-row wave keeps O, Q and a tile's operands in 256 VGPRs)
using ShapeD = PShape<8, 1, 2, 4, 256>;

// A work item of the persistent kernel: query tile qt (S::ITEM_ROWS/G4 rows
// of G4 heads) of kv-head slot y of sequence s, described by wave-uniform
// scalars.  `live` is false past the end of the queue and for query tiles
// past a sequence's rows.
struct Item {
  bool live;
  int s, kvh, head0, q0, Lq, k0, Lk, P, row_begin, key_end, n_kt;
};

// Item fields of query tile qt of kv-head slot y of sequence s.
// floor(n / d) for 0 <= n < 2^22 and 1 <= d < 2^22 without the integer
// division sequence: the float estimate n * (1/d) is within one of the
// quotient (relative error below 2^-22), and one step each way corrects it.
__device__ __forceinline__ int small_div(int n, int d) {
  int q = static_cast<int>(static_cast<float>(n) * __builtin_amdgcn_rcpf(static_cast<float>(d)));
  if (q * d > n)
    --q;
  else if ((q + 1) * d <= n)
    ++q;
  return q;
}
__device__ __forceinline__ Item fill_item(const PrefillArgs &a, int s, int y, int qt, int rows, int q0, int Lq, int k0,
                                          int Lk) {
  Item it{};
  it.live = false;
  it.s = s;
  it.kvh = small_div(y, a.quads);
  it.head0 = it.kvh * a.G + (y - it.kvh * a.quads) * 4;
  it.q0 = q0;
  it.Lq = Lq;
  it.row_begin = qt * rows;
  if (it.row_begin >= Lq) return it;
  it.k0 = k0;
  it.Lk = Lk;
  it.P = Lk - Lq;
  const int row_last = min(it.row_begin + rows, Lq) - 1;
  it.key_end = a.causal ? max(0, min(Lk, row_last + it.P + 1)) : Lk;
  it.n_kt = (it.key_end + kKeys - 1) / kKeys;
  it.live = true;
  return it;
}

// Queue order by query tile (used when the sequence bounds do not fit in
// LDS): XCD x's groups u = x, x + 8, ... (every group without pinning), from
// the last query tile down; items past a sequence's rows are not live.
template <class S>
__device__ __forceinline__ Item describe_by_tile(const PrefillArgs &a, int idx, int n_items, int n_x, int n_y, int cx,
                                                 int x) {
  Item it{};
  it.live = false;
  if (idx >= n_items) return it;
  const int qt = n_x - 1 - idx / cx;
  const int u = a.pin ? x + 8 * (idx % cx) : idx % cx;
  const int s = u / n_y;
  const int rows = 16 * S::QS * (S::NW / a.G4);
  const int q0 = ld_const(a.cu_q + s), k0 = ld_const(a.cu_k + s);
  return fill_item(a, s, u % n_y, qt, rows, q0, ld_const(a.cu_q + s + 1) - q0, k0, ld_const(a.cu_k + s + 1) - k0);
}

// Queue order by cost: the live items of XCD x's groups (see above), by
// cost level (key tiles >> level_shift) from the highest down, then by
// sequence, kv-head slot and query tile from the last down -- longest
// first, so the last items a workgroup takes are short ones, and no index
// is spent on an item without rows.  Each workgroup builds, at launch, the
// sequence bounds and a table of level starts in LDS and, when the queue's
// whole item list fits, that list (describe_by_table); otherwise each item
// is derived from the two when taken (describe_by_cost).
struct CostQueue {
  const int *lev;  // LDS: first queue index of each level
  const int *cuq;  // LDS: cu_seqlens_q, cu_seqlens_k
  const int *cuk;
  const uint32_t *tab;  // LDS: the queue's items in order (by_cost == 2)
  int x, n_y, rows, ystep;
  int rows_log2, ystep_log2;  // rows and ystep are powers of two
};
// Kv-head slots of sequence s in the queue: y0, y0 + ystep, ... < n_y.
__device__ __forceinline__ int first_slot(const CostQueue &cq, int s) {
  return cq.ystep == 8 ? ((cq.x - s * cq.n_y) & 7) : 0;
}
__device__ __forceinline__ int n_slots(const CostQueue &cq, int y0) {
  return y0 < cq.n_y ? ((cq.n_y - 1 - y0) >> cq.ystep_log2) + 1 : 0;
}
// Smallest query tile (of nq) whose item has at least v key tiles.
__device__ __forceinline__ int first_tile_with(const PrefillArgs &a, const CostQueue &cq, int v, int nq, int Lk,
                                               int P) {
  if (v <= 0) return 0;
  if (!a.causal) return (Lk + kKeys - 1) / kKeys >= v ? 0 : nq;
  const int t = kKeys * (v - 1);  // the item needs key_end > t (v <= n_levels << level_shift)
  if (Lk <= t) return nq;
  const int need = t - P;  // (qt + 1) * rows > need
  return need < 0 ? 0 : min(need >> cq.rows_log2, nq);
}
// Cost level of query tile qt of a sequence (as fill_item computes key_end).
__device__ __forceinline__ int cost_level(const PrefillArgs &a, const CostQueue &cq, int qt, int Lq, int Lk) {
  const int row_last = min((qt + 1) * cq.rows, Lq) - 1;
  const int key_end = a.causal ? max(0, min(Lk, row_last + Lk - Lq + 1)) : Lk;
  return min(((key_end + kKeys - 1) / kKeys) >> a.level_shift, a.n_levels - 1);
}
// Item at queue index idx.  Called by whole waves (all 64 lanes).
__device__ __forceinline__ Item describe_by_cost(const PrefillArgs &a, const CostQueue &cq, int idx, int n_items) {
  Item it{};
  it.live = false;
  if (idx >= n_items) return it;
  // The lane index from an instruction the compiler cannot hoist: addresses
  // derived from it are recomputed per call instead of being kept (or
  // spilled) across the tile loops.
  int lane;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane));
  const int nl = a.n_levels;
  // Level: the lowest L whose start is <= idx (starts fall as L rises).
  const int step = (nl + 63) / 64;
  const int l1 = min(lane * step, nl - 1);
  const int b = __builtin_amdgcn_readfirstlane(
      __builtin_popcountll(__builtin_amdgcn_ballot_w64(lane * step < nl && cq.lev[l1] > idx)));
  int L = 0;
  if (b > 0) {
    const int base = (b - 1) * step + 1;
    const int l2 = min(base + lane, nl - 1);
    L = base + __builtin_amdgcn_readfirstlane(
                   __builtin_popcountll(__builtin_amdgcn_ballot_w64(lane < step && base + lane < nl && cq.lev[l2] > idx)));
  }
  int r = idx - cq.lev[L];
  const int lo_v = L << a.level_shift;
  const bool top = L == nl - 1;  // the last level takes every item above it
  const int hi_v = (L + 1) << a.level_shift;
  // The sequence: items of level L in sequence order, 64 sequences per step.
  for (int base = 0; base < a.num_seqs; base += 64) {
    const int s = base + lane;
    int cnt = 0, qlo = 0, nqt = 0;
    if (s < a.num_seqs) {
      const int Lq = cq.cuq[s + 1] - cq.cuq[s], Lk = cq.cuk[s + 1] - cq.cuk[s];
      const int nq = Lq > 0 ? (Lq + cq.rows - 1) >> cq.rows_log2 : 0;
      qlo = first_tile_with(a, cq, lo_v, nq, Lk, Lk - Lq);
      const int qhi = top ? nq : first_tile_with(a, cq, hi_v, nq, Lk, Lk - Lq);
      nqt = max(0, qhi - qlo);
      cnt = nqt * n_slots(cq, first_slot(cq, s));
    }
    const int incl = wave_iscan(cnt);
    const int total = __builtin_amdgcn_readlane(incl, 63);
    if (r < total) {
      const int ls = __builtin_amdgcn_readfirstlane(
          static_cast<int>(__builtin_ctzll(__builtin_amdgcn_ballot_w64(incl > r))));
      const int s_it = base + ls;
      r -= __builtin_amdgcn_readlane(incl - cnt, ls);
      const int n_t = __builtin_amdgcn_readlane(nqt, ls);
      const int yi = small_div(r, n_t);
      const int qt = __builtin_amdgcn_readlane(qlo, ls) + n_t - 1 - (r - yi * n_t);
      const int y = first_slot(cq, s_it) + cq.ystep * yi;
      const int q0 = cq.cuq[s_it], k0 = cq.cuk[s_it];
      return fill_item(a, s_it, y, qt, cq.rows, q0, cq.cuq[s_it + 1] - q0, k0, cq.cuk[s_it + 1] - k0);
    }
    r -= total;
  }
  return it;  // not reached for idx < n_items
}

// Item at queue index idx from the list built at launch (by_cost == 2):
// one LDS read and the sequence bounds, instead of the search above.
__device__ __forceinline__ Item describe_by_table(const PrefillArgs &a, const CostQueue &cq, int idx, int n_items) {
  Item it{};
  it.live = false;
  if (idx >= n_items) return it;
  const uint32_t e = __builtin_amdgcn_readfirstlane(cq.tab[idx]);
  const int s = e >> 22, y = (e >> 14) & 255, qt = e & 16383;
  const int q0 = cq.cuq[s], k0 = cq.cuk[s];
  return fill_item(a, s, y, qt, cq.rows, q0, cq.cuq[s + 1] - q0, k0, cq.cuk[s + 1] - k0);
}

// Persistent prefill: S::WG_PER_CU workgroups per CU pull work items from
// per-XCD queues.  The hardware dispatcher keeps only about half of the CUs
// busy when one-per-CU workgroups of very different lengths are launched as
// a plain grid; a queue keeps every CU fed until the work runs out.
//
// Queue: items are grouped as described above work_grid -- XCD x (workgroups L with
// L % 8 == x) owns the groups u = x, x + 8, ... and serves them from its own
// counter queue[x], in query-tile order from the last tile down (longest
// first).  Thread 0 fetches two items ahead; indices reach the other waves
// through LDS, and each item is described (sequence bounds, keys, tiles) one
// item ahead.  queue[8] counts finished workgroups; the last one puts all
// nine words back to zero, so the workspace is ready for the next call.
//
// K/V copies form one stream across items: each stream entry is one 32-key
// tile (of the item being copied, or an empty load when none is queued)
// copied into ring slot (entry index mod SLOTS), kAhead entries ahead of the
// tile being computed.  While an item computes its last tiles, the stream is
// already copying the next item's first ones.  All copy control is scalar
// (wave-uniform): descriptors whose range ends at the tile's last valid key
// (rows past it read as zeros), the block table walked one block at a time
// with scalar loads, the next item's copy parameters set when it is queued.
//
// Per tile, after one barrier: the K reads of tile j+1, the lazy-rescale
// check of tile j, the next stream entry, the QK products of tile j+1
// interleaved with the exp / pack work of tile j, then O += P V of tile j.
// Tiles every row of a wave sees completely run a mask-free loop; the rest
// (the causal diagonal, the end of the keys, a missing block) the masked one.
// An item's output is stored at the start of the next one, right after that
// item's Q loads are issued, so the stores cover the Q latency.
//
// vmcnt accounting: each stream entry is 2 * COPS loads per wave, and the
// waits count only younger stream entries -- except that a new item's first
// kAhead tiles may precede the Q loads and the previous item's output stores
// (a fixed count per wave), which the waits then add.
template <class T, int D, class S, bool GATED, bool FP8, bool TAB>
__device__ __forceinline__ void prefill_persistent(const PrefillArgs &a) {
  using DT = DTile<T, D>;
  constexpr int NW = S::NW, QS = S::QS, kSlots = S::SLOTS, kAhead = S::AHEAD;
  constexpr int RW = 16 * QS;        // query rows per wave
  constexpr int CR = kKeys / NW;     // tile rows each wave copies
  constexpr int SRC_ROWB = FP8 ? D : 2 * D;  // bytes of one key of one kv head in the cache
  constexpr int COPS = CR * SRC_ROWB / 1024;  // 1 KiB loads per K (or V) per wave and entry
  constexpr int LPR = SRC_ROWB / 16;          // lanes per row in a copy (16 bytes each)
  // fp8: a tile's codes are packed rows of D bytes at the start of the K (V)
  // half of the slot, swizzled by swz8.
  static_assert(S::D == D, "launch shape built for this head_dim");
  static_assert(COPS >= 1 && CR * SRC_ROWB == 1024 * COPS, "a wave copies whole 1 KiB pieces");
  static_assert(!FP8 || COPS == 1, "fp8: one 1 KiB copy of codes per K (or V) per wave");
  constexpr int QOPS = QS * DT::NKK;        // Q loads per wave and item
  constexpr int SOPS = QS * (DT::NJ / 2);   // output stores per wave and item
  // Stores that write nothing, after the Q loads: the compiler counts them
  // (it does not see the K/V copies), so one wait for at most kPad
  // operations shows it -- as it holds on the hardware, where at least these
  // kPad follow the Q loads -- that Q and the queue fetch before them are
  // complete, without a wait for the copies in flight.
  constexpr int kPad = 2 * COPS * kAhead;
  constexpr int EOPS = QOPS + SOPS + kPad;
  static_assert(CR % 4 == 0, "a copy moves whole groups of 4 rows");
  static_assert(2 * COPS * kAhead + EOPS < 64, "vmcnt range");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  static_assert(S::RING_BYTES == kSlots * DT::SLOT_B, "ring size");
  int *lds_item = reinterpret_cast<int *>(smem + S::RING_BYTES);  // fetched queue indices
  int *lds_n = lds_item + 4;                                      // queue size (cost order)
  int *lds_lev = lds_item + 8;                                    // level starts (cost order)
  int *lds_cuq = lds_lev + kQueueLevels;
  int *lds_cuk = lds_cuq + kMaxSeqs + 1;
  uint32_t *lds_tab = reinterpret_cast<uint32_t *>(lds_cuk + kMaxSeqs + 1);  // the queue's items

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int m = lane & 15, g = lane >> 4;
  // log2(e) x the softmax scale; with fp8 K also x the item's K scale (the
  // products are formed from the unscaled codes)
  float sl2 = a.scale_log2;
  const bool paged = a.block_tables != nullptr;
  const int row_in_item = RW * (wave / a.G4);  // this wave's first row within an item
  const int head_in_item = wave % a.G4;

  const int n_x = a.n_qtiles, n_y = a.Hkv * a.quads;
  const int U = n_y * a.num_seqs;
  const int x = a.pin ? static_cast<int>(blockIdx.x & 7) : 0;
  const int cx = a.pin ? (U - x + 7) >> 3 : U;
  uint32_t *ctr = a.queue + x;
  const int item_rows = 16 * QS * (NW / a.G4);
  const CostQueue cq{lds_lev, lds_cuq,   lds_cuk, lds_tab, x, n_y, item_rows, a.pin ? 8 : 1, 31 - __builtin_clz(item_rows),
                     a.pin ? 3 : 0};
  if (a.by_cost) {
    // Sequence bounds into LDS, then the live items of this queue counted
    // per cost level, then each level's first index (highest level first).
    for (int i = threadIdx.x; i <= a.num_seqs; i += blockDim.x) {
      lds_cuq[i] = a.cu_q[i];
      lds_cuk[i] = a.cu_k[i];
    }
    for (int i = threadIdx.x; i < a.n_levels; i += blockDim.x) lds_lev[i] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < a.num_seqs * n_x; i += blockDim.x) {
      const int sq = i / n_x, qt = i - sq * n_x;
      const int Lq = lds_cuq[sq + 1] - lds_cuq[sq];
      const int w = n_slots(cq, first_slot(cq, sq));
      if (qt * cq.rows < Lq && w > 0)
        atomicAdd(&lds_lev[cost_level(a, cq, qt, Lq, lds_cuk[sq + 1] - lds_cuk[sq])], w);
    }
    __syncthreads();
    if (wave == 0) {
      int carry = 0;
      for (int top = a.n_levels - 1; top >= 0; top -= 64) {
        const int L = top - lane;
        const int c = L >= 0 ? lds_lev[L] : 0;
        const int incl = wave_iscan(c);
        if (L >= 0) lds_lev[L] = carry + incl - c;
        carry += __builtin_amdgcn_readlane(incl, 63);
      }
      if (lane == 0) *lds_n = carry;
    }
    if constexpr (TAB) {
      // The queue's items listed in order.  First the queue index of each
      // (level, sequence)'s first item -- a level's sequences in order --
      // kept in the ring, which no copy has written yet; then every live
      // (sequence, query tile) writes its items (one per kv-head slot) at
      // their places: sequence, slot, then query tile from the last down.
      int *first = reinterpret_cast<int *>(smem);
      __syncthreads();
      for (int L = wave; L < a.n_levels; L += NW) {
        const int lo_v = L << a.level_shift, hi_v = (L + 1) << a.level_shift;
        int carry = lds_lev[L];
        for (int base = 0; base < a.num_seqs; base += 64) {
          const int s = base + lane;
          int cnt = 0;
          if (s < a.num_seqs) {
            const int Lq = lds_cuq[s + 1] - lds_cuq[s], Lk = lds_cuk[s + 1] - lds_cuk[s];
            const int nq = Lq > 0 ? (Lq + cq.rows - 1) >> cq.rows_log2 : 0;
            const int qlo = first_tile_with(a, cq, lo_v, nq, Lk, Lk - Lq);
            const int qhi = L == a.n_levels - 1 ? nq : first_tile_with(a, cq, hi_v, nq, Lk, Lk - Lq);
            cnt = max(0, qhi - qlo) * n_slots(cq, first_slot(cq, s));
          }
          const int incl = wave_iscan(cnt);
          if (s < a.num_seqs) first[L * a.num_seqs + s] = carry + incl - cnt;
          carry += __builtin_amdgcn_readlane(incl, 63);
        }
      }
      __syncthreads();
      for (int i = threadIdx.x; i < a.num_seqs * n_x; i += blockDim.x) {
        const int sq = i / n_x, qt = i - sq * n_x;
        const int Lq = lds_cuq[sq + 1] - lds_cuq[sq], Lk = lds_cuk[sq + 1] - lds_cuk[sq];
        const int y0 = first_slot(cq, sq), w = n_slots(cq, y0);
        if (qt * cq.rows < Lq && w > 0) {
          const int L = cost_level(a, cq, qt, Lq, Lk);
          const int nq = (Lq + cq.rows - 1) >> cq.rows_log2;
          const int qlo = first_tile_with(a, cq, L << a.level_shift, nq, Lk, Lk - Lq);
          const int qhi = L == a.n_levels - 1 ? nq : first_tile_with(a, cq, (L + 1) << a.level_shift, nq, Lk, Lk - Lq);
          int pos = first[L * a.num_seqs + sq] + (qhi - 1 - qt);
          for (int yi = 0; yi < w; ++yi, pos += qhi - qlo)
            lds_tab[pos] = (static_cast<uint32_t>(sq) << 22) | (static_cast<uint32_t>(y0 + cq.ystep * yi) << 14) | qt;
        }
      }
      __syncthreads();  // the list is complete, and the ring free for the copies
    }
  }

  // ---------------------------------------------------------------- stream
  // Copy-stream arguments in registers of their own (the host bounds the
  // row stride by 1 MiB, so byte counts of a tile fit 32 bits).
  const uint8_t *const kbase = own_sgpr(a.k);
  const int64_t v_minus_k = own_sgpr(static_cast<int64_t>(a.v - a.k));
  const int kv_rs = own_sgpr(static_cast<int>(a.kv_rs));
  const int tile_bytes = kKeys * kv_rs;
  const int64_t blk_bytes = own_sgpr(static_cast<int64_t>(a.block_size) * a.kv_rs);
  const int num_blocks = own_sgpr(a.num_blocks);
  const int max_blocks = own_sgpr(a.max_blocks);
  const int tiles_per_blk = paged ? a.block_size / kKeys : 0x40000000;
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
      (__attribute__((address_space(3))) uint8_t *)(smem)));
  const uint32_t lds_last = lds0 + (kSlots - 1) * DT::SLOT_B;  // the last ring slot
  // The stream issues runs of entries that share a descriptor shape: a run
  // ends at a block boundary, before an item's partial last tile, at the end
  // of an item, or after one empty entry.  Per entry the common path only
  // counts down, advances the source address and the ring slot, and issues
  // the copies; the rest happens once per run (next_run).
  int st_pos = 0;                   // entries issued so far
  int run_left = 0;                 // entries left in the current run
  const uint8_t *st_src = kbase;    // K source of the next entry (its row 0, at the item's kv head)
  uint32_t st_nrec = 0;             // bytes each copy of the run may read (0: rows read as zeros)
  uint32_t st_dst = lds0;           // ring slot of the next entry
  int st_rem = 0;                   // keys of the item being copied not yet in a run
  int st_left = 0, st_bidx = 0, st_blk_next = 0;  // paged: tiles left in the block, next entry and its value
  int st_head = 0;                  // byte offset of the item's kv head within a row
  const int32_t *st_bt = nullptr;
  // The item queued to be copied next, in the form the stream takes over.
  int nx_rem = 0;       // its keys (0: none queued)
  int nx_head = 0;      // its kv head's byte offset within a row
  int64_t nx_base = 0;  // paged: address of its block-table row; packed: byte offset of its first key
  int nx_blk0 = 0;      // paged: its first block-table entry
  int nx_first = 0;     // stream index of the queued item's first tile, once started
  // A copied tile lay in a missing block: from then on every tile takes the
  // masked path (which checks its block); plain_end bounds the current
  // item's mask-free loop.
  int bad_seen = 0, plain_end = 0;
  // This wave's rows of a tile and its 16-byte pieces (the kv head's offset
  // is in the source address).
  // fp8: 16 codes per lane, the 16-byte units of a row swizzled by swz8.
  uint32_t src_k[COPS], src_v[COPS];
#pragma unroll
  for (int c = 0; c < COPS; ++c) {
    if constexpr (FP8) {
      // lane l lands in unit l % LPR of row drow: it loads the unit swz8 puts there
      const int drow = CR * wave + lane / LPR;
      src_k[c] = src_v[c] = static_cast<uint32_t>(drow * kv_rs + (((lane % LPR) ^ swz8<D>(drow)) << 4));
    } else {
      const int drow = CR * wave + (64 / LPR) * c + lane / LPR;
      const uint32_t row_off = static_cast<uint32_t>(drow * kv_rs);
      src_k[c] = row_off + (((lane % LPR) ^ swz_k(drow)) << 4);
      src_v[c] = row_off + (((lane % LPR) ^ swz_v(drow)) << 4);
    }
  }
  // Block-table entry bidx of a sequence's row (paged only).
  auto blk_entry = [&](const int32_t *bt, int bidx) { return bidx < max_blocks ? ld_const(bt + bidx) : -1; };
  auto queue_copy = [&](const Item &it) {
    nx_rem = (it.live && it.n_kt > 0) ? it.key_end : 0;
    nx_head = it.kvh * SRC_ROWB;
    if (paged) {
      const int32_t *bt = a.block_tables + static_cast<int64_t>(it.s) * a.bt_stride;
      nx_base = static_cast<int64_t>(reinterpret_cast<uintptr_t>(bt));
      nx_blk0 = nx_rem > 0 ? blk_entry(bt, 0) : 0;
    } else {
      nx_base = static_cast<int64_t>(it.k0) * kv_rs + nx_head;
    }
  };
  // Sets up the next run (run_left == 0 on entry).
  auto next_run = [&]() {
    if (st_rem <= 0 && nx_rem > 0) {  // start the queued item
      st_rem = nx_rem;
      nx_rem = 0;
      st_head = nx_head;
      st_bt = paged ? reinterpret_cast<const int32_t *>(static_cast<uintptr_t>(nx_base)) : nullptr;
      st_src = kbase + (paged ? 0 : nx_base);
      st_blk_next = nx_blk0;
      st_bidx = 0;
      st_left = paged ? 0 : 0x40000000;
      nx_first = st_pos;
    }
    if (st_rem <= 0) {  // nothing to copy: one empty entry
      st_nrec = 0;
      run_left = 1;
      return;
    }
    bool ok = true;
    if (st_left == 0) {  // entering the next block (paged)
      const int blk = st_blk_next;
      st_blk_next = blk_entry(st_bt, st_bidx + 1);  // used a block from now
      ++st_bidx;
      ok = blk >= 0 && blk < num_blocks;
      if (!ok) {
        bad_seen = 1;
        plain_end = 0;
      }
      st_src = kbase + static_cast<int64_t>(ok ? blk : 0) * blk_bytes + st_head;
      st_left = tiles_per_blk;
    } else if (paged) {
      ok = st_nrec != 0;  // the same block as the previous run
    }
    const int full = min(st_left, st_rem / kKeys);  // whole tiles left in the block and the item
    if (full > 0) {
      run_left = full;
      st_left -= full;
      st_rem -= full * kKeys;
      st_nrec = ok ? static_cast<uint32_t>(tile_bytes) : 0u;
    } else {  // the item's partial last tile
      run_left = 1;
      st_left -= 1;
      st_nrec = ok ? static_cast<uint32_t>(st_rem * kv_rs) : 0u;
      st_rem = 0;
    }
  };
  auto issue = [&]() {
    if (run_left == 0) next_run();
    const uint32_t dst = st_dst + wave * (CR * SRC_ROWB);
    const u32x4 rk = rsrc_words(st_src, st_nrec);
    const u32x4 rv = rsrc_words(st_src + v_minus_k, st_nrec);
#pragma unroll
    for (int c = 0; c < COPS; ++c) {
      dma16_opaque(dst + 1024 * c, rk, src_k[c]);
      dma16_opaque(dst + DT::TILE_B + 1024 * c, rv, src_v[c]);
    }
    st_src += tile_bytes;
    st_dst = st_dst == lds_last ? lds0 : st_dst + DT::SLOT_B;
    --run_left;
    ++st_pos;
  };
  // ------------------------------------------------------- operand offsets
  // K^T operand kk: key row m (row m + 16 is +16 rows), dims 32kk + 8g.. ;
  // V^T operand j: rows r0 and r0 + 16 (both swizzles ignore row bit 4).
  // The byte offset of operand kk is m * ROWB + (((4kk + g) ^ swz_k(m)) << 4)
  // = kbase_l + ((kk << 6) ^ kx_l), and that of operand j is
  // r0 * ROWB + (((2j + (vq >> 1)) ^ swz_v(r0)) << 4) + 8 (vq & 1)
  // = vbase_l + ((j << 5) ^ vx_l): the operand index only meets the swizzle's
  // upper bits, so two registers per lane give every offset (one
  // xor-and-add per read).  unhoist() keeps the compiler from turning them
  // back into one loop-invariant register per operand.
  // fp8 code tiles (rows of D bytes, swz8): K^T operand kk of rows m is piece
  // 4kk + g at (((4kk + g) ^ 2 swz8(m)) << 3) = kbase_l + ((kk << 5) ^ kx_l),
  // that of rows m + 16 operand kk ^ KF's offset + 16 rows; V^T operand j:
  // lane (g, rho = (l & 15) >> 1, p = l & 1) addresses row R = 4g + rho
  // (rho < 4) or 16 + 4g + rho - 4, piece 2j + p: vbase_l + ((j << 4) ^ vx_l).
  uint32_t kbase_l, kx_l, vbase_l, vx_l;
  if constexpr (FP8) {
    const int s8 = 2 * swz8<D>(m);
    kbase_l = m * D + ((g ^ (s8 & 3)) << 3);
    kx_l = (s8 & ~3) << 3;
    const int rho = (lane & 15) >> 1, vp = lane & 1;
    const int r = rho < 4 ? 4 * g + rho : 12 + 4 * g + rho;
    vbase_l = r * D + (vp << 3);
    vx_l = (2 * swz8<D>(r)) << 3;
  } else {
    kbase_l = m * DT::ROWB + ((g ^ (swz_k(m) & 3)) << 4);
    kx_l = (swz_k(m) & 12) << 4;
    const int vg = lane >> 4, vk = (lane >> 2) & 3, vq = lane & 3;
    const int r0 = 4 * vg + vk;
    vbase_l = r0 * DT::ROWB + (((vq >> 1) ^ (swz_v(r0) & 1)) << 4) + (vq & 1) * 8;
    vx_l = (swz_v(r0) & 14) << 4;
  }
  // eight fp8 codes -> eight 16-bit values (exact: every e4m3 value is a bf16
  // and an f16 value; the scales are applied to the scores and the output)
  auto widen8 = [](const u32x2 &w) {
    return u32x4{T::template fp8x2<false>(w[0]), T::template fp8x2<true>(w[0]), T::template fp8x2<false>(w[1]),
                 T::template fp8x2<true>(w[1])};
  };
  // K^T and V^T operands as read from LDS: 16-bit values, or fp8 codes that
  // are widened just before their products (op), so that a read has a whole
  // section of products to land in and the conversions sit between products.
  using KV = std::conditional_t<FP8, u32x2, u32x4>;
  auto op = [&](const KV &x) -> u32x4 {
    if constexpr (FP8)
      return widen8(x);
    else
      return x;
  };
  auto unhoist = [&]() { asm volatile("" : "+v"(kx_l), "+v"(vx_l)); };

  // Q operands of an item for this wave: always QOPS loads, so the count the
  // waits add is fixed.  A row past the sequence (or of an item past the
  // queue) loads an existing row instead; its scores and output are computed
  // but never stored, and nothing selects on the loaded values, which would
  // make the compiler wait for them -- and for every K/V copy in flight.
  u32x4 qf[QS][DT::NKK];
  auto load_q = [&](const Item &it) {
    const int head = it.live ? it.head0 + head_in_item : 0;
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) {
      const int r = it.row_begin + row_in_item + 16 * qs + m;
      const int row = (it.live && r < it.Lq) ? it.q0 + r : it.q0;
      const uint8_t *qp = a.q + static_cast<int64_t>(row) * a.q_rs + static_cast<int64_t>(head) * a.q_hs;
#pragma unroll
      for (int kk = 0; kk < DT::NKK; ++kk) qf[qs][kk] = load16(qp + (8 * g + 32 * kk) * 2);
    }
  };

  f32x4 o[QS][DT::NJ];  // O^T accumulators of the item computed last
  float lsum[QS];       // its row sums of P: this lane's keys (the four lanes of a row add up at the store)
#pragma unroll
  for (int qs = 0; qs < QS; ++qs) {
    lsum[qs] = 0.f;
#pragma unroll
    for (int j = 0; j < DT::NJ; ++j) o[qs][j] = f32x4{0, 0, 0, 0};
  }
  // Output of an item: SOPS stores per wave.  Lane (g, m) holds dims
  // 16j + 4g .. +3 of row m for every j.  The lanes of lane groups g and g^1
  // (same row) trade one 8-byte piece per pair of j through permlane16_swap,
  // so each writes 16 contiguous bytes: even g dims 16j0 + 4g .. +7, odd g
  // dims 16j1 + 4(g-1) .. +7 (j0 = 2p, j1 = 2p + 1).  The stores go through a
  // descriptor covering the sequence's rows of this head, so rows past the
  // end (and a wave with no rows) are dropped by the range check, not skipped.
  auto store_out_plain = [&](const Item &it) {
    const bool odd = (g & 1) != 0;
    const float vscale = FP8 ? ld_const(a.v_scale + it.kvh) : 1.f;  // fp8: V's scale (P V from the codes)
    const int wrow0 = it.row_begin + row_in_item;
    const int head = it.head0 + head_in_item;
    const uint8_t *obase = a.out + static_cast<int64_t>(it.q0) * a.o_rs + static_cast<int64_t>(head) * a.o_hs;
    const uint32_t orange = wrow0 < it.Lq ? static_cast<uint32_t>((it.Lq - 1) * a.o_rs + D * 2) : 0u;
    const auto ro = make_rsrc(obase, orange);
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) {
      const float l = sum32(sum16(lsum[qs]));  // the row sum of row m (lanes m, m + 16, m + 32, m + 48)
      const int row = wrow0 + 16 * qs + m;
      const float inv = (l > 0.f ? 1.0f / l : 0.f) * vscale;
      const uint32_t roff = row < it.Lq ? static_cast<uint32_t>(row * a.o_rs) : 0x7fffffffu;
#pragma unroll
      for (int p = 0; p < DT::NJ / 2; ++p) {
        const f32x4 v0 = o[qs][2 * p] * inv, v1 = o[qs][2 * p + 1] * inv;
        const uint32_t c00 = T::pack2(v0[0], v0[1]), c01 = T::pack2(v0[2], v0[3]);
        const uint32_t c10 = T::pack2(v1[0], v1[1]), c11 = T::pack2(v1[2], v1[3]);
        const uint32_t x0 = odd ? c00 : c10, x1 = odd ? c01 : c11;  // the piece the partner needs
        // After the swap, even lanes find the partner's value in the
        // second result, odd lanes in the first.
        const auto r0 = __builtin_amdgcn_permlane16_swap(x0, x0, false, false);
        const auto r1 = __builtin_amdgcn_permlane16_swap(x1, x1, false, false);
        const uint32_t y0 = odd ? static_cast<uint32_t>(r0[0]) : static_cast<uint32_t>(r0[1]);
        const uint32_t y1 = odd ? static_cast<uint32_t>(r1[0]) : static_cast<uint32_t>(r1[1]);
        const int dim0 = odd ? 16 * (2 * p + 1) + 4 * (g - 1) : 16 * (2 * p) + 4 * g;
        const u32x4 w = odd ? u32x4{y0, y1, c10, c11} : u32x4{c00, c01, y0, y1};
        const uint32_t voff_o = roff == 0x7fffffffu ? roff : roff + dim0 * 2;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, w),
                                               ro, static_cast<int>(voff_o), 0, 0);
      }
    }
  };

  auto store_out_gated = [&](const Item &it) {
    const bool odd = (g & 1) != 0;
    const float vscale = FP8 ? ld_const(a.v_scale + it.kvh) : 1.f;  // fp8: V's scale (P V from the codes)
    const int wrow0 = it.row_begin + row_in_item;
    const int head = it.head0 + head_in_item;
    const uint8_t *obase = a.out + static_cast<int64_t>(it.q0) * a.o_rs + static_cast<int64_t>(head) * a.o_hs;
    const uint32_t orange = wrow0 < it.Lq ? static_cast<uint32_t>((it.Lq - 1) * a.o_rs + D * 2) : 0u;
    const auto ro = make_rsrc(obase, orange);
    // Output dims [dim0, dim0 + 8) of a lane for store p (after the swap below).
    auto dim0_of = [&](int p) { return odd ? 16 * (2 * p + 1) + 4 * (g - 1) : 16 * (2 * p) + 4 * g; };
    // Gated output (models/qwen3_5.py:140-142): the gate's 16 bytes at each
    // store's address, loaded for one 16-row block before its products.
    const uint8_t *gbase = nullptr;
    uint32_t grange = 0;
    if constexpr (GATED) {
      gbase = a.gate + static_cast<int64_t>(it.q0) * a.g_rs + static_cast<int64_t>(head) * a.g_hs;
      grange = wrow0 < it.Lq ? static_cast<uint32_t>((it.Lq - 1) * a.g_rs + D * 2) : 0u;
    }
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) {
      const float l = sum32(sum16(lsum[qs]));  // the row sum of row m (lanes m, m + 16, m + 32, m + 48)
      const int row = wrow0 + 16 * qs + m;
      u32x4 gv[DT::NJ / 2];
      if constexpr (GATED) {
        const auto rg = make_rsrc(gbase, grange);
#pragma unroll
        for (int p = 0; p < DT::NJ / 2; ++p) {
          const uint32_t goff = row < it.Lq ? static_cast<uint32_t>(row * a.g_rs + dim0_of(p) * 2) : 0x7fffffffu;
          gv[p] = buffer_load16_nt(rg, static_cast<int>(goff));
        }
      }
      const float inv = (l > 0.f ? 1.0f / l : 0.f) * vscale;
      const uint32_t roff = row < it.Lq ? static_cast<uint32_t>(row * a.o_rs) : 0x7fffffffu;
#pragma unroll
      for (int p = 0; p < DT::NJ / 2; ++p) {
        const f32x4 v0 = o[qs][2 * p] * inv, v1 = o[qs][2 * p + 1] * inv;
        const uint32_t c00 = T::pack2(v0[0], v0[1]), c01 = T::pack2(v0[2], v0[3]);
        const uint32_t c10 = T::pack2(v1[0], v1[1]), c11 = T::pack2(v1[2], v1[3]);
        const uint32_t x0 = odd ? c00 : c10, x1 = odd ? c01 : c11;  // the piece the partner needs
        // After the swap, even lanes find the partner's value in the
        // second result, odd lanes in the first.
        const auto r0 = __builtin_amdgcn_permlane16_swap(x0, x0, false, false);
        const auto r1 = __builtin_amdgcn_permlane16_swap(x1, x1, false, false);
        const uint32_t y0 = odd ? static_cast<uint32_t>(r0[0]) : static_cast<uint32_t>(r0[1]);
        const uint32_t y1 = odd ? static_cast<uint32_t>(r1[0]) : static_cast<uint32_t>(r1[1]);
        u32x4 w = odd ? u32x4{y0, y1, c10, c11} : u32x4{c00, c01, y0, y1};
        if constexpr (GATED) {
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const float o0 = T::to_float(static_cast<uint16_t>(w[t] & 0xffffu));
            const float o1 = T::to_float(static_cast<uint16_t>(w[t] >> 16));
            w[t] = T::pack2(gate_one<T>(o0, gv[p][t] & 0xffffu), gate_one<T>(o1, gv[p][t] >> 16));
          }
        }
        const uint32_t voff_o = roff == 0x7fffffffu ? roff : roff + dim0_of(p) * 2;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, w),
                                               ro, static_cast<int>(voff_o), 0, 0);
      }
    }
  };

  auto store_out = [&](const Item &it) {
    if constexpr (GATED) store_out_gated(it);
    else store_out_plain(it);
  };

  // ----------------------------------------------------------------- queue
  if (threadIdx.x == 0) {
    lds_item[0] = static_cast<int>(atomicAdd(ctr, 1u));
    lds_item[1] = static_cast<int>(atomicAdd(ctr, 1u));
  }
  __syncthreads();
  const int n_items = a.by_cost ? __builtin_amdgcn_readfirstlane(*lds_n) : cx * n_x;
  auto describe = [&](int idx) {
    if constexpr (TAB) return describe_by_table(a, cq, idx, n_items);
    else return a.by_cost ? describe_by_cost(a, cq, idx, n_items) : describe_by_tile<S>(a, idx, n_items, n_x, n_y, cx, x);
  };
  int idx_cur = __builtin_amdgcn_readfirstlane(lds_item[0]);
  int idx_nxt = __builtin_amdgcn_readfirstlane(lds_item[1]);
  Item cur = describe(idx_cur);
  // The next item: described one ahead and kept, or -- from the list, where
  // describing is cheap -- described again where it is used, so its fields
  // hold no registers through the tile loops.  Measured with the list:
  // describing again is faster at head_dim 128 (cfg3_long -1%, fp8 K/V -0.4%,
  // 96 fewer scalar spills), keeping the item at 256 (-3%).
  constexpr bool kRedescribe = TAB && D == 128;
  Item nxt{};
  if constexpr (!kRedescribe) nxt = describe(idx_nxt);
  auto next_item = [&]() -> Item {
    if constexpr (kRedescribe) return describe(idx_nxt);
    else return nxt;
  };
  Item prev{};  // the item whose output is still in o / lsum
  prev.live = false;
  queue_copy(cur);

  for (int k = 0;; ++k) {
    // The previous item's output, then this item's Q -- loaded at one place
    // only: Q is not carried around the loop, so the compiler never copies
    // (and waits for) loaded registers; and the output registers are free
    // before the Q registers fill.
    int epi_pos = -1;  // stream entries before this index precede the Q loads and stores just issued
    if (prev.live) {
      store_out(prev);
      epi_pos = st_pos;
    }
    if (idx_cur >= n_items) break;
    // Thread 0 fetches item k + 2.  The Q loads issued after it let the
    // compiler's own wait for the result (at the end of the item) count
    // them; the copies in flight then need not complete.
    uint32_t fetched;
    if (threadIdx.x == 0) fetched = atomicAdd(ctr, 1u);
    load_q(cur);
    asm volatile("" ::: "memory");  // the padding stays behind the Q loads
    {
      // Every store falls outside `none`; 64 bytes apart, they are not merged.
      const auto none = make_rsrc(a.queue, 0);
#pragma unroll
      for (int i = 0; i < kPad; ++i) __builtin_amdgcn_raw_buffer_store_b32(0u, none, 64 * i, 0, 0);
    }
    if (cur.live) {
      // Stream index of the item's first tile: already in the stream, or
      // started now (an item without tiles is never queued).
      int p0 = st_pos;
      if (cur.n_kt > 0) {
        if (nx_rem > 0) issue();
        p0 = nx_first;
      }
      queue_copy(next_item());
      while (st_pos < p0 + kAhead) issue();
      // Wait for tile 0 (younger: kAhead - 1 stream entries, plus the Q
      // loads and stores above if tile 0 preceded them).
      if (p0 < epi_pos)
        wait_vmcnt<2 * COPS * (kAhead - 1) + EOPS>();
      else
        wait_vmcnt<2 * COPS * (kAhead - 1)>();
      raw_barrier();
      if constexpr (FP8) sl2 = a.scale_log2 * ld_const(a.k_scale + cur.kvh);

      const int Lq = cur.Lq, Lk = cur.Lk, P = cur.P, n_kt = cur.n_kt;
      const int wrow0 = cur.row_begin + row_in_item;
      const bool wave_live = wrow0 < Lq;
      const int wrow_last = min(wrow0 + RW - 1, Lq - 1);
      const int wave_key_end = a.causal ? min(Lk, wrow_last + P + 1) : Lk;
      // Tiles this wave computes (a prefix: a causal wave stops at its own
      // diagonal) and, among them, the leading tiles that need no mask.
      const int wave_nkt = wave_live ? min(n_kt, (wave_key_end + kKeys - 1) / kKeys) : 0;
      int n_plain = min(wave_nkt, Lk / kKeys);
      if (a.causal) n_plain = min(n_plain, max(0, wrow0 + P + 1) / kKeys);
      const int32_t *bt_row = paged ? a.block_tables + static_cast<int64_t>(cur.s) * a.bt_stride : nullptr;

      // K^T operands of the tile in ring slot `kt` (its LDS address).
      auto kread = [&](uint32_t kt, KV (&kf)[DT::NKK][2]) {
#pragma unroll
        for (int kk = 0; kk < DT::NKK; ++kk) {
          if constexpr (FP8) {
            constexpr int KF = D == 128 ? 2 : 4;  // swz8: rows m + 16 flip this bit of kk
            kf[kk][0] = lds_load_b64<0>(((kk << 5) ^ kx_l) + (kt + kbase_l));
            kf[kk][1] = lds_load_b64<16 * D>((((kk ^ KF) << 5) ^ kx_l) + (kt + kbase_l));
          } else {
            const uint32_t ka = ((kk << 6) ^ kx_l) + (kt + kbase_l);
            kf[kk][0] = lds_load_b128<0>(ka);
            kf[kk][1] = lds_load_b128<16 * DT::ROWB>(ka);
          }
        }
      };
      auto qk = [&](const KV (&kf)[DT::NKK][2], f32x4 (&sc)[QS][2]) {
#pragma unroll
        for (int qs = 0; qs < QS; ++qs)
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) sc[qs][ks] = f32x4{0, 0, 0, 0};
#pragma unroll
        for (int kk = 0; kk < DT::NKK; ++kk)
#pragma unroll
          for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int qs = 0; qs < QS; ++qs) sc[qs][ks] = T::mfma16x16x32(op(kf[kk][ks]), qf[qs][kk], sc[qs][ks]);
      };

      float m_use[QS];  // running row max, scaled (log2) domain
#pragma unroll
      for (int qs = 0; qs < QS; ++qs) {
        m_use[qs] = kNegInf;
        lsum[qs] = 0.f;
#pragma unroll
        for (int j = 0; j < DT::NJ; ++j) o[qs][j] = f32x4{0, 0, 0, 0};
      }
      // Q is complete from here on: at most kPad operations are younger than
      // the Q loads' padding, which follows them.
      wait_vmcnt<kPad>();
#pragma unroll
      for (int qs = 0; qs < QS; ++qs)
#pragma unroll
        for (int kk = 0; kk < DT::NKK; ++kk) asm volatile("" : "+v"(qf[qs][kk]));
      f32x4 sc[QS][2];  // scores of the tile whose P is formed next
      if (wave_nkt > 0) {
        KV kf[DT::NKK][2];
        unhoist();
        kread(lds0 + (p0 % kSlots) * DT::SLOT_B, kf);
        qk(kf, sc);
      }
      const int epi_tiles = epi_pos - p0 - 1;  // leading tiles whose wait adds the item's start operations

      // Scores of the tile whose P is being formed, and the subtrahend of its
      // exponents (the running maximum after the tile's rescale check).
      float xt[QS][8], mref[QS];
      float alpha[QS];    // rescale factors of o before the pending products join it
      bool pend = false;  // whether they differ from 1
      // One unit of P: elements 2t, 2t + 1 of rows block qs, exponentiated
      // against the running maximum, added to the row sums and packed to 16
      // bits.
      auto p_unit = [&](int qs, int t) {
        const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(xt[qs][2 * t], sl2, -mref[qs]));
        const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(xt[qs][2 * t + 1], sl2, -mref[qs]));
        lsum[qs] += e0 + e1;
        return T::pack2(e0, e1);
      };
      // Lazy-rescale check of key tile jt (scores sc, masked as the tile
      // needs): xt takes the scores, m_use the running maxima, mref the
      // subtrahend of P.  The running maximum m_use of a row (the same in the
      // four lanes that hold the row) only moves when some element exceeds it
      // by more than kRescale, so P = 2^(s - m_use) <= 2^kRescale.  Each lane
      // checks its own elements; the cross-lane row maximum is only formed
      // when a maximum moves.  The row sums are rescaled at once; the
      // function returns whether a maximum moved, and alpha then holds the
      // factors for o, applied before this tile's products (formed with the
      // new maxima) join it -- at the start of the next tile, once the
      // previous tile's products are in.
      auto check = [&](auto mask_tag, int jt, bool blk_ok, float (&alpha)[QS]) {
        constexpr bool MASK = decltype(mask_tag)::value;
        const int kbase = jt * kKeys;
        float mnew[QS];
        bool grow = false;
#pragma unroll
        for (int qs = 0; qs < QS; ++qs) {
          int lim = 0;
          if constexpr (MASK) {
            const int row = wrow0 + 16 * qs + m;
            lim = a.causal ? min(Lk - 1, row + P) : Lk - 1;  // last visible key
            if (!blk_ok) lim = -1;
          }
#pragma unroll
          for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
              float v = sc[qs][ks][rr];
              if constexpr (MASK) v = (kbase + 16 * ks + 4 * g + rr > lim) ? kNegInf : v;
              xt[qs][4 * ks + rr] = v;
            }
          // this lane's maximum over its 8 keys of row m (scaled)
          mnew[qs] = max3_raw(max3_raw(xt[qs][0], xt[qs][1], xt[qs][2]),
                              max3_raw(xt[qs][3], xt[qs][4], xt[qs][5]), vmax_raw(xt[qs][6], xt[qs][7])) * sl2;
          grow |= mnew[qs] > m_use[qs] + kRescale;
        }
        bool moved = false;
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
#pragma unroll
          for (int qs = 0; qs < QS; ++qs) {
            const float m_new = fmaxf(m_use[qs], max32_raw(max16_raw(mnew[qs])));
            alpha[qs] = (m_use[qs] == kNegInf) ? 0.f : __builtin_amdgcn_exp2f(m_use[qs] - m_new);
            lsum[qs] *= alpha[qs];  // the row sums of earlier tiles' P (this tile's join after this)
            m_use[qs] = m_new;
          }
          moved = true;
        }
#pragma unroll
        for (int qs = 0; qs < QS; ++qs) mref[qs] = (m_use[qs] == kNegInf) ? 0.f : m_use[qs];
        return moved;
      };
      auto rescale = [&](const float (&alpha)[QS]) {
#pragma unroll
        for (int qs = 0; qs < QS; ++qs)
#pragma unroll
          for (int j = 0; j < DT::NJ; ++j) o[qs][j] *= alpha[qs];
      };
      // V^T operand j of the tile in ring slot `slot`: rows r0 and r0 + 16
      // (fp8: one transposing 8-bit read of rows R, widened by op at its products).
      auto vread = [&](uint32_t slot, int j) -> KV {
        if constexpr (FP8) {
          return lds_load_tr8(((j << 4) ^ vx_l) + (slot + DT::TILE_B + vbase_l));
        } else {
          const uint32_t vt = ((j << 5) ^ vx_l) + (slot + DT::TILE_B + vbase_l);
          const u32x2 lo = lds_load_tr16<0>(vt), hi = lds_load_tr16<16 * DT::ROWB>(vt);
          return u32x4{lo[0], lo[1], hi[0], hi[1]};
        }
      };
      // O^T += V^T P^T of the previous tile (operands vf, pb, read before the
      // barrier), with P of this tile (units of xt) formed in between -- one
      // unit, two exponentials and a pack, per two products -- so that the
      // exponentials run while the matrix core works.  The K reads of tile
      // jt + 1 (ring slot slot_next) are issued halfway.
      auto pv_p = [&](const KV (&vf)[DT::NJ], const u32x4 (&pb)[QS], uint32_t (&pw)[QS][4], uint32_t slot_next,
                      KV (&kf)[DT::NKK][2]) {
        // 16 products either way: 8 query rows x 2 ... -- PPU products per unit
        // of P (2 with two 16-row blocks at head_dim 128, 4 with one at 256)
        constexpr int NP = DT::NJ * QS, U = 4 * QS, PPU = NP / U;
        static_assert(NP == 16 && (PPU == 2 || PPU == 4), "16 products, 2 or 4 per unit of P");
        // fp8: conversions per unit -- the next unit's V^T operands, widened
        // while this unit's products run (the first before the section)
        constexpr int CV = FP8 ? 4 * DT::NJ / U : 0;
        kread(slot_next, kf);
        u32x4 vw[DT::NJ];
        constexpr int JPU = DT::NJ / U > 0 ? DT::NJ / U : 1;  // V^T operands per unit (rounded up)
#pragma unroll
        for (int j = 0; j < JPU; ++j) vw[j] = op(vf[j]);
#pragma unroll
        for (int i = 0; i < NP; ++i) {
          const int j = i / QS, qs = i % QS;
          if (FP8 && i % PPU == 0) {
            const int u = i / PPU;
#pragma unroll
            for (int jn = (u + 1) * DT::NJ / U; jn < (u + 2) * DT::NJ / U && jn < DT::NJ; ++jn)
              if (jn >= JPU) vw[jn] = op(vf[jn]);
          }
          o[qs][j] = T::mfma16x16x32(FP8 ? vw[j] : op(vf[j]), pb[qs], o[qs][j]);
          if (i % PPU == PPU - 1) {
            const int u = i / PPU;
            pw[u / 4][u % 4] = p_unit(u / 4, u % 4);
          }
        }
        if (FP8) __builtin_amdgcn_sched_group_barrier(0x002, CV, 0);  // VALU: the first operands
#pragma unroll
        for (int u = 0; u < U; ++u) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);           // MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 2 + CV / 2, 0);  // VALU
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);           // MFMA
          __builtin_amdgcn_sched_group_barrier(0x400, 2, 0);           // transcendental
          if (PPU == 4) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 3 + CV - CV / 2, 0);  // VALU
          if (PPU == 4) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          // DS read (K): halfway; fp8 codes (half the registers) after the first unit
          if (u == (FP8 ? 0 : U / 2 - 1)) __builtin_amdgcn_sched_group_barrier(0x100, 2 * DT::NKK, 0);
        }
      };
      auto p_only = [&](uint32_t (&pw)[QS][4]) {
#pragma unroll
        for (int u = 0; u < 4 * QS; ++u) pw[u / 4][u % 4] = p_unit(u / 4, u % 4);
      };
      auto pv_only = [&](const KV (&vf)[DT::NJ], const u32x4 (&pb)[QS]) {
        if constexpr (FP8) {
          // each operand widened just before its products, so that the
          // widened operands are never all live at once
#pragma unroll
          for (int j = 0; j < DT::NJ; ++j)
#pragma unroll
            for (int qs = 0; qs < QS; ++qs) o[qs][j] = T::mfma16x16x32(op(vf[j]), pb[qs], o[qs][j]);
#pragma unroll
          for (int j = 0; j < DT::NJ; ++j) {
            __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);   // VALU
            __builtin_amdgcn_sched_group_barrier(0x008, QS, 0);  // MFMA
          }
        } else {
#pragma unroll
          for (int qs = 0; qs < QS; ++qs)
#pragma unroll
            for (int j = 0; j < DT::NJ; ++j) o[qs][j] = T::mfma16x16x32(vf[j], pb[qs], o[qs][j]);
        }
      };
      // QK products of tile jt + 1 (kf) into sn, with the V^T operands of
      // tile jt (ring slot `slot`) read into vf in between: one transposing
      // read per product.  Products that share an accumulator are 2 QS
      // apart.
      auto qk_v = [&](const KV (&kf)[DT::NKK][2], f32x4 (&sn)[QS][2], uint32_t slot, KV (&vf)[DT::NJ]) {
        // V^T operands per product: 1/2 at head_dim 128 (two 16-row
        // blocks), 1 at 256 (one); each operand is two transposing reads.
        // K operands die as V operands fill, so the two never hold all
        // their registers at once.
        constexpr int NP = DT::NKK * 2 * QS;  // products
        static_assert(NP == 2 * DT::NJ || NP == DT::NJ, "one V operand per one or two products");
        constexpr int PPV = NP / DT::NJ;      // products per V operand
#pragma unroll
        for (int qs = 0; qs < QS; ++qs)
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) sn[qs][ks] = f32x4{0, 0, 0, 0};
        // fp8: each K operand widened while the previous one's products run
        u32x4 kw[DT::NKK][2];
        if constexpr (FP8) kw[0][0] = op(kf[0][0]);
#pragma unroll
        for (int i = 0; i < NP; ++i) {
          const int kk = i / (2 * QS), ks = (i / QS) % 2, qs = i % QS;
          if (FP8 && qs == 0 && 2 * kk + ks + 1 < 2 * DT::NKK) {
            const int n = 2 * kk + ks + 1;
            kw[n >> 1][n & 1] = op(kf[n >> 1][n & 1]);
          }
          sn[qs][ks] = T::mfma16x16x32(FP8 ? kw[kk][ks] : op(kf[kk][ks]), qf[qs][kk], sn[qs][ks]);
          if (i % PPV == 0) vf[i / PPV] = vread(slot, i / PPV);
        }
        constexpr int CK = FP8 ? 4 / QS : 0;  // conversions per product
        if (FP8) __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU: the first K operand
#pragma unroll
        for (int i = 0; i < NP; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);        // MFMA
          __builtin_amdgcn_sched_group_barrier(0x100, 2 / PPV, 0);  // DS read
          if (FP8) __builtin_amdgcn_sched_group_barrier(0x002, CK, 0);  // VALU
        }
      };
      // One key tile jt (ring slot `slot`; tile jt + 1 in slot_next), after
      // the barrier that completes tile jt + 1: the pending rescale, the
      // check of tile jt, the next stream entry, O += P V of tile jt - 1 (vf,
      // pb; PV) with tile jt's P formed and tile jt + 1's K read in between,
      // the QK products of tile jt + 1 with tile jt's V^T read in between.
      // On return vf and pb hold tile jt's operands and sc tile jt + 1's
      // scores.
      auto tile = [&](auto pv_tag, auto mask_tag, int jt, uint32_t slot, uint32_t slot_next, bool blk_ok,
                      KV (&vf)[DT::NJ], u32x4 (&pb)[QS]) {
        unhoist();
        if (pend) rescale(alpha);  // tile jt - 1's maxima, before its products join o
        pend = check(mask_tag, jt, blk_ok, alpha);
        issue();
        uint32_t pw[QS][4];
        KV kf[DT::NKK][2];  // tile jt + 1 (discarded past the last)
        if constexpr (decltype(pv_tag)::value) {
          pv_p(vf, pb, pw, slot_next, kf);
        } else {
          kread(slot_next, kf);
          p_only(pw);
        }
#pragma unroll
        for (int qs = 0; qs < QS; ++qs) pb[qs] = u32x4{pw[qs][0], pw[qs][1], pw[qs][2], pw[qs][3]};
        __builtin_amdgcn_sched_barrier(0);  // the two sections are scheduled apart
        f32x4 sn[QS][2];
        qk_v(kf, sn, slot, vf);
#pragma unroll
        for (int qs = 0; qs < QS; ++qs)
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) sc[qs][ks] = sn[qs][ks];
      };
      // Once per tile jt and wave, in tile order, in every loop below: wait
      // for this wave's copies of tile jt + 1 (younger: kAhead - 2 stream
      // entries, plus the Q loads and stores of the item's start if tile
      // jt + 1 preceded them).
      auto sync = [&](int jt) {
        if (jt < epi_tiles)
          wait_vmcnt<2 * COPS * (kAhead - 2) + EOPS>();
        else
          wait_vmcnt<2 * COPS * (kAhead - 2)>();
        wait_lgkmcnt0();  // and its reads of tiles jt - 1 and jt are done
        raw_barrier();    // tile jt + 1 complete; slot of tile jt - 1 free
      };
      // Whether the block of key tile jt exists (the masked loop once a
      // missing block has been seen).
      auto block_ok = [&](int jt) {
        const int blk = ld_const(bt_row + jt * kKeys / a.block_size);
        return blk >= 0 && blk < num_blocks;
      };

      // Ring slots (LDS addresses) of tiles jt and jt + 1.
      uint32_t slot = lds0 + (p0 % kSlots) * DT::SLOT_B;
      uint32_t slot_next = slot == lds_last ? lds0 : slot + DT::SLOT_B;
      auto advance = [&]() {
        slot = slot_next;
        slot_next = slot_next == lds_last ? lds0 : slot_next + DT::SLOT_B;
      };
      KV vf[DT::NJ];  // V^T operands and P of the tile whose products are pending
      u32x4 pb[QS];
      int jt = 0;
      plain_end = bad_seen ? 0 : n_plain;
      if (n_kt > 0) {  // tile 0: no earlier tile's products
        sync(0);
        if (wave_nkt > 0) {
          if (plain_end > 0)
            tile(std::false_type{}, std::false_type{}, 0, slot, slot_next, true, vf, pb);
          else
            tile(std::false_type{}, std::true_type{}, 0, slot, slot_next, !bad_seen || !paged || block_ok(0), vf, pb);
        } else {
          issue();
        }
        advance();
        jt = 1;
      }
      for (; jt < plain_end; ++jt) {
        sync(jt);
        tile(std::true_type{}, std::false_type{}, jt, slot, slot_next, true, vf, pb);
        advance();
      }
      for (; jt < n_kt; ++jt) {
        sync(jt);
        if (jt < wave_nkt) {
          tile(std::true_type{}, std::true_type{}, jt, slot, slot_next, !bad_seen || !paged || block_ok(jt), vf, pb);
        } else {
          issue();
          if (jt == wave_nkt) {  // the wave's last tile
            unhoist();
            if (pend) rescale(alpha);
            pv_only(vf, pb);
          }
        }
        advance();
      }
      if (n_kt > 0 && wave_nkt == n_kt) {  // the item's last tile
        unhoist();
        if (pend) rescale(alpha);
        pv_only(vf, pb);
      }
    } else {
      queue_copy(next_item());
    }
    // Next item: publish the fetched index (slot k + 2 of 4: a wave still
    // reading slot k + 1 cannot be overtaken, the write comes after the
    // barrier that follows its read).  A plain barrier: the fence of
    // __syncthreads() would wait for the K/V copies in flight.
    if (threadIdx.x == 0) {
      lds_item[(k + 2) & 3] = static_cast<int>(fetched);
      wait_lgkmcnt0();
    }
    raw_barrier();
    const int idx_new = __builtin_amdgcn_readfirstlane(lds_item[(k + 2) & 3]);
    prev = cur;
    if constexpr (kRedescribe) {
      cur = describe(idx_nxt);
    } else {
      cur = nxt;
      nxt = describe(idx_new);
    }
    idx_cur = idx_nxt;
    idx_nxt = idx_new;
  }
  wait_vmcnt<0>();  // the stream's last (empty) copies and the last stores complete before the workgroup ends
  if (threadIdx.x == 0) {
    if (atomicAdd(a.queue + 8, 1u) == gridDim.x - 1) {
      // Every other workgroup has taken its last index and finished.
#pragma unroll
      for (int c = 0; c < 9; ++c) atomicExch(a.queue + c, 0u);
    }
  }
}

// The body lives in a device function: its inline assembly uses register
// constraints that only the device compilation accepts.
template <class T, int D, class S, bool GATED, bool FP8, bool TAB>
__global__ __launch_bounds__(64 * S::NW) __attribute__((amdgpu_waves_per_eu(S::WPE)))
void varlen_prefill_dma_kernel(const PrefillArgs a) {
  prefill_persistent<T, D, S, GATED, FP8, TAB>(a);
}

template <class T, int D, class S, bool FP8>
int launch_prefill_dma(PrefillArgs a, hipStream_t st) {
  const int rows_per_item = S::ITEM_ROWS / a.G4;
  a.n_qtiles = (a.max_seqlen_q + rows_per_item - 1) / rows_per_item;
  const int64_t U = static_cast<int64_t>(a.Hkv) * a.quads * a.num_seqs;
  const int64_t total = work_grid(a.n_qtiles, U);
  if (total > 0x7fffffff) return fail(NQ_EINVAL, "varlen_prefill: too many work items");
  if (!a.queue) return fail(NQ_EINVAL, "varlen_prefill: null workspace");
  a.pin = U >= 8;
  // Cost order when the sequence bounds fit in LDS and counting the items
  // at launch stays short; query-tile order otherwise.
  a.by_cost = a.num_seqs <= kMaxSeqs && static_cast<int64_t>(a.num_seqs) * a.n_qtiles <= 65536;
  const int nkt_max = (a.max_seqlen_k + kKeys - 1) / kKeys;  // key tiles of the longest item
  a.level_shift = 0;
  while ((nkt_max >> a.level_shift) + 1 > kQueueLevels) ++a.level_shift;
  a.n_levels = (nkt_max >> a.level_shift) + 1;
  // The queue's items listed in LDS at launch when every queue fits the list
  // (its groups x query tiles bound it), the (level, sequence) starts fit the
  // ring and the packed words hold the fields.
  const int64_t cx_max = U >= 8 ? (U + 7) / 8 : U;
  if (a.by_cost && cx_max * a.n_qtiles <= S::MAX_ITEMS && static_cast<int64_t>(a.num_seqs) * a.n_levels * 4 <= S::RING_BYTES &&
      U / a.num_seqs <= 256 && a.n_qtiles <= 16384)
    a.by_cost = 2;
  // S::WG_PER_CU resident workgroups per CU, never more than there are
  // items; a multiple of 8 so every XCD gets the same count.
  int64_t grid = (static_cast<int64_t>(device_cus()) * S::WG_PER_CU + 7) / 8 * 8;
  if (grid > total) grid = total;  // work_grid() is a multiple of 8 when pinned
  auto *kern = a.gate ? (a.by_cost == 2 ? varlen_prefill_dma_kernel<T, D, S, true, FP8, true>
                                        : varlen_prefill_dma_kernel<T, D, S, true, FP8, false>)
                     : (a.by_cost == 2 ? varlen_prefill_dma_kernel<T, D, S, false, FP8, true>
                                        : varlen_prefill_dma_kernel<T, D, S, false, FP8, false>);
  kern<<<static_cast<int>(grid), 64 * S::NW, S::LDS_BYTES, st>>>(a);
  return check_launch(a.gate ? "varlen_prefill(gated)" : "varlen_prefill");
}

template <class T, bool FP8, int D>
int launch_prefill(PrefillArgs a, hipStream_t s) {
  if constexpr (D == 256) {
    return launch_prefill_dma<T, D, ShapeD, FP8>(a, s);
  } else {
    return launch_prefill_dma<T, D, ShapeC, FP8>(a, s);  // fp8 copies: one 1 KiB piece per wave
  }
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" int64_t nq_prefill_workspace_bytes(void) { return kQueueWords * sizeof(uint32_t); }

static int varlen_prefill_impl(const void *q, int64_t q_row_stride, int64_t q_head_stride, const void *k,
                               const void *v, int64_t kv_row_stride, const int32_t *cu_seqlens_q,
                               const int32_t *cu_seqlens_k, int max_seqlen_q, int max_seqlen_k,
                               const int32_t *block_tables, int64_t bt_stride, int max_blocks_per_seq,
                               int64_t num_blocks, void *out, int64_t out_row_stride, int64_t out_head_stride,
                               int num_seqs, int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                               float softmax_scale, int causal, int q_dtype, int kv_dtype, const float *k_scale,
                               const float *v_scale, void *workspace, int64_t workspace_bytes, const void *gate,
                               int64_t gate_row_stride, int64_t gate_head_stride, int64_t total_q,
                               void *stream) {
  if (num_seqs == 0 || max_seqlen_q == 0) return NQ_OK;
  if (num_seqs < 0 || max_seqlen_q < 0 || max_seqlen_k < 0 || num_q_heads <= 0 || num_kv_heads <= 0)
    return fail(NQ_EINVAL, "varlen_prefill: bad sizes");
  if (num_q_heads % num_kv_heads != 0)
    return fail(NQ_EINVAL, "varlen_prefill: num_q_heads %d not a multiple of num_kv_heads %d", num_q_heads,
                num_kv_heads);
  const int G = num_q_heads / num_kv_heads;
  if (G > 4 && G % 4 != 0) return fail(NQ_EUNSUPPORTED, "varlen_prefill: GQA group %d (need <= 4 or a multiple of 4)", G);
  if (G == 3) return fail(NQ_EUNSUPPORTED, "varlen_prefill: GQA group 3");
  if (head_dim != 128 && head_dim != 256)
    return fail(NQ_EUNSUPPORTED, "varlen_prefill: head_dim %d (built: 128, 256)", head_dim);
  if (q_dtype != NQ_BF16 && q_dtype != NQ_F16)
    return fail(NQ_EUNSUPPORTED, "varlen_prefill: q dtype %d (need f16/bf16)", q_dtype);
  const bool fp8 = kv_dtype == NQ_FP8_E4M3;
  if (!fp8 && kv_dtype != q_dtype)
    return fail(NQ_EUNSUPPORTED, "varlen_prefill: kv dtype %d with q dtype %d", kv_dtype, q_dtype);
  if (fp8 && (!k_scale || !v_scale)) return fail(NQ_EINVAL, "varlen_prefill: fp8 K/V needs scales");
  if (!q || !k || !v || !cu_seqlens_q || !cu_seqlens_k || !out) return fail(NQ_EINVAL, "varlen_prefill: null pointer");
  if (block_tables) {
    if (block_size <= 0 || block_size % kKeys != 0)
      return fail(NQ_EUNSUPPORTED, "varlen_prefill: block_size %d must be a multiple of %d", block_size, kKeys);
    if (max_blocks_per_seq <= 0 || bt_stride < max_blocks_per_seq)
      return fail(NQ_EINVAL, "varlen_prefill: block table width");
    if (static_cast<int64_t>(max_blocks_per_seq) * block_size < max_seqlen_k)
      return fail(NQ_EINVAL, "varlen_prefill: block table narrower than max_seqlen_k");
  }
  const int qsz = 2, ksz = fp8 ? 1 : 2;
  if ((q_row_stride * qsz) % 16 || (q_head_stride * qsz) % 16 || !aligned(q, 16) || (kv_row_stride * ksz) % 16 ||
      !aligned(k, 16) || !aligned(v, 16) || (out_row_stride * qsz) % 16 || (out_head_stride * qsz) % 16 ||
      !aligned(out, 16))
    return fail(NQ_EINVAL, "varlen_prefill: q/k/v/out alignment");
  if (kv_row_stride * ksz > (1 << 20)) return fail(NQ_EINVAL, "varlen_prefill: K/V row stride too large");
  // Output stores address a sequence's rows of one head with 32-bit offsets.
  if ((static_cast<int64_t>(max_seqlen_q) + 256) * out_row_stride * qsz >= (int64_t{1} << 31))
    return fail(NQ_EINVAL, "varlen_prefill: max_seqlen_q %d x output row stride too large", max_seqlen_q);
  if ((!workspace || workspace_bytes < nq_prefill_workspace_bytes() || !aligned(workspace, 4)))
    return fail(NQ_EINVAL, "varlen_prefill: workspace of %lld bytes at %p (need %lld, 4-byte aligned)",
                (long long)workspace_bytes, workspace, (long long)nq_prefill_workspace_bytes());
  PrefillArgs a{};
  a.queue = static_cast<uint32_t *>(workspace);
  a.q = static_cast<const uint8_t *>(q);
  a.q_rs = q_row_stride * qsz;
  a.q_hs = q_head_stride * qsz;
  a.k = static_cast<const uint8_t *>(k);
  a.v = static_cast<const uint8_t *>(v);
  a.kv_rs = kv_row_stride * ksz;
  a.cu_q = cu_seqlens_q;
  a.cu_k = cu_seqlens_k;
  a.block_tables = block_tables;
  a.bt_stride = bt_stride;
  a.max_blocks = max_blocks_per_seq;
  a.num_blocks = static_cast<int>(num_blocks < 0x7fffffff ? num_blocks : 0x7fffffff);
  a.out = static_cast<uint8_t *>(out);
  a.o_rs = out_row_stride * qsz;
  a.o_hs = out_head_stride * qsz;
  // The gate rides in the kernel's output store.
  if (gate) {
    if ((gate_row_stride * qsz) % 16 || (gate_head_stride * qsz) % 16 || !aligned(gate, 16))
      return fail(NQ_EINVAL, "varlen_prefill_gated: gate alignment");
    if ((static_cast<int64_t>(max_seqlen_q) + 256) * gate_row_stride * qsz >= (int64_t{1} << 31))
      return fail(NQ_EINVAL, "varlen_prefill_gated: max_seqlen_q x gate row stride too large");
    if (total_q < 0) return fail(NQ_EINVAL, "varlen_prefill_gated: total_q < 0");
    a.gate = static_cast<const uint8_t *>(gate);
    a.g_rs = gate_row_stride * qsz;
    a.g_hs = gate_head_stride * qsz;
  }
  a.Hq = num_q_heads;
  a.Hkv = num_kv_heads;
  a.G = G;
  a.G4 = G < 4 ? G : 4;
  a.quads = G < 4 ? 1 : G / 4;
  a.block_size = block_size;
  a.num_seqs = num_seqs;
  a.max_seqlen_q = max_seqlen_q;
  a.max_seqlen_k = max_seqlen_k;
  a.causal = causal;
  a.scale_log2 = softmax_scale * kLog2e;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  hipStream_t st = static_cast<hipStream_t>(stream);
  int rc;
  if (head_dim == 256) {
    if (q_dtype == NQ_BF16)
      rc = fp8 ? launch_prefill<BF16, true, 256>(a, st) : launch_prefill<BF16, false, 256>(a, st);
    else
      rc = fp8 ? launch_prefill<F16, true, 256>(a, st) : launch_prefill<F16, false, 256>(a, st);
  } else if (q_dtype == NQ_BF16) {
    rc = fp8 ? launch_prefill<BF16, true, 128>(a, st) : launch_prefill<BF16, false, 128>(a, st);
  } else {
    rc = fp8 ? launch_prefill<F16, true, 128>(a, st) : launch_prefill<F16, false, 128>(a, st);
  }
  return rc;
}

extern "C" int nq_varlen_prefill(const void *q, int64_t q_row_stride, int64_t q_head_stride, const void *k,
                                 const void *v, int64_t kv_row_stride, const int32_t *cu_seqlens_q,
                                 const int32_t *cu_seqlens_k, int max_seqlen_q, int max_seqlen_k,
                                 const int32_t *block_tables, int64_t bt_stride, int max_blocks_per_seq,
                                 int64_t num_blocks, void *out, int64_t out_row_stride,
                                 int64_t out_head_stride, int num_seqs, int num_q_heads, int num_kv_heads,
                                 int head_dim, int block_size, float softmax_scale, int causal, int q_dtype,
                                 int kv_dtype, const float *k_scale, const float *v_scale, void *workspace,
                                 int64_t workspace_bytes, void *stream) {
  return varlen_prefill_impl(q, q_row_stride, q_head_stride, k, v, kv_row_stride, cu_seqlens_q, cu_seqlens_k,
                             max_seqlen_q, max_seqlen_k, block_tables, bt_stride, max_blocks_per_seq, num_blocks,
                             out, out_row_stride, out_head_stride, num_seqs, num_q_heads, num_kv_heads, head_dim,
                             block_size, softmax_scale, causal, q_dtype, kv_dtype, k_scale, v_scale, workspace,
                             workspace_bytes, nullptr, 0, 0, 0, stream);
}

extern "C" int nq_varlen_prefill_gated(
    const void *q, int64_t q_row_stride, int64_t q_head_stride, const void *k, const void *v,
    int64_t kv_row_stride, const int32_t *cu_seqlens_q, const int32_t *cu_seqlens_k, int max_seqlen_q,
    int max_seqlen_k, const int32_t *block_tables, int64_t bt_stride, int max_blocks_per_seq, int64_t num_blocks,
    void *out, int64_t out_row_stride, int64_t out_head_stride, int num_seqs, int num_q_heads, int num_kv_heads,
    int head_dim, int block_size, float softmax_scale, int causal, int q_dtype, int kv_dtype, const float *k_scale,
    const float *v_scale, void *workspace, int64_t workspace_bytes, const void *gate, int64_t gate_row_stride,
    int64_t gate_head_stride, int64_t total_q, void *stream) {
  if (!gate) return fail(NQ_EINVAL, "varlen_prefill_gated: null gate");
  return varlen_prefill_impl(q, q_row_stride, q_head_stride, k, v, kv_row_stride, cu_seqlens_q, cu_seqlens_k,
                             max_seqlen_q, max_seqlen_k, block_tables, bt_stride, max_blocks_per_seq, num_blocks,
                             out, out_row_stride, out_head_stride, num_seqs, num_q_heads, num_kv_heads, head_dim,
                             block_size, softmax_scale, causal, q_dtype, kv_dtype, k_scale, v_scale, workspace,
                             workspace_bytes, gate, gate_row_stride, gate_head_stride, total_q, stream);
}
