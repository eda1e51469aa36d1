// Paged decode attention for gfx950 (every sequence has one query token).
//
// Work decomposition (planned on the host once per batch, pkv_plan_decode):
//
//  * Pieces. A sequence of np pages is cut into pieces of part_pages pages,
//    the remainder last; a remainder shorter than both kMinTail pages and
//    half a piece is folded into the piece before it. The small remainders give the deal below pieces that
//    fill the gaps between bins (measured 2% faster than pieces of nearly
//    equal size over six batches of 256 lognormal sequences). The cut
//    depends only on that sequence's own length, so its result never
//    depends on what it is batched with: a piece's arithmetic is the same
//    wherever it runs, and the partials of a cut sequence merge in a fixed
//    order.
//  * Bins. The pieces are dealt to a fixed number of bins, longest first, each
//    to the bin with the least work so far (LPT), so every bin ends up with
//    about the same number of pages. A bin is one workgroup per group of up
//    to 4 KV heads, and the grid is only as large as what stays resident, so
//    no workgroup waits for a slot and all of them stream until about the
//    same time. In a bin, the pieces of cut sequences that are not their
//    sequence's last come first (they publish while everything streams),
//    whole sequences next, and last pieces at the end (a last piece reads
//    its sequence's arrival count when it starts and, if every other piece
//    has published, merges at its end without publishing its own).
//  * Waves. Each wave owns one KV head and runs the bin's page stream on its
//    own (no workgroup barrier anywhere): it loads its head's 128-byte slice
//    of every token row (whole cache lines, eight lanes a row) into registers
//    one page ahead of use, copies the page to its private LDS tile, and
//    reads the tile back in the matrix-core operand layouts. One page in
//    flight per wave measured faster than two or three: with 2048 waves
//    streaming, deeper prefetch only lengthens the queue at the memory
//    system (the first page lands later, and the stream is no faster).
//    Every step issues the same loads on every path (no page skipped at the
//    end of the stream, Q and new rows staged in LDS per batch of items,
//    page words read with scalar loads), so the wait for a page never waits
//    for the page issued after it.
//
// Per wave, head and page (G query heads share the KV head, G <= 16):
//  1. S^T = K Q^T with one 16x16x32 MFMA per 32 dims: the K rows (from LDS)
//     are the A operand, Q^T the B operand (column n = query head n, zero
//     beyond G). Lane (head n, group g) then holds the scores of tokens
//     4g..4g+3 of the page for head n;
//  2. online softmax in registers: mask past kv_len, running max / sum with
//     two row swaps (v_permlane16_swap, v_permlane32_swap: VALU, no LDS
//     round trip); p = 2^(s*scale*log2e - m) rounded to the pool
//     dtype -- four values per lane that are exactly the A operand of a
//     16x16x16 MFMA. The reference max m moves lazily (only when a head's
//     max grows by more than 2^8), so most pages skip the rescale of o;
//  3. PV on MFMA: ds_read_b64_tr_b16 hands each lane 4 consecutive tokens of
//     one V dim, the B operand, one read per 16 dims.
//
// Loads cover only a page's rows below kv_len (the plan carries each page's
// live row count beside its id): the tail of a sequence's last page is
// outside the buffer range and reads as zeros without a memory access.
//
// Cut sequences merge in the same launch. Each piece publishes its partial
// (o, m, l) with 16-byte buffer stores carrying the sc1 (agent coherence)
// bit, which write through the per-XCD L2, waits until they have completed
// (s_waitcnt), then bumps its (sequence, head) arrival counter. The wave that
// sees the last arrival reads the partials back with sc1 loads (never a
// stale L2 line) and writes the output; a last piece that finds every other
// piece arrived merges without publishing its own. This avoids a second
// launch and an agent-scope release fence, whose L2 write-back walks the
// whole cache.
//
// Fused append (optional): when the caller passes the step's new K/V rows,
// the wave whose piece holds a sequence's last page writes its head's slice
// of the new row to slot_mapping's slot and patches the copy it loaded, so a
// decode step costs one launch per layer instead of two. The patch is
// applied only when slot_mapping names the same slot as the page table, so
// the result is exactly "append, then attend" (the caller guarantees that no
// other sequence of the launch reads that slot).
#include <algorithm>
#include <mutex>
#include <queue>
#include <vector>

#include "mfma.h"

namespace pkv {

constexpr int kMaxPartPages = 64;   // bound on part_pages (ABI)
constexpr int kMaxWaves = 4;        // KV heads (one per wave) per workgroup
constexpr int kPageIdBits = 27;     // a plan page word: id | (live rows - 1) << 27 | bad << 31
constexpr int kHdrInts = 4;         // bin header {n_items, n_pages, 0, 0}
constexpr int kItemInts = 8;        // {seq, n_pages, first token, kv_len, slot, n_pieces,
                                    //  first slot, flags}
constexpr int kItemLast = 1;        // flags: the piece holds its sequence's last page
constexpr int kStageMax = 8;        // items staged in LDS at a time (at most)
constexpr int kPlanTail = 64;       // zero ints after the last bin (words read past its end)
constexpr int kMinTail = 4;         // a remainder of a cut below this (and below half a
                                    // piece) joins the piece before it

// KV heads per workgroup: one wave each, at most kMaxWaves, dividing Hkv.
__host__ __device__ static inline int heads_per_wg(int hkv) { return hkv % 4 == 0 ? 4 : hkv % 2 == 0 ? 2 : 1; }

// Layout of one partition's partial output: per (slot, KV head), NGR groups
// of 4 head rows, each NDB dim blocks of 16 lanes x 4 rows (float4 per
// lane) -- exactly the MFMA accumulator layout, so a wave stores and loads
// it with one 16-byte access per lane and dim block.
template <int D, int G> struct PartLayout {
  static constexpr int NGR = (G + 3) / 4;
  static constexpr int NDB = D / 16;
  static constexpr int FLOATS = NGR * NDB * 64;  // per (slot, KV head)
};

// Split-K merge for one KV head h of sequence seq, run by the wave that
// published the last partial, or by the sequence's last piece with its own
// partial still in registers (`own`). Lanes run over partitions for each
// head row's max M and sum L; then, 64 partitions at a time, the weights
// 2^(m_s - M) go to this wave's LDS scratch as [partition][GS rows], and the
// partial outputs are read in the producers' own layout: lane (n, g) takes
// row group rg = g % NGR of the chunk's partitions cn - 1 - j for j = g / NGR,
// g / NGR + SPLIT, ..., and the SPLIT lane groups that share a row group are
// summed by shuffles at the end. The chunk's last partition goes to lane
// group 0, whose lanes (n, rg) hold exactly that row group of an own
// partial in their accumulators, so `own` needs no data movement for o and
// enters the sums in the same place with the same bits a store and load
// would give. The summation order depends only on the partition count, so
// the result does not depend on the batch or on which wave merges.
template <typename T, int D, int G>
__device__ __forceinline__ void merge_head(T* __restrict__ out, float* wts, int seq, int h,
                                           int n_kv_heads, int nparts, int slot0,
                                           __amdgpu_buffer_rsrc_t ro, __amdgpu_buffer_rsrc_t rm,
                                           bool own, const f32x4* own_o, float own_m,
                                           float own_l) {
  typedef PartLayout<D, G> PL;
  constexpr int NDB = D / 16;
  constexpr int NGR = PL::NGR;
  constexpr int SPLIT = 4 / NGR;
  constexpr int GS = 4 * NGR;              // weight rows per partition (>= G)
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
  const int rg = g % NGR, so = g / NGR;
  const int Hq = n_kv_heads * G;
  const int own_part = own ? nparts - 1 : -1;
  // (m, l) of every head of partitions c0 + lane; an own partition's come
  // from lanes 0 .. G - 1, which hold head r's running max and sum
  auto load_ml = [&](int c0, float* mr, float* lr) {
    const bool mine = c0 + lane == own_part;
    const bool ok = c0 + lane < nparts && !mine;
    const uint32_t b2 = (uint32_t)(((int64_t)(slot0 + (ok ? c0 + lane : 0)) * Hq + h * G) * 8);
#pragma unroll
    for (int r = 0; r < G; ++r) {
      const f32x2 ml =
          __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(rm, b2 + 8 * r, 0, kSc1));
      const float m_own = lane_value(own_m, r), l_own = lane_value(own_l, r);
      mr[r] = ok ? ml[0] : mine ? m_own : -INFINITY;
      lr[r] = ok ? ml[1] : mine ? l_own : 0.f;
    }
  };
  // Partition c0 + cn - 1 - j of this lane's row group (j < cn).
  auto load_part = [&](int c0, int j, f32x4* v) {
    const int cn = min(64, nparts - c0);
    const int pi = c0 + cn - 1 - (j < cn ? j : 0);
    const bool mine = pi == own_part;   // then j == 0: lane group 0
    const uint32_t off = (uint32_t)(((int64_t)(slot0 + pi) * n_kv_heads + h) * PL::FLOATS * 4);
#pragma unroll
    for (int b = 0; b < NDB; ++b)
      v[b] = j >= cn ? f32x4{0.f, 0.f, 0.f, 0.f}
             : mine ? own_o[b]
                    : __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                    ro, off + ((rg * NDB + b) * 16 + n) * 16, 0,
                                                    kSc1));
  };
  // The first partitions do not depend on the maximum: their loads go out
  // with the (m, l) loads, so a sequence of up to SPLIT partitions merges in
  // one round trip.
  f32x4 v[NDB];
  load_part(0, so, v);
  float mr[G], lr[G], M[G], L[G];
#pragma unroll
  for (int r = 0; r < G; ++r) { M[r] = -INFINITY; L[r] = 0.f; }
  for (int c0 = 0; c0 < nparts; c0 += 64) {
    load_ml(c0, mr, lr);
#pragma unroll
    for (int r = 0; r < G; ++r) M[r] = fmaxf(M[r], wave_max(mr[r]));
  }
  f32x4 acc[NDB];
#pragma unroll
  for (int b = 0; b < NDB; ++b) acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int c0 = 0; c0 < nparts; c0 += 64) {
    if (nparts > 64) load_ml(c0, mr, lr);  // else still in registers
#pragma unroll
    for (int r = 0; r < GS; ++r) {
      float wv = 0.f;
      if (r < G) {
        wv = c0 + lane < nparts ? __builtin_amdgcn_exp2f(mr[r] - M[r]) : 0.f;
        L[r] += wave_sum(wv * lr[r]);
      }
      wts[lane * GS + r] = wv;
    }
    wave_lds_sync();
    const int cn = min(64, nparts - c0);
    for (int j = so; j < cn; j += SPLIT) {
      if (c0 > 0 || j > so) load_part(c0, j, v);
      const f32x4 wr = *reinterpret_cast<const f32x4*>(wts + (cn - 1 - j) * GS + 4 * rg);
#pragma unroll
      for (int b = 0; b < NDB; ++b) acc[b] += wr * v[b];
    }
    wave_lds_sync();  // the next chunk rewrites the weights
  }
#pragma unroll
  for (int b = 0; b < NDB; ++b) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (SPLIT >= 4) acc[b][i] = sum_x16(acc[b][i]);
      if (SPLIT >= 2) acc[b][i] = sum_x32(acc[b][i]);
    }
  }
  if (so == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * rg + i;
      float lr_ = L[0];
#pragma unroll
      for (int rr = 1; rr < G; ++rr)  // static indices keep L in registers
        if (r == rr) lr_ = L[rr];
      if (r < G) {
        const float inv = 1.f / lr_;   // one division per row, not per element
#pragma unroll
        for (int b = 0; b < NDB; ++b)
          out[((int64_t)seq * Hq + h * G + r) * D + 16 * b + n] = (T)(acc[b][i] * inv);
      }
    }
  }
}

#ifdef PKV_TIMELINE
// Instrumented build only (-DPKV_TIMELINE): every wave records, in 100 MHz
// s_memrealtime ticks, {start, first page done, last page done, end,
// pages, items, merges, ticks spent merging} with plain vector stores, for
// wave (bin * head groups + group) * waves + wave below kTimelineWaves. Read back with
// pkv_timeline_read.
constexpr int kTimelineWaves = 16384;
__device__ unsigned long long pkv_timeline[kTimelineWaves * 8];
#define PKV_TL(...) __VA_ARGS__
#else
#define PKV_TL(...)
#endif

// One wave's LDS tile: 16 K rows then 16 V rows of its head, each padded by
// 16 bytes so the K operand reads and the transposed V reads of a wave spread
// over the banks.
template <typename T, int D> struct Tile {
  static constexpr int RB = D * (int)sizeof(T);   // bytes of one head's row
  static constexpr int RS = RB + 16;
  static constexpr int BYTES = 2 * 16 * RS;
};

// A wave's item slots in LDS: C items of {Q rows of the G query heads of
// its KV head, the KV head's slice of the new K row, of the new V row}.
template <typename T, int D, int G> struct Stage {
  static constexpr int QB = G * D * (int)sizeof(T);
  static constexpr int RB = D * (int)sizeof(T);
  static constexpr int SLOT = QB + 2 * RB;
  static constexpr int C = 4096 / QB < 1 ? 1 : 4096 / QB > 8 ? 8 : 4096 / QB;
  static constexpr int QC = QB / 16;          // 16-byte chunks of the Q rows
  static constexpr int RC = RB / 16;          // of a new row slice
  static constexpr int CPI = SLOT / 16;       // per slot
  static constexpr int ROUNDS = (C * CPI + 63) / 64;
  static constexpr int BYTES = C * SLOT;
};

// A wave's two rings in LDS, for the stores it defers: KR new K/V row
// slices of its KV head (the fused append; RB2 bytes each) with their
// slots, and KO finished whole-sequence outputs (the rows of the G query
// heads of its KV head; OB bytes each) with their sequence ids. They share
// what a wave's share of 80 KiB leaves beside its tile and item slots (so
// two workgroups of four waves still fit a compute unit): the row ring up
// to half of it, the output ring the rest, each at most 16 entries. At
// head_dim 128 there is no row ring (KR = 0: the new rows are stored at
// once): its code would take the one-query-head kernel past 256 VGPRs, to
// one wave a SIMD.
template <typename T, int D, int G> struct Rings {
  static constexpr int OB = G * D * (int)sizeof(T);
  static constexpr int RB2 = 2 * D * (int)sizeof(T);
  static constexpr int FREE = 20480 - Tile<T, D>::BYTES - Stage<T, D, G>::BYTES - 2 * 64;
  static constexpr int KR0 = (FREE / 2 < FREE - OB ? FREE / 2 : FREE - OB) / RB2;
  static constexpr int KR = D > 64 ? 0 : KR0 < 1 ? 1 : KR0 > 16 ? 16 : KR0;
  static constexpr int KO0 = (FREE - KR * RB2) / OB;
  static constexpr int KO = KO0 < 1 ? 1 : KO0 > 16 ? 16 : KO0;
  static constexpr int ROWS = KR * RB2 + 64;     // row slices, then 16 slot ids
  static constexpr int BYTES = ROWS + KO * OB + 64;
};

// One workgroup per (bin, group of KV heads); wave w streams KV head
// hg * waves + w through the bin's pages, one piece (item) after another,
// without restarting the page pipeline at item boundaries. The bin's plan
// block at plan + bin * stride is {n_items, n_pages, 0, 0}, then n_pages page
// words (id | (live rows - 1) << 27 | bad << 31); its n_items items of
// kItemInts end the block, item i at plan + (bin + 1) * stride - (i + 1) *
// kItemInts. Header, first words and first items thus all sit at addresses
// known before any of them is read, so one round trip fetches them all and
// the first page and Q loads go out after it (the block is at least
// kHdrInts + kStageMax items long, so the first batch's item reads stay
// inside it).
//
// Cut sequences. A piece that is not its sequence's last publishes its
// partial (o, m, l) with sc1 stores and goes on streaming; its arrival is
// counted two pages later, when the wait for a page loaded after those
// stores has (vmcnt counts in order) also seen the stores complete, and the
// count it returns is checked at once. The last piece of a
// cut sequence runs at the end of its bin: it reads the arrival counter when
// it starts and, if every other piece has arrived by then, merges at its end
// without counting itself, its own partial taken from its registers (the
// same bits a store and a load would give, in the same place of the
// summation, so both paths produce the same output) and never stored;
// otherwise it publishes and counts its own arrival, and whichever piece
// arrives last merges.
template <typename T, int D, int G>
__global__ __launch_bounds__(kMaxWaves * 64) void decode_kernel(
    const T* __restrict__ q, T* __restrict__ out, T* __restrict__ kpool, T* __restrict__ vpool,
    int64_t num_blocks, const int32_t* __restrict__ plan, int32_t stride, int32_t n_kv_heads,
    float scale_log2, const T* __restrict__ k_new, const T* __restrict__ v_new,
    const int32_t* __restrict__ slot_mapping, float* part_o, float* part_ml, uint32_t o_bytes,
    uint32_t ml_bytes, int32_t* counters, int32_t* status) {
  typedef typename Mma<T>::vec8 vec8;
  typedef typename Mma<T>::vec4 vec4;
  typedef PartLayout<D, G> PL;
  typedef Tile<T, D> TL;
  constexpr int PS = 16;
  constexpr int NCH = D / 32;          // QK MFMA k-chunks per head row
  constexpr int NDB = D / 16;          // PV MFMA dim blocks
  constexpr int RB = TL::RB;           // bytes of one head's row
  constexpr int CPR = RB / 16;         // 16-byte chunks per head row
  constexpr int RPI = 64 / CPR;        // rows per wave load instruction
  constexpr int NLD = PS / RPI;        // load instructions per page and tensor
  constexpr int RS = TL::RS;
  constexpr int NGR = PL::NGR;
  constexpr int OPS = 2 * NLD;         // vector memory instructions per page load
  static_assert(NLD * RPI == PS && CPR * RPI == 64, "a wave loads whole head rows");

  extern __shared__ __align__(16) unsigned char smem[];
  PKV_TL(const unsigned long long tl_start = __builtin_amdgcn_s_memrealtime();
         unsigned long long tl_first = 0, tl_merge = 0; int tl_merges = 0;)
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int hgw = heads_per_wg(n_kv_heads);          // KV heads of this workgroup (waves)
  // grid (head groups, bins): the bin's plan block needs no division, so its
  // address is ready as soon as the kernel arguments are, and workgroups
  // dispatch in (bin, group) order (a bin's groups on neighbouring XCDs:
  // measured 2% faster than the two on one XCD)
  const int bin = blockIdx.y;
  const int h = blockIdx.x * hgw + wave;             // this wave's KV head
  const int Hq = n_kv_heads * G;
  const uint32_t frow = (uint32_t)(n_kv_heads * RB);        // bytes per token row
  const int64_t row_elems = (int64_t)n_kv_heads * D;
  unsigned char* kl = smem + wave * TL::BYTES;       // this wave's tile: K rows
  unsigned char* vl = kl + PS * RS;                  // then V rows
  const int n = lane & 15;   // MFMA row/column within a 16-lane block
  const int g = lane >> 4;   // MFMA k-group

  const int32_t* bp = plan + (int64_t)bin * stride;
  const int32_t* words = bp + kHdrInts;
  const int32_t* items_end = bp + stride;   // item i: items_end - (i + 1) * kItemInts
  typedef Stage<T, D, G> SG;
  static_assert(SG::C <= kStageMax, "the first batch's items lie inside the block");
  // read together with the header: the first batch's (seq, flags), the
  // first item and the first two page words
  int sq0[SG::C], fl0[SG::C];
#pragma unroll
  for (int j = 0; j < SG::C; ++j) {
    sq0[j] = items_end[-(j + 1) * kItemInts];
    fl0[j] = items_end[-(j + 1) * kItemInts + 7];
  }
  struct Item { int seq, np, tok0, kv, slot, nparts, slot0, flags; };
  auto item_at = [&](int i) __attribute__((always_inline)) -> Item {
    const int32_t* it = items_end - (int64_t)(i + 1) * kItemInts;
    return Item{it[0], it[1], it[2], it[3], it[4], it[5], it[6], it[7]};
  };
  Item cur = item_at(0);
  // the next item's fields, read one item ahead (the slot below a bin's last
  // item still lies inside its plan block: header and page words precede it)
  Item nxt = item_at(1);
  int wcur = words[0];
  int wnext = words[1];
  const int n_items = bp[0], n_pages = bp[1];
  // (keeps every one of these reads ahead of the branch below, so they go
  // out together instead of after it)
#pragma unroll
  for (int j = 0; j < SG::C; ++j) asm volatile("" ::"s"(sq0[j]), "s"(fl0[j]));
  asm volatile("" ::"s"(cur.seq), "s"(cur.np), "s"(cur.tok0), "s"(cur.kv), "s"(cur.slot),
               "s"(cur.nparts), "s"(cur.slot0), "s"(cur.flags), "s"(wcur), "s"(wnext), "s"(q),
               "s"(k_new), "s"(v_new));
  if (n_items <= 0) return;

  // This lane's chunk of a page: row k * RPI + lane / CPR, bytes
  // (lane % CPR) * 16 of the head's slice -- CPR lanes cover a row, so every
  // load instruction reads whole cache lines.
  const int lrow0 = lane / CPR;
  const uint32_t lcol = (uint32_t)(lane % CPR) * 16;
  // Page p of the stream (p wave-uniform, word w = words[p]); past the
  // bin's last page every load is outside its range: no access, zeros.
  auto load_page = [&](int p, int w, vec8* kr, vec8* vr) __attribute__((always_inline)) {
    const bool in = p < n_pages;
    const int64_t page = in ? (w & ((1 << kPageIdBits) - 1)) : 0;
    const uint32_t live = in ? (((uint32_t)w >> kPageIdBits) & 15u) + 1u : 0u;
    const __amdgpu_buffer_rsrc_t rk = ws_rsrc(kpool + page * PS * row_elems, live * frow);
    const __amdgpu_buffer_rsrc_t rv = ws_rsrc(vpool + page * PS * row_elems, live * frow);
#pragma unroll
    for (int k = 0; k < NLD; ++k) {
      const uint32_t off = (uint32_t)(k * RPI + lrow0) * frow + (uint32_t)(h * RB) + lcol;
      kr[k] = __builtin_bit_cast(vec8, __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, kNt));
      vr[k] = __builtin_bit_cast(vec8, __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, kNt));
    }
  };
  // ---- items: fields from the plan (scalar loads); Q and the new row of
  // SG::C items at a time staged in this wave's LDS slots, loaded in one
  // batch (the first batch before the first pages, so waiting for it never
  // waits for a page).
  const bool fuse = k_new != nullptr;
  unsigned char* stg = smem + hgw * TL::BYTES + wave * SG::BYTES;
  // Loads of the slots of items i0 .. i0 + C - 1: lane chunk c = 64 r + lane
  // is 16 bytes w of item i's slot (Q rows of the KV head's G query heads,
  // then the KV head's slice of the new K row and of the new V row).
  // (seq, flags) of items i0 .. i0 + C - 1 (the last item repeated past the end)
  auto stage_fields = [&](int i0, int* sq, int* fl) __attribute__((always_inline)) {
    const int ns = min(SG::C, n_items - i0);
#pragma unroll
    for (int j = 0; j < SG::C; ++j) {
      const int32_t* it = items_end - (int64_t)(i0 + min(j, ns - 1) + 1) * kItemInts;
      sq[j] = it[0];
      fl[j] = it[7];
    }
  };
  auto stage_load = [&](int i0, const int* sq, const int* fl, u32x4* d)
                        __attribute__((always_inline)) {
    const int ns = min(SG::C, n_items - i0);
#pragma unroll
    for (int r = 0; r < SG::ROUNDS; ++r) {
      const int c = r * 64 + lane;
      const int i = c / SG::CPI, w = c - i * SG::CPI;
      // item i's fields by masks (a select chain here becomes a lookup
      // table in scratch memory)
      int si = 0, fi = 0;
#pragma unroll
      for (int j = 0; j < SG::C; ++j) {
        const int msk = -(int)(i == j);
        si |= sq[j] & msk;
        fi |= fl[j] & msk;
      }
      const unsigned char* src = nullptr;
      if (i < ns) {
        if (w < SG::QC)
          src = reinterpret_cast<const unsigned char*>(q + ((int64_t)si * Hq + h * G) * D) + w * 16;
        else if (fuse && (fi & kItemLast))
          src = reinterpret_cast<const unsigned char*>(
                    (w < SG::QC + SG::RC ? k_new : v_new) + (int64_t)si * row_elems + h * D) +
                (w < SG::QC + SG::RC ? w - SG::QC : w - SG::QC - SG::RC) * 16;
      }
      // each read once per item: streaming hint
      d[r] = src ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src))
                 : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto stage_store = [&](const u32x4* d) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < SG::ROUNDS; ++r) {
      const int c = r * 64 + lane;
      if (c < SG::C * SG::CPI) *reinterpret_cast<u32x4*>(stg + c * 16) = d[r];
    }
    wave_lds_sync();
  };
  u32x4 sgd[SG::ROUNDS];
  stage_load(0, sq0, fl0, sgd);
  // One page in flight: its registers and its word; the next page's word is
  // read a step ahead.
  vec8 kr[NLD], vr[NLD];
  load_page(0, wcur, kr, vr);
  stage_store(sgd);

  vec8 qb[NCH], kx{}, vx{};
  int new_slot = 0;
  // Item i (slot i % C staged) becomes current: Q^T as the QK B operand
  // (column n = query head h*G + n, zero beyond G) and this lane's 16 bytes
  // of the new row.
  auto take_item = [&](int i) __attribute__((always_inline)) {
    const unsigned char* sl = stg + (i % SG::C) * SG::SLOT;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const vec8 t = *reinterpret_cast<const vec8*>(
          sl + ((n < G ? n : 0) * D + c * 32 + g * 8) * (int)sizeof(T));
      qb[c] = (n < G) ? t : vec8{};
    }
    kx = *reinterpret_cast<const vec8*>(sl + SG::QB + lcol);
    vx = *reinterpret_cast<const vec8*>(sl + SG::QB + RB + lcol);
    new_slot = (fuse && (cur.flags & kItemLast)) ? slot_mapping[cur.seq] : 0;
  };
  take_item(0);
  int it_idx = 0;
  int it_start = 0, it_end = cur.np;   // the current item's pages in the stream

  f32x4 o[NDB];
  float m_run = -INFINITY, l_run = 0.f;  // per head column n (replicated over g)
#pragma unroll
  for (int b = 0; b < NDB; ++b) o[b] = f32x4{0.f, 0.f, 0.f, 0.f};

  const __amdgpu_buffer_rsrc_t ro = ws_rsrc(part_o, o_bytes);
  const __amdgpu_buffer_rsrc_t rm = ws_rsrc(part_ml, ml_bytes);

  // Lane 4 g + i's value of v, in every lane of group g (heads 4 g + i < G;
  // other groups, whose rows are padding, get 1)
  auto from_lane = [&](float v, int i) __attribute__((always_inline)) {
    float x = 1.f;
#pragma unroll
    for (int gg = 0; 4 * gg < G; ++gg) {
      x = g == gg ? lane_value(v, 4 * gg + i) : x;
    }
    return x;
  };

  // Deferred stores. A whole sequence's output is normalised at the item's
  // end into the next entry of this wave's LDS output ring (lane (dim column
  // n, group g) holds heads 4g..4g+3 of dims 16b + n), and the fused
  // append's new row slices go to the row ring instead of the pool. A full
  // ring is stored in 16-byte pieces at the start of the next step, before
  // that step's page loads, and whatever the rings hold at the end of the
  // stream: a bin of many short sequences then writes in a few bursts
  // instead of a round of stores among the page reads at every item
  // (capacity phase A, 16 sequences a bin: 67.5 against 75.5 us a launch).
  // No other wave of the launch reads a new row's slot (the fusion's
  // precondition), and the kernel patches its own loaded copy at once, so
  // the deferral changes no result. Stores issued after a page's loads
  // would make the single wait at the top of the loop, which serves every
  // path, also wait for them; issued before them, they complete within the
  // wait for the page.
  typedef Rings<T, D, G> RG;
  unsigned char* rrow = smem + hgw * (TL::BYTES + SG::BYTES) + wave * RG::BYTES;
  int32_t* rrow_slot = reinterpret_cast<int32_t*>(rrow + RG::KR * RG::RB2);
  unsigned char* ring = rrow + RG::ROWS;
  int32_t* ring_seq = reinterpret_cast<int32_t*>(ring + RG::KO * RG::OB);
  int n_out = 0;    // outputs the output ring holds
  int n_rows = 0;   // row slices the row ring holds
  bool rows_full = false;
  // The row ring's first `cnt` entries to the pools: 16-byte piece c is
  // piece c % NCR of entry c / NCR (K slice, then V slice). Both rings are
  // written with the streaming hint: nothing in this launch reads them back.
  auto write_rows = [&](int cnt) __attribute__((always_inline)) {
    constexpr int NCR = RG::RB2 / 16;
    constexpr int HALF = NCR / 2;
#pragma unroll 1
    for (int c0 = 0; c0 < cnt * NCR; c0 += 64) {
      const int c = c0 + lane;
      if (c < cnt * NCR) {
        const int e = c / NCR, part = c - e * NCR;
        unsigned char* d = reinterpret_cast<unsigned char*>(
            (part < HALF ? kpool : vpool) + (int64_t)rrow_slot[e] * row_elems);
        __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(rrow + c * 16),
                                    reinterpret_cast<u32x4*>(d + h * RB + (part % HALF) * 16));
      }
    }
  };
  auto finish_out = [&]() __attribute__((always_inline)) {
    unsigned char* ol = ring + n_out * RG::OB;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * g + i;
      const float li = from_lane(l_run, i);  // lane r holds head r's sum
      if (r < G) {
        const float inv = 1.f / li;   // one division per row, not per element
#pragma unroll
        for (int b = 0; b < NDB; ++b)
          *reinterpret_cast<T*>(ol + (r * D + 16 * b + n) * (int)sizeof(T)) = (T)(o[b][i] * inv);
      }
    }
  };
  // The ring's first `cnt` rows to out: 16-byte piece c is piece c % NCK of
  // row c / NCK. (A rolled loop: unrolled, its loads stay live and cost
  // 30 VGPRs.)
  auto write_out = [&](int cnt) __attribute__((always_inline)) {
    constexpr int NCK = RG::OB / 16;
#pragma unroll 1
    for (int c0 = 0; c0 < cnt * NCK; c0 += 64) {
      const int c = c0 + lane;
      if (c < cnt * NCK) {
        const int row = c / NCK;
        T* dst = out + ((int64_t)ring_seq[row] * Hq + h * G) * D;
        __builtin_nontemporal_store(
            *reinterpret_cast<const u32x4*>(ring + c * 16),
            reinterpret_cast<u32x4*>(reinterpret_cast<unsigned char*>(dst) + (c - row * NCK) * 16));
      }
    }
  };
  bool ring_full = false;

  // The current item's last page: write the new row (fused append) and patch
  // the loaded copy when slot_mapping agrees with the page table.
  auto append_row = [&](int w, vec8* kq, vec8* vq) __attribute__((always_inline)) {
    const int tl = (cur.kv - 1) % PS;  // newest token's row within its page
    const int64_t page = w & ((1 << kPageIdBits) - 1);
    const bool in_range = new_slot >= 0 && (int64_t)new_slot < num_blocks * PS;
    if (!in_range) {
      if (lane == 0) flag(status, PKV_STATUS_BAD_SLOT);
      return;
    }
    const bool patch = (int64_t)new_slot == page * PS + tl;
    if constexpr (RG::KR > 0) {   // into the row ring's next entry
      unsigned char* e = rrow + n_rows * RG::RB2;
      if (lane == 0) rrow_slot[n_rows] = new_slot;
      rows_full = ++n_rows == RG::KR;
#pragma unroll
      for (int k = 0; k < NLD; ++k) {
        if (k * RPI + lrow0 == tl) {
          *reinterpret_cast<vec8*>(e + lcol) = kx;
          *reinterpret_cast<vec8*>(e + RB + lcol) = vx;
          if (patch) {
            kq[k] = kx;
            vq[k] = vx;
          }
        }
      }
    } else {                      // into the pools at once
      unsigned char* kd = reinterpret_cast<unsigned char*>(kpool + new_slot * row_elems);
      unsigned char* vd = reinterpret_cast<unsigned char*>(vpool + new_slot * row_elems);
#pragma unroll
      for (int k = 0; k < NLD; ++k) {
        if (k * RPI + lrow0 == tl) {
          *reinterpret_cast<vec8*>(kd + h * RB + lcol) = kx;
          *reinterpret_cast<vec8*>(vd + h * RB + lcol) = vx;
          if (patch) {
            kq[k] = kx;
            vq[k] = vx;
          }
        }
      }
    }
  };

  // Merge (seq, h) from the stored partials and reset its counter.
  auto merge = [&](int sq, int nparts, int slot0, bool own) __attribute__((always_inline)) {
    PKV_TL(const unsigned long long tm = __builtin_amdgcn_s_memrealtime(); ++tl_merges;)
    merge_head<T, D, G>(out, reinterpret_cast<float*>(kl), sq, h, n_kv_heads, nparts, slot0,
                        ro, rm, own, o, m_run, l_run);
    if (lane == 0)
      __hip_atomic_store(counters + (int64_t)sq * n_kv_heads + h, 0, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    PKV_TL(tl_merge += __builtin_amdgcn_s_memrealtime() - tm;)
  };
  // Count an arrival whose partial has completed; the returned count.
  auto arrive = [&](int sq) __attribute__((always_inline)) -> int {
    int old = 0;
    if (lane == 0)
      old = __hip_atomic_fetch_add(counters + (int64_t)sq * n_kv_heads + h, 1, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    return old;
  };
  // A deferred arrival: pa_state 1 once a partial is stored; it is counted
  // at page pa_at.
  int pa_state = 0, pa_at = 0, pa_seq = 0, pa_nparts = 0, pa_slot0 = 0, pa_old = 0;
  // check a counted arrival: the last one merges
  auto finish_arrival = [&]() __attribute__((always_inline)) {
    if (__builtin_amdgcn_readfirstlane(pa_old) == pa_nparts - 1)
      merge(pa_seq, pa_nparts, pa_slot0, false);
    pa_state = 0;
  };
  auto flush_arrival = [&]() __attribute__((always_inline)) {  // count a pending arrival now
    if (pa_state == 1) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      pa_old = arrive(pa_seq);
      finish_arrival();
    }
  };
  int b_count = 0;   // the arrival counter as the last piece of a cut sequence found it

  // Item end: the output (whole sequence), or the partial of a cut sequence.
  auto end_item = [&](int p) __attribute__((always_inline)) {
    if (cur.slot < 0) {
      finish_out();
      if (lane == 0) ring_seq[n_out] = cur.seq;
      ring_full = ++n_out == RG::KO;
    } else {
      flush_arrival();   // at most one deferred arrival at a time
      const bool last = cur.flags & kItemLast;
      if (last && __builtin_amdgcn_readfirstlane(b_count) == cur.nparts - 1) {
        // the sequence's last piece, and every other piece had arrived when
        // it started: it merges, its own partial straight from registers,
        // and publishes nothing
        merge(cur.seq, cur.nparts, cur.slot0, true);
      } else {
        const uint32_t head_off =
            (uint32_t)(((int64_t)cur.slot * n_kv_heads + h) * PL::FLOATS * 4);
        if (g < NGR) {
#pragma unroll
          for (int b = 0; b < NDB; ++b)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o[b]), ro,
                                                   head_off + ((g * NDB + b) * 16 + n) * 16, 0,
                                                   kSc1);
        }
        if (lane < G)
          __builtin_amdgcn_raw_buffer_store_b64(
              __builtin_bit_cast(u32x2, f32x2{m_run, l_run}), rm,
              (uint32_t)(((int64_t)cur.slot * Hq + h * G + lane) * 8), 0, kSc1);
        asm volatile("" ::: "memory");  // the stores stay before the loads that follow
        pa_seq = cur.seq;
        pa_nparts = cur.nparts;
        pa_slot0 = cur.slot0;
        if (!last && p + 2 < n_pages) {
          // count it once a page loaded after the stores has arrived
          pa_state = 1;
          pa_at = p + 2;
        } else {
          // the last piece with others still out, or the stream ends: count
          // it now; whichever piece arrives last merges
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
          pa_old = arrive(cur.seq);
          finish_arrival();
        }
      }
    }
    ++it_idx;
    if (it_idx < n_items) {
      if (it_idx % SG::C == 0) {   // the next batch of slots
        int sq[SG::C], fl[SG::C];
        stage_fields(it_idx, sq, fl);
        stage_load(it_idx, sq, fl, sgd);
        stage_store(sgd);
      }
      cur = nxt;
      nxt = item_at(it_idx + 1);
      take_item(it_idx);
      it_start = it_end;
      it_end += cur.np;
      m_run = -INFINITY;
      l_run = 0.f;
#pragma unroll
      for (int b = 0; b < NDB; ++b) o[b] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };

  auto compute = [&](int p) __attribute__((always_inline)) {
    const int tp = cur.tok0 + (p - it_start) * PS;  // first token of the page
    // S^T: lane (n, g) gets the scores of tokens 4g..4g+3 for head n.
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    const unsigned char* kp = kl + n * RS + g * 16;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      acc = Mma<T>::qk(*reinterpret_cast<const vec8*>(kp + c * 64), qb[c], acc);
    float sc[4];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sc[i] = tp + 4 * g + i < cur.kv ? acc[i] * scale_log2 : -INFINITY;
      mx = fmaxf(mx, sc[i]);
    }
    mx = max_x32(max_x16(mx));
    // Lazy rescale: the reference max moves only when some head's max
    // grows by more than 2^8, so p <= 256 and o / l is unchanged.
    if (__builtin_amdgcn_ballot_w64(mx > m_run + 8.f)) {
      const float m_new = fmaxf(m_run, mx);  // finite: every page has a live token
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
      m_run = m_new;
      // lane (n, g) holds output rows 4g+i, whose factor lives in lane 4g+i
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a = from_lane(alpha, i);
#pragma unroll
        for (int b = 0; b < NDB; ++b) o[b][i] *= a;
      }
    }
    vec4 pr;
    float ls = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float e = __builtin_amdgcn_exp2f(sc[i] - m_run);
      ls += e;
      pr[i] = (T)e;
    }
    ls = sum_x32(sum_x16(ls));
    l_run += ls;
    const unsigned char* vp = vl + (4 * g + (n >> 2)) * RS + 4 * (n & 3) * (int)sizeof(T);
#pragma unroll
    for (int b = 0; b < NDB; ++b) {
      const i16x4 raw = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_i16x4*)(vp + 16 * b * sizeof(T)));
      o[b] = Mma<T>::pv(pr, __builtin_bit_cast(vec4, raw), o[b]);
    }
  };

  // Step p: stage page p into the wave's tile (patched with the new row at
  // a sequence's last page), send the loads of page p + 1 into the same
  // registers, then compute page p. Every step issues exactly one page's
  // loads (past the bin's last page: no access), so on every path through
  // the loop the wait for page p counts only page p's loads.
  for (int p = 0; p < n_pages; ++p) {
    if (fuse && (cur.flags & kItemLast) && p == it_end - 1) append_row(wcur, kr, vr);
    if (wcur < 0 && lane == 0) flag(status, PKV_STATUS_BAD_PAGE);
#pragma unroll
    for (int k = 0; k < NLD; ++k) {
      const uint32_t loff = (uint32_t)(k * RPI + lrow0) * RS + lcol;
      *reinterpret_cast<vec8*>(kl + loff) = kr[k];
      *reinterpret_cast<vec8*>(vl + loff) = vr[k];
    }
    wave_lds_sync();
    if (RG::KR > 0 && rows_full) {   // full rings, before this step's loads
      write_rows(RG::KR);
      rows_full = false;
      n_rows = 0;
    }
    if (ring_full) {
      write_out(RG::KO);
      ring_full = false;
      n_out = 0;
    }
    if (p == it_start && (cur.flags & kItemLast) && cur.slot >= 0 && lane == 0)
      b_count = __hip_atomic_load(counters + (int64_t)cur.seq * n_kv_heads + h,
                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    wcur = wnext;
    wnext = words[p + 2];   // inside the plan block: its words are followed by items
    load_page(p + 1, wcur, kr, vr);
    compute(p);
    PKV_TL(if (p == 0) tl_first = __builtin_amdgcn_s_memrealtime();)
    // (after compute: a merge below uses the wave's tile as scratch)
    if (pa_state != 0 && p == pa_at) {
      // Page p's loads were issued after the partial's stores and have
      // arrived (vmcnt counts in order); only page p + 1's loads may still
      // be outstanding, so this wait leaves the stores complete.
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(OPS) : "memory");
      pa_old = arrive(pa_seq);
      finish_arrival();
    }
    if (p == it_end - 1) end_item(p);
    wave_lds_sync();  // this page's tile reads are done before the next copy
  }
  PKV_TL(const unsigned long long tl_last = __builtin_amdgcn_s_memrealtime();)
  if (n_rows + n_out > 0) wave_lds_sync();   // the last entries and their ids
  if (RG::KR > 0 && n_rows > 0) write_rows(n_rows);
  if (n_out > 0) write_out(n_out);
  flush_arrival();
#ifdef PKV_TIMELINE
  {
    const int wid = (blockIdx.y * gridDim.x + blockIdx.x) * hgw + wave;
    const unsigned long long tl_end = __builtin_amdgcn_s_memrealtime();
    if (lane < 8 && wid < kTimelineWaves) {
      const unsigned long long rec[8] = {tl_start, tl_first, tl_last, tl_end,
                                         (unsigned long long)n_pages, (unsigned long long)n_items,
                                         (unsigned long long)tl_merges, tl_merge};
      unsigned long long v = rec[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) v = lane == i ? rec[i] : v;
      pkv_timeline[(int64_t)wid * 8 + lane] = v;
    }
  }
#endif
}

template <typename T, int D, int G>
static size_t decode_lds_bytes(int hgw) {
  return (size_t)hgw * (Tile<T, D>::BYTES + Stage<T, D, G>::BYTES + Rings<T, D, G>::BYTES);
}

template <typename T, int D, int G>
static void launch(const void* q, void* out, void* kp, void* vp, int64_t nb,
                   const int32_t* plan, int32_t n_work, int32_t stride, int32_t Hkv, float sl2,
                   const void* kn, const void* vn, const int32_t* slots, float* po, float* pml,
                   uint32_t o_bytes, uint32_t ml_bytes, int32_t* cnt, int32_t* status,
                   hipStream_t s) {
  const int hgw = heads_per_wg(Hkv);
  const size_t lds = decode_lds_bytes<T, D, G>(hgw);
  const int groups = Hkv / hgw;
  hipLaunchKernelGGL((decode_kernel<T, D, G>), dim3((unsigned)groups, (unsigned)(n_work / groups)),
                     dim3(hgw * 64), lds, s, (const T*)q, (T*)out, (T*)kp, (T*)vp, nb, plan,
                     stride, Hkv, sl2, (const T*)kn, (const T*)vn, slots, po, pml, o_bytes,
                     ml_bytes, cnt, status);
}

// Workgroups of decode_kernel<T, D, G> that stay resident on one compute
// unit (registers and LDS), 0 on error.
template <typename T, int D, int G>
static int resident(int Hkv) {
  const int hgw = heads_per_wg(Hkv);
  int n = 0;
  const size_t lds = decode_lds_bytes<T, D, G>(hgw);
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_kernel<T, D, G>, hgw * 64, lds) !=
      hipSuccess)
    return 0;
  return n;
}

typedef void (*LaunchFn)(const void*, void*, void*, void*, int64_t, const int32_t*, int32_t,
                         int32_t, int32_t, float, const void*, const void*, const int32_t*,
                         float*, float*, uint32_t, uint32_t, int32_t*, int32_t*, hipStream_t);
typedef int (*ResidentFn)(int);
struct Variant { LaunchFn launch; ResidentFn resident; };

template <typename T, int D>
static Variant pick_g(int G) {
  switch (G) {
    case 1: return {launch<T, D, 1>, resident<T, D, 1>};
    case 2: return {launch<T, D, 2>, resident<T, D, 2>};
    case 4: return {launch<T, D, 4>, resident<T, D, 4>};
    case 8: return {launch<T, D, 8>, resident<T, D, 8>};
    case 16: return {launch<T, D, 16>, resident<T, D, 16>};
    default: return {nullptr, nullptr};
  }
}

static Variant fast_variant(int32_t dtype, int32_t Hkv, int32_t D, int32_t G,
                            int32_t page_size) {
  if (page_size != 16 || Hkv < 1) return {nullptr, nullptr};
  if (dtype == PKV_DTYPE_F16) {
    if (D == 64) return pick_g<_Float16, 64>(G);
    if (D == 128) return pick_g<_Float16, 128>(G);
  } else if (dtype == PKV_DTYPE_BF16) {
    if (D == 64) return pick_g<__bf16, 64>(G);
    if (D == 128) return pick_g<__bf16, 128>(G);
  }
  return {nullptr, nullptr};
}

static LaunchFn fast_decode(int32_t dtype, int32_t Hkv, int32_t D, int32_t G,
                            int32_t page_size, int32_t pp) {
  if (pp < 1 || pp > kMaxPartPages) return nullptr;
  return fast_variant(dtype, Hkv, D, G, page_size).launch;
}

// Floats of partial output per (slot, KV head): the accumulator tile of
// ceil(G/4) groups of 4 head rows.
static int64_t part_floats(int32_t G, int32_t D) { return (int64_t)((G + 3) / 4) * 4 * D; }

// generic fallback lives in attention.hip
int generic_decode(const void* q, void* out, const void* kp, const void* vp, int64_t nb,
                   const int32_t* indptr, const int32_t* indices, const int32_t* kv_lens,
                   int32_t n_seqs, int32_t Hq, int32_t Hkv, int32_t D, int32_t ps, float scale,
                   int32_t dtype, int32_t* status, hipStream_t s);
int check_seq_pages(int32_t i, int32_t np, int32_t kv, int32_t last, int32_t ps);
int check_geometry(int32_t Hq, int32_t Hkv, int32_t D, int32_t ps, int32_t dtype);

}  // namespace pkv

using namespace pkv;

extern "C" int pkv_decode_fast_path(int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                    int32_t page_size, int32_t dtype, int32_t part_pages) {
  if (n_kv_heads <= 0 || n_heads % n_kv_heads) return 0;
  return fast_decode(dtype, n_kv_heads, head_dim, n_heads / n_kv_heads, page_size, part_pages)
             ? 1 : 0;
}

extern "C" int pkv_decode_workgroups(int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                     int32_t dtype, int32_t per_cu) {
  if (n_kv_heads <= 0 || n_heads % n_kv_heads || per_cu <= 0) return 0;
  const Variant v = fast_variant(dtype, n_kv_heads, head_dim, n_heads / n_kv_heads, 16);
  if (!v.resident) return 0;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  const int fit = v.resident(n_kv_heads);
  return cus * std::min(per_cu, fit);
}

extern "C" int pkv_plan_decode(const int32_t* kv_indptr, const int32_t* kv_indices,
                               const int32_t* kv_lens, const int32_t* kv_last_page_len,
                               int32_t n_seqs, int32_t page_size, int64_t num_blocks,
                               int32_t n_kv_heads, int32_t part_pages, int32_t max_workgroups,
                               int32_t* plan, int64_t plan_capacity, int64_t* plan_needed,
                               int32_t* n_work_out, int32_t* n_slots_out,
                               int32_t* plan_stride_out) {
  if (n_seqs <= 0 || page_size <= 0 || part_pages <= 0 || part_pages > kMaxPartPages)
    return fail(PKV_ERR_INVALID, "n_seqs and page_size must be positive and part_pages in "
                "[1, %d]", kMaxPartPages);
  if (page_size > 16)
    return fail(PKV_ERR_INVALID, "page_size=%d: the decode plan holds at most 16 rows a page",
                page_size);
  if (n_kv_heads <= 0 || max_workgroups <= 0)
    return fail(PKV_ERR_INVALID, "n_kv_heads and max_workgroups must be positive");
  if (num_blocks <= 0 || num_blocks > (1LL << kPageIdBits))
    return fail(PKV_ERR_INVALID, "num_blocks=%lld outside [1, 2^%d] (decode plan page words)",
                (long long)num_blocks, kPageIdBits);
  if (kv_indptr[0] != 0) return fail(PKV_ERR_INVALID, "kv_indptr must start at 0");
  // Pieces of every sequence (part_pages pages each, the remainder last,
  // folded into the piece before it when shorter than both kMinTail and half
  // a piece), and slots
  // for cut sequences. Role: 0 a cut sequence's piece before its last, 1 a
  // whole sequence, 2 a cut sequence's last piece (it merges).
  struct Item { int32_t seq, first, np, slot, nparts, slot0, role; int64_t cost; };
  std::vector<Item> items;
  items.reserve(n_seqs);
  int32_t slots = 0;
  for (int32_t i = 0; i < n_seqs; ++i) {
    const int32_t np = kv_indptr[i + 1] - kv_indptr[i];
    int rc = check_seq_pages(i, np, kv_lens[i], kv_last_page_len[i], page_size);
    if (rc) return rc;
    const int32_t full = np / part_pages, rem = np % part_pages;
    const bool fold = full > 0 && rem > 0 && rem < std::min(kMinTail, (part_pages + 1) / 2);
    const int32_t k = full + (rem > 0 && !fold ? 1 : 0);
    int32_t first = 0;
    for (int32_t p = 0; p < k; ++p) {
      const int32_t m = p < full ? part_pages + (fold && p + 1 == full ? rem : 0) : rem;
      const int32_t role = k == 1 ? 1 : p + 1 == k ? 2 : 0;
      // cost in 1/16 pages: the pages, a start-up per piece (Q, output) and,
      // for a last piece, the merge it runs at the end of its bin
      const int64_t cost = (int64_t)m * 16 + 4 + (role == 2 ? 40 : 0);
      items.push_back({i, first, m, k > 1 ? slots + p : -1, k, k > 1 ? slots : -1, role, cost});
      first += m;
    }
    if (k > 1) slots += k;
  }
  const int hgw = heads_per_wg(n_kv_heads);
  const int n_groups = n_kv_heads / hgw;
  int64_t bins = std::max<int64_t>(1, max_workgroups / n_groups);
  bins = std::min<int64_t>(bins, (int64_t)items.size());
  // A cut piece at least half a bin long usually ends its bin, so the
  // publish / count / merge chain after its last page adds to that bin's
  // time instead of overlapping the next piece's pages: it is charged 72
  // (4.5 pages) instead of the last piece's 40 (measured on the batch-256
  // decode step: 1.4% faster; no change where bins hold many pieces).
  {
    int64_t total = 0;
    for (const Item& x : items) total += (int64_t)x.np * 16;
    const int64_t half_bin = total / bins / 2;
    for (Item& x : items)
      if (x.role != 1 && (int64_t)x.np * 16 >= half_bin) x.cost = (int64_t)x.np * 16 + 4 + 72;
  }
  // longest-processing-time-first deal into the least-loaded bin
  std::vector<int32_t> order(items.size());
  for (size_t i = 0; i < order.size(); ++i) order[i] = (int32_t)i;
  std::stable_sort(order.begin(), order.end(),
                   [&](int32_t a, int32_t b) { return items[a].cost > items[b].cost; });
  typedef std::pair<int64_t, int32_t> Load;  // (work, bin)
  std::priority_queue<Load, std::vector<Load>, std::greater<Load>> heap;
  for (int32_t b = 0; b < bins; ++b) heap.push({0, b});
  // (flat arrays: the bin of every item in dealing order, then the items of
  // each bin gathered by a counting sort, so planning allocates nothing per bin)
  const size_t n_items = items.size();
  std::vector<int32_t> bin_of(n_items), bin_count((size_t)bins + 1, 0);
  std::vector<int64_t> bin_pages((size_t)bins, 0);
  for (int32_t ix : order) {
    Load l = heap.top();
    heap.pop();
    bin_of[ix] = l.second;
    ++bin_count[l.second + 1];
    bin_pages[l.second] += items[ix].np;
    heap.push({l.first + items[ix].cost, l.second});
  }
  int64_t stride = kHdrInts + kStageMax * kItemInts;
  for (int64_t b = 0; b < bins; ++b)
    stride = std::max<int64_t>(stride, kHdrInts + ((bin_pages[b] + 3) & ~3LL) +
                                           kItemInts * (int64_t)bin_count[b + 1]);
  // in a bin: pieces before a cut sequence's last, whole sequences, then last
  // pieces, each in dealing order (longest first): a stable sort by (bin, role)
  for (int64_t b = 0; b < bins; ++b) bin_count[b + 1] += bin_count[b];
  std::vector<int32_t> by_bin(n_items);
  {
    std::vector<int32_t> fill(bin_count.begin(), bin_count.end() - 1);
    for (int role = 0; role < 3; ++role)
      for (int32_t ix : order)
        if (items[ix].role == role) by_bin[fill[bin_of[ix]]++] = ix;
  }
  const int64_t need = bins * stride + kPlanTail;
  if (plan_needed) *plan_needed = need;
  if (stride > 0x7fffffff || need > plan_capacity)
    return fail(PKV_ERR_CAPACITY, "decode plan needs %lld entries, capacity %lld",
                (long long)need, (long long)plan_capacity);
  std::fill(plan, plan + need, 0);
  for (int64_t b = 0; b < bins; ++b) {
    int32_t* bp = plan + b * stride;
    bp[0] = bin_count[b + 1] - bin_count[b];
    bp[1] = (int32_t)bin_pages[b];
    int32_t* w = bp + kHdrInts;
    for (int32_t j = bin_count[b]; j < bin_count[b + 1]; ++j) {
      int32_t* it = bp + stride - (int64_t)(j - bin_count[b] + 1) * kItemInts;
      const Item& x = items[by_bin[j]];
      const int32_t np_seq = kv_indptr[x.seq + 1] - kv_indptr[x.seq];
      for (int32_t t = 0; t < x.np; ++t) {
        const int32_t pg = x.first + t;
        const int32_t id = kv_indices[kv_indptr[x.seq] + pg];
        const bool bad = id < 0 || (int64_t)id >= num_blocks;
        const int32_t live = pg == np_seq - 1 ? kv_last_page_len[x.seq] : page_size;
        *w++ = (int32_t)((uint32_t)(bad ? 0 : id) | ((uint32_t)(live - 1) << kPageIdBits) |
                         (bad ? 0x80000000u : 0u));
      }
      const bool last = x.first + x.np == np_seq;
      const int32_t vals[kItemInts] = {x.seq, x.np, x.first * page_size, kv_lens[x.seq],
                                       x.slot, x.nparts, x.slot0, last ? kItemLast : 0};
      for (int k = 0; k < kItemInts; ++k) *it++ = vals[k];
    }
  }
  *n_work_out = (int32_t)(bins * n_groups);
  *n_slots_out = slots;
  *plan_stride_out = (int32_t)stride;
  return PKV_OK;
}

// Workspace: the arrival counters (n_seqs x n_kv_heads, padded to 256 bytes),
// then the partial outputs and the (m, l) pairs. Every counter is zero
// before a launch and after it.
static int64_t counter_bytes(int32_t n_seqs, int32_t n_kv_heads) {
  return ((int64_t)n_seqs * n_kv_heads * 4 + 255) / 256 * 256;
}

extern "C" int64_t pkv_decode_workspace_bytes(int32_t n_seqs, int32_t n_slots,
                                              int32_t n_heads, int32_t n_kv_heads,
                                              int32_t head_dim) {
  if (n_seqs <= 0 || n_kv_heads <= 0 || n_slots <= 0 || n_heads <= 0) return 0;
  if (n_heads % n_kv_heads) return 0;
  const int64_t po = (int64_t)n_slots * n_kv_heads * part_floats(n_heads / n_kv_heads, head_dim);
  return counter_bytes(n_seqs, n_kv_heads) + (po + (int64_t)n_slots * n_heads * 2) * 4;
}

namespace pkv {

// The decode launch shared by both entry points. `zero_counters` clears the
// arrival counters at the front of the workspace with a fill kernel first
// (kept to a kernel, not a memset, so the call can sit inside a captured
// graph).
__global__ void zero_words(int32_t* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

static int attend_decode(const void* q, void* out, void* k_pool, void* v_pool,
                         int64_t num_blocks, const int32_t* kv_indptr,
                         const int32_t* kv_indices, const int32_t* kv_lens, int32_t n_seqs,
                         int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                         int32_t page_size, float scale, int32_t dtype, const int32_t* plan,
                         int32_t n_work, int32_t n_slots, int32_t plan_stride,
                         const void* k_new, const void* v_new, const int32_t* slot_mapping,
                         void* workspace, int64_t workspace_bytes, bool zero_counters,
                         int32_t* status_word, void* stream) {
  int rc = check_geometry(n_heads, n_kv_heads, head_dim, page_size, dtype);
  if (rc) return rc;
  if (n_seqs <= 0) return PKV_OK;
  hipStream_t s = (hipStream_t)stream;
  const int32_t G = n_heads / n_kv_heads;
  LaunchFn fn = fast_decode(dtype, n_kv_heads, head_dim, G, page_size, 1);
  if (!fn) {
    if (k_new)
      return fail(PKV_ERR_INVALID, "a fused append needs the fast decode path "
                                   "(see pkv_decode_fast_path)");
    return generic_decode(q, out, k_pool, v_pool, num_blocks, kv_indptr, kv_indices, kv_lens,
                          n_seqs, n_heads, n_kv_heads, head_dim, page_size, scale, dtype,
                          status_word, s);
  }
  if (!plan || n_work <= 0 || n_slots < 0 || plan_stride < kHdrInts + kStageMax * kItemInts)
    return fail(PKV_ERR_INVALID, "decode needs a plan (pkv_plan_decode)");
  if (n_work % (n_kv_heads / heads_per_wg(n_kv_heads)))
    return fail(PKV_ERR_INVALID, "n_work=%d is not a whole number of bins", n_work);
  if ((k_new == nullptr) != (v_new == nullptr) || (k_new && !slot_mapping))
    return fail(PKV_ERR_INVALID, "a fused append needs k_new, v_new and slot_mapping");
  const uintptr_t al = (uintptr_t)q | (uintptr_t)out | (uintptr_t)k_pool | (uintptr_t)v_pool |
                       (uintptr_t)k_new | (uintptr_t)v_new;
  if (al % 16) return fail(PKV_ERR_INVALID, "q, out, pools and new rows must be 16-byte aligned");
  float* po = nullptr;
  float* pml = nullptr;
  int32_t* cnt = nullptr;
  uint32_t o_bytes = 0, ml_bytes = 0;
  if (n_slots > 0) {
    const int64_t need =
        pkv_decode_workspace_bytes(n_seqs, n_slots, n_heads, n_kv_heads, head_dim);
    if (!workspace || workspace_bytes < need || (uintptr_t)workspace % 256)
      return fail(PKV_ERR_CAPACITY, "split-K plan needs %lld 256-byte-aligned workspace "
                  "bytes, got %lld", (long long)need, (long long)workspace_bytes);
    // [arrival counters, n_seqs * n_kv_heads | partial outputs
    //  [n_slots][Hkv][part_floats] | (m, l) [n_slots][Hq][2]]
    const int64_t pf = (int64_t)n_slots * n_kv_heads * part_floats(G, head_dim);
    const int64_t mlf = (int64_t)n_slots * n_heads * 2;
    if ((pf + mlf) * 4 > 0x7fffffffLL)
      return fail(PKV_ERR_INVALID, "split-K partials exceed 2 GiB; use larger partitions");
    cnt = (int32_t*)workspace;
    po = (float*)((char*)workspace + counter_bytes(n_seqs, n_kv_heads));
    pml = po + pf;
    o_bytes = (uint32_t)(pf * 4);
    ml_bytes = (uint32_t)(mlf * 4);
    if (zero_counters) {
      const int64_t words = counter_bytes(n_seqs, n_kv_heads) / 4;
      hipLaunchKernelGGL(zero_words, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, s,
                         cnt, words);
      PKV_LAUNCH_CHECK();
    }
  }
  fn(q, out, k_pool, v_pool, num_blocks, plan, n_work, plan_stride, n_kv_heads, scale * kLog2e,
     k_new, v_new, slot_mapping, po, pml, o_bytes, ml_bytes, cnt, status_word, s);
  PKV_LAUNCH_CHECK();
  return PKV_OK;
}

// Workspace of the no-allocation entry point: one file-scope device array,
// which every GPU the library runs on holds (at its own address) until the
// process ends. In host code `scratch` names a host-side stand-in, never the
// device memory: the device address is looked up once per device with
// hipGetSymbolAddress and only that address is passed to kernels.
static __device__ __align__(256) unsigned char scratch[PKV_DECODE_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

// This device's address of `scratch`, looked up on the first call on the
// device (with it current); nullptr with the error set on failure.
static void* scratch_on_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fail(PKV_ERR_HIP, "no current HIP device (or device index above %d)", kMaxDevices - 1);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      fail(PKV_ERR_HIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
           hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

}  // namespace pkv

extern "C" int pkv_attend_decode(const void* q, void* out, void* k_pool, void* v_pool,
                                 int64_t num_blocks, const int32_t* kv_indptr,
                                 const int32_t* kv_indices, const int32_t* kv_lens,
                                 int32_t n_seqs, int32_t n_heads, int32_t n_kv_heads,
                                 int32_t head_dim, int32_t page_size, float scale,
                                 int32_t dtype, const int32_t* plan, int32_t n_work,
                                 int32_t n_slots, int32_t plan_stride, const void* k_new,
                                 const void* v_new, const int32_t* slot_mapping,
                                 void* workspace, int64_t workspace_bytes,
                                 int32_t* status_word, void* stream) {
  return attend_decode(q, out, k_pool, v_pool, num_blocks, kv_indptr, kv_indices, kv_lens,
                       n_seqs, n_heads, n_kv_heads, head_dim, page_size, scale, dtype, plan,
                       n_work, n_slots, plan_stride, k_new, v_new, slot_mapping, workspace,
                       workspace_bytes, false, status_word, stream);
}

extern "C" int pkv_attend_decode_noalloc(const void* q, void* out, void* k_pool, void* v_pool,
                                         int64_t num_blocks, const int32_t* kv_indptr,
                                         const int32_t* kv_indices, const int32_t* kv_lens,
                                         int32_t n_seqs, int32_t n_heads, int32_t n_kv_heads,
                                         int32_t head_dim, int32_t page_size, float scale,
                                         int32_t dtype, const int32_t* plan, int32_t n_work,
                                         int32_t n_slots, int32_t plan_stride,
                                         const void* k_new, const void* v_new,
                                         const int32_t* slot_mapping, int32_t* status_word,
                                         void* stream) {
  void* ws = nullptr;
  if (n_slots > 0) {
    const int64_t need =
        pkv_decode_workspace_bytes(n_seqs, n_slots, n_heads, n_kv_heads, head_dim);
    if (need <= 0)
      return fail(PKV_ERR_INVALID, "invalid geometry for a split-K plan");
    if (need > (int64_t)PKV_DECODE_SCRATCH_BYTES)
      return fail(PKV_ERR_CAPACITY, "split-K plan needs %lld workspace bytes; the "
                  "no-allocation entry point holds at most %lld (use pkv_attend_decode with a "
                  "workspace, or larger partitions)", (long long)need,
                  (long long)PKV_DECODE_SCRATCH_BYTES);
    ws = scratch_on_current_device();
    if (!ws) return PKV_ERR_HIP;
  }
  return attend_decode(q, out, k_pool, v_pool, num_blocks, kv_indptr, kv_indices, kv_lens,
                       n_seqs, n_heads, n_kv_heads, head_dim, page_size, scale, dtype, plan,
                       n_work, n_slots, plan_stride, k_new, v_new, slot_mapping, ws,
                       (int64_t)PKV_DECODE_SCRATCH_BYTES, true, status_word, stream);
}

#ifdef PKV_TIMELINE
// Copies the instrumented build's per-wave decode timeline (the last launch
// that wrote each record) to host memory: at most `bytes` bytes.
extern "C" int pkv_timeline_read(void* host, int64_t bytes) {
  if (bytes > (int64_t)sizeof(pkv::pkv_timeline)) bytes = sizeof(pkv::pkv_timeline);
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(pkv::pkv_timeline), (size_t)bytes, 0,
                             hipMemcpyDeviceToHost) == hipSuccess ? 0 : -1;
}
#endif
