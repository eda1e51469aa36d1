// Paged decode attention for gfx950 (every sequence has one query token).
//
// Work decomposition (planned on the host once per batch): a sequence's
// pages are cut into partitions of at most part_pages pages (split-K over
// the KV axis; the split depends only on that sequence's own length, so its
// result never depends on what it is batched with). One workgroup owns one
// partition for a group of up to 4 KV heads: one wave per KV head (two heads
// per wave beyond 8 KV heads in a group).
//
// Memory: a page is 16 token rows x (all KV heads x head_dim) contiguous in
// the pool; a head group's slice of a row is 512 contiguous bytes at the
// headline geometry. The workgroup reads its slice of every row whole --
// lane chunk k is bytes [16 c, +16) of the slice sequence, c = tid + k *
// threads -- so each wave instruction covers whole 128-byte lines. The pages
// arrive in registers two pages ahead of use, are copied to one of two
// padded LDS page buffers, and one barrier per page separates filling a
// buffer from reading it. Small workgroups (4 waves) keep four resident per
// compute unit, so one workgroup's start and end latencies overlap others'
// streaming.
//
// Per wave, head and page (G query heads share the KV head, G <= 16):
//  1. S^T = K Q^T with one 16x16x32 MFMA per 32 dims: the K rows (from LDS)
//     are the A operand, Q^T the B operand (column n = query head n, zero
//     beyond G). Lane (head n, group g) then holds the scores of tokens
//     4g..4g+3 of the page for head n;
//  2. online softmax in registers: mask past kv_len, running max / sum with
//     two cross-lane steps; p = 2^(s*scale*log2e - m) rounded to the pool
//     dtype -- four values per lane that are exactly the A operand of a
//     16x16x16 MFMA. The reference max m moves lazily (only when a head's
//     max grows by more than 2^8), so most pages skip the rescale of o;
//  3. PV on MFMA: ds_read_b64_tr_b16 hands each lane 4 consecutive tokens of
//     one V dim, the B operand, one read per 16 dims. V rows past kv_len are
//     zeroed in LDS so stale bits can never reach the sum.
//
// Split sequences merge in the same launch. Each partition publishes its
// partial (o, m, l) with 16-byte buffer stores carrying the sc1 (agent
// coherence) bit, which write through the per-XCD L2, waits until they have
// completed (s_waitcnt vmcnt(0)), then bumps its sequence's arrival counter.
// The workgroup that sees the last arrival reads the partials back with sc1
// loads (never a stale L2 line) and writes the output. This avoids a second
// launch and an agent-scope release fence, whose L2 write-back walks the
// whole cache.
//
// Packs: when no sequence of the batch is split, a partition holds up to 16
// whole consecutive sequences (segments) whose pages follow each other in
// kv_indices. The page pipeline runs straight through the pack; at each
// segment's last page the wave writes that sequence's output, resets its
// softmax state and switches to the next sequence's Q, loaded one segment
// ahead. Per page and sequence the arithmetic is the same as in a partition
// of its own, so results do not depend on the packing.
//
// Loads cover only a page's rows below kv_len: the tail of a sequence's last
// page is outside the buffer range and reads as zeros without a memory access.
//
// Fused append (optional): when the caller passes the step's new K/V rows,
// the workgroup that owns a sequence's last page writes the new row to
// slot_mapping's slot and patches the copy it loaded, so a decode step costs
// one launch per layer instead of two. The patch is applied only when
// slot_mapping names the same slot as the page table, so the result is
// exactly "append, then attend" (the caller guarantees that no other
// sequence of the launch reads that slot).
#include <algorithm>
#include <mutex>
#include <vector>

#include "mfma.h"

namespace pkv {

// {seq, index of the partition's first page in kv_indices, n_pages, partial
//  slot (-1: the partition is the whole sequence), kv_len, first token,
//  n_partitions of the sequence, first slot of the sequence}
constexpr int kWorkInts = 8;
constexpr int kMaxWaves = 8;      // waves per workgroup (one per KV head), at most
constexpr int kGroupHeads = 4;    // KV heads per workgroup (its slice of each page row)
constexpr int kMaxPartPages = 64; // a partition's page ids fit one wave-wide load
constexpr int kMaxPackSeqs = 16;  // sequences per pack (one lane each; patch bits)

// Layout of one partition's partial output: per (slot, KV head), NGR groups
// of 4 head rows, each NDB dim blocks of 16 lanes x 4 rows (float4 per
// lane) -- exactly the MFMA accumulator layout, so a wave stores and loads
// it with one 16-byte access per lane and dim block.
template <int D, int G> struct PartLayout {
  static constexpr int NGR = (G + 3) / 4;
  static constexpr int NDB = D / 16;
  static constexpr int FLOATS = NGR * NDB * 64;  // per (slot, KV head)
};

// Split-K merge for one KV head h of sequence seq, run by the workgroup that
// published the last partial. Lanes run over partitions for each head row's
// max M and sum L; then, 64 partitions at a time, the weights 2^(m_s - M)
// go to this wave's LDS scratch as [partition][GS rows], and the partial
// outputs are read in the producers' own layout: lane (n, g) takes row group
// rg = g % NGR of every SPLIT-th partition starting at g / NGR, MB
// partitions per round trip, and the SPLIT lane groups that share a row
// group are summed by shuffles at the end. The summation order depends only
// on the partition count, so the result does not depend on the batch.
template <typename T, int D, int G>
__device__ __forceinline__ void merge_head(T* __restrict__ out, float* wts, int seq, int h,
                                           int n_kv_heads, int nparts, int slot0,
                                           __amdgpu_buffer_rsrc_t ro, __amdgpu_buffer_rsrc_t rm) {
  typedef PartLayout<D, G> PL;
  constexpr int NDB = D / 16;
  constexpr int NGR = PL::NGR;
  constexpr int SPLIT = 4 / NGR;
  constexpr int GS = 4 * NGR;              // weight rows per partition (>= G)
  constexpr int MB = 1;                    // partitions per lane per round trip
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
  const int rg = g % NGR, so = g / NGR;
  const int Hq = n_kv_heads * G;
  auto load_ml = [&](int c0, float* mr, float* lr) {
    const bool ok = c0 + lane < nparts;
    const uint32_t b2 = (uint32_t)(((int64_t)(slot0 + (ok ? c0 + lane : 0)) * Hq + h * G) * 8);
#pragma unroll
    for (int r = 0; r < G; ++r) {
      const f32x2 ml =
          __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(rm, b2 + 8 * r, 0, kSc1));
      mr[r] = ok ? ml[0] : -INFINITY;
      lr[r] = ok ? ml[1] : 0.f;
    }
  };
  // The partial outputs of one batch: MB partitions of this lane's stride.
  auto load_batch = [&](int c0, int s0, f32x4 (*v)[NDB]) {
    const int cn = min(64, nparts - c0);
#pragma unroll
    for (int u = 0; u < MB; ++u) {
      const int sl = s0 + u * SPLIT;
      const uint32_t off =
          (uint32_t)(((int64_t)(slot0 + c0 + (sl < cn ? sl : 0)) * n_kv_heads + h) *
                     PL::FLOATS * 4);
#pragma unroll
      for (int b = 0; b < NDB; ++b)
        v[u][b] = sl < cn ? __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                ro, off + ((rg * NDB + b) * 16 + n) * 16, 0, kSc1))
                          : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  // The first batch does not depend on the maximum: its loads go out with
  // the (m, l) loads, so a sequence of up to SPLIT * MB partitions merges in
  // one round trip.
  f32x4 v[MB][NDB];
  load_batch(0, so, v);
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
    for (int s0 = so; s0 < cn; s0 += SPLIT * MB) {
      if (c0 > 0 || s0 > so) load_batch(c0, s0, v);
#pragma unroll
      for (int u = 0; u < MB; ++u) {
        const int sl = s0 + u * SPLIT;
        if (sl < cn) {
          const f32x4 wr = *reinterpret_cast<const f32x4*>(wts + sl * GS + 4 * rg);
#pragma unroll
          for (int b = 0; b < NDB; ++b) acc[b] += wr * v[u][b];
        }
      }
    }
    wave_lds_sync();  // the next chunk rewrites the weights
  }
#pragma unroll
  for (int b = 0; b < NDB; ++b) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (SPLIT >= 4) acc[b][i] += __shfl_xor(acc[b][i], 16, 64);
      if (SPLIT >= 2) acc[b][i] += __shfl_xor(acc[b][i], 32, 64);
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
#pragma unroll
        for (int b = 0; b < NDB; ++b)
          out[((int64_t)seq * Hq + h * G + r) * D + 16 * b + n] = (T)(acc[b][i] / lr_);
      }
    }
  }
}

// One workgroup per partition, covering every KV head: NW = n_kv_heads / HPW
// waves, wave w owning heads w, w + NW, ... Each page (16 token rows of all
// heads, contiguous in the pool) is loaded as whole rows -- lane chunk k is
// bytes [16 (tid + k NW 64), +16) of the page, so every wave instruction
// reads whole 128-byte lines of consecutive memory -- into registers two
// pages ahead, copied into a padded LDS tile, and each wave reads its heads'
// columns from there: K rows as the A operand of the QK MFMA (ds_read_b128),
// V through ds_read_b64_tr_b16 as the B operand of the PV MFMA.
template <typename T, int D, int G, int HPW, bool PACK>
__global__ __launch_bounds__(kMaxWaves * 64) void decode_kernel(
    const T* __restrict__ q, T* __restrict__ out, T* __restrict__ kpool, T* __restrict__ vpool,
    int64_t num_blocks, const int32_t* __restrict__ kv_indices,
    const int32_t* __restrict__ kv_indptr, const int32_t* __restrict__ kv_lens,
    const int32_t* __restrict__ work, int32_t n_kv_heads, float scale_log2,
    const T* __restrict__ k_new, const T* __restrict__ v_new,
    const int32_t* __restrict__ slot_mapping, float* part_o, float* part_ml,
    uint32_t o_bytes, uint32_t ml_bytes, int32_t* counters, int32_t* status) {
  typedef typename Mma<T>::vec8 vec8;
  typedef typename Mma<T>::vec4 vec4;
  typedef PartLayout<D, G> PL;
  constexpr int PS = 16;
  constexpr int NCH = D / 32;         // QK MFMA k-chunks per head row
  constexpr int NDB = D / 16;         // PV MFMA dim blocks
  constexpr int CPL = HPW * D / 32;   // 16-byte chunks per lane per page and tensor
  constexpr int NGR = PL::NGR;

  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int NW = blockDim.x >> 6;
  const int HGW = NW * HPW;                          // KV heads of this workgroup
  const int n_groups = n_kv_heads / HGW;
  const int wi = blockIdx.x / n_groups;              // partition
  const int hg = blockIdx.x - wi * n_groups;         // head group: heads hg*HGW ..
  const int frow = n_kv_heads * D * (int)sizeof(T);  // bytes per token row, all heads
  const int rowb = HGW * D * (int)sizeof(T);         // bytes of the group's slice of a row
  const int RS = rowb + 16;                          // padded LDS row stride
  // Two page buffers, each [16][RS] K rows then [16][RS] V rows.
  constexpr int kBufs = 2;
  // past both the page tiles and the merge scratch (see decode_lds_bytes)
  int* s_flag = reinterpret_cast<int*>(smem + max(kBufs * 2 * PS * RS, NW * 64 * 4 * NGR * 4));

  const int32_t* w = work + kWorkInts * wi;
  const int seq0 = w[0], pbase = w[1], npp = w[2], slot = w[3];
  const int tok0 = w[5], nparts = w[6], slot0 = w[7];
  // A pack holds w[4] whole consecutive sequences from seq0 (segments), whose
  // pages follow each other in kv_indices from pbase: lane s < nseq holds
  // segment s's first page within the pack and its kv_len. Otherwise the
  // partition is one segment and w[4] its sequence's kv_len.
  int nseq = 1, lane_first = 0, lane_kv = w[4], lane_slot = 0;
  if constexpr (PACK) {
    nseq = min(max(w[4], 1), kMaxPackSeqs);  // the planner's bound; shifts stay in range
    if (lane < nseq) {
      lane_first = kv_indptr[seq0 + lane] - pbase;
      lane_kv = kv_lens[seq0 + lane];
      if (k_new != nullptr) lane_slot = slot_mapping[seq0 + lane];
    }
  }
  auto seg_of = [&](int j) -> int {  // segment of page j (wave-uniform)
    if constexpr (!PACK) return 0;
    return __builtin_popcountll(__builtin_amdgcn_ballot_w64(lane < nseq && lane_first <= j)) - 1;
  };
  auto seg_first = [&](int s) { return PACK ? __builtin_amdgcn_readlane(lane_first, s) : 0; };
  auto seg_end = [&](int s) {        // one past the segment's last page
    return PACK && s + 1 < nseq ? __builtin_amdgcn_readlane(lane_first, s + 1) : npp;
  };
  auto seg_kv = [&](int s) { return __builtin_amdgcn_readlane(lane_kv, s); };
  // first token of page j within its sequence
  auto page_tok = [&](int j, int s) { return PACK ? (j - seg_first(s)) * 16 : tok0 + j * 16; };
  int seq = seq0;                    // sequence of the segment being computed
  const int kv_len = seg_kv(0);
  const int Hq = n_kv_heads * G;
  const int64_t row = (int64_t)n_kv_heads * D;
  const int n = lane & 15;   // MFMA row/column within a 16-lane block
  const int g = lane >> 4;   // MFMA k-group

  // Lane j holds the partition's j-th page id (npp <= 64).
  int pid = 0;
  if (lane < npp) pid = kv_indices[pbase + lane];
  const bool bad = lane < npp && (pid < 0 || (int64_t)pid >= num_blocks);
  if (bad) pid = 0;
  if (__builtin_amdgcn_ballot_w64(bad) && tid == 0) flag(status, PKV_STATUS_BAD_PAGE);

  // This lane's chunks of a page: byte offset in the page, token row, LDS offset.
  const int cpr = rowb / 16;
  uint32_t goff[CPL], loff[CPL];
  int lrow[CPL];
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int c = tid + k * NW * 64;
    lrow[k] = c / cpr;
    goff[k] = (uint32_t)(lrow[k] * frow + hg * rowb + (c - lrow[k] * cpr) * 16);
    loff[k] = (uint32_t)(lrow[k] * RS + (c - lrow[k] * cpr) * 16);
  }
  // Only the page's rows below kv_len are in the buffer range: the rows past
  // it (the tail of a sequence's last page) read as zeros without a memory
  // access.
  auto load_page = [&](int j, vec8* kr, vec8* vr) {
    const int64_t page = __builtin_amdgcn_readlane(pid, j);
    const int sj = seg_of(j);
    const int live = min(PS, seg_kv(sj) - page_tok(j, sj));
    const uint32_t bytes = (uint32_t)live * (uint32_t)frow;
    const __amdgpu_buffer_rsrc_t rk = ws_rsrc(kpool + page * PS * row, bytes);
    const __amdgpu_buffer_rsrc_t rv = ws_rsrc(vpool + page * PS * row, bytes);
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      kr[k] = __builtin_bit_cast(vec8, __builtin_amdgcn_raw_buffer_load_b128(rk, goff[k], 0, kNt));
      vr[k] = __builtin_bit_cast(vec8, __builtin_amdgcn_raw_buffer_load_b128(rv, goff[k], 0, kNt));
    }
  };
  vec8 kA[CPL], vA[CPL], kB[CPL], vB[CPL];
  load_page(0, kA, vA);
  if (npp > 1) load_page(1, kB, vB);

  // Q^T as the QK B operand per owned head: column n = query head h*G + n.
  vec8 qb[HPW][NCH];
  auto load_q = [&](auto& dst, int sq) {
#pragma unroll
    for (int hh = 0; hh < HPW; ++hh) {
      const int h = hg * HGW + wave + hh * NW;
      const T* qr = q + ((int64_t)sq * Hq + h * G + (n < G ? n : 0)) * D + g * 8;
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        vec8 t = *reinterpret_cast<const vec8*>(qr + c * 32);
        dst[hh][c] = (n < G) ? t : vec8{};
      }
    }
  };
  load_q(qb, seq0);
  // a pack's next segment's Q is loaded one segment ahead
  vec8 qn[PACK ? HPW : 1][PACK ? NCH : 1];
  if constexpr (PACK) {
    if (nseq > 1) load_q(qn, seq0 + 1);
  }

  // Fused append: the workgroup whose partition holds the newest token writes
  // that row (all heads) to slot_mapping's slot now; the loaded copy of the
  // row is patched before it reaches LDS.
  // A pack owns the newest token of every segment. Bit s of `patch` says
  // whether segment s's loaded copy of its newest row is patched.
  auto append_row = [&](int sq, int kv, int last_j) -> bool {
    const int tl = (kv - 1) % PS;   // newest token's row within its page
    const int64_t csr_slot = (int64_t)__builtin_amdgcn_readlane(pid, last_j) * PS + tl;
    const int64_t new_slot = slot_mapping[sq];
    const bool in_range = new_slot >= 0 && new_slot < num_blocks * PS;
    if (!in_range && tid == 0) flag(status, PKV_STATUS_BAD_SLOT);
    if (in_range) {
      const unsigned char* kn = reinterpret_cast<const unsigned char*>(k_new + sq * row);
      const unsigned char* vn = reinterpret_cast<const unsigned char*>(v_new + sq * row);
      unsigned char* kd = reinterpret_cast<unsigned char*>(kpool + new_slot * row);
      unsigned char* vd = reinterpret_cast<unsigned char*>(vpool + new_slot * row);
#pragma unroll
      for (int k = 0; k < CPL; ++k) {
        if (lrow[k] == tl) {
          const uint32_t col = goff[k] - (uint32_t)tl * frow;
          *reinterpret_cast<vec8*>(kd + col) = *reinterpret_cast<const vec8*>(kn + col);
          *reinterpret_cast<vec8*>(vd + col) = *reinterpret_cast<const vec8*>(vn + col);
        }
      }
    }
    return new_slot == csr_slot;
  };
  uint32_t patch = 0, in_range_bits = 0;
  if (k_new != nullptr) {
    if constexpr (PACK) {
      // every segment ends in the pack: its new row is written, and patched
      // into the loaded copy, when its last page is staged
      for (int s = 0; s < nseq; ++s) {
        const int tl = (seg_kv(s) - 1) % PS;
        const int64_t csr_slot =
            (int64_t)__builtin_amdgcn_readlane(pid, seg_end(s) - 1) * PS + tl;
        const int64_t new_slot = __builtin_amdgcn_readlane(lane_slot, s);
        const bool in_range = new_slot >= 0 && new_slot < num_blocks * PS;
        if (!in_range && tid == 0) flag(status, PKV_STATUS_BAD_SLOT);
        patch |= (uint32_t)(new_slot == csr_slot) << s;
        in_range_bits |= (uint32_t)in_range << s;
      }
    } else if (tok0 + npp * PS >= kv_len) {
      patch = append_row(seq0, kv_len, npp - 1);
    }
  }

  f32x4 o[HPW][NDB];
  float m_run[HPW], l_run[HPW];  // per head column n (replicated over g)
#pragma unroll
  for (int hh = 0; hh < HPW; ++hh) {
    m_run[hh] = -INFINITY;
    l_run[hh] = 0.f;
#pragma unroll
    for (int b = 0; b < NDB; ++b) o[hh][b] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // Page j lives in LDS buffer j % 2. Step j writes page j+1 (already in
  // registers) into the other buffer, refills those registers with page j+3,
  // runs every wave's heads over page j, and ends with the one barrier of the
  // step: page j+1 is then complete and page j's buffer free for page j+2.
  auto stage = [&](int j, vec8* kr, vec8* vr) {
    unsigned char* kl = smem + (j & 1) * 2 * PS * RS;
    unsigned char* vl = kl + PS * RS;
    const int s = seg_of(j);
    const int kv = seg_kv(s);
    if (PACK && ((in_range_bits >> s) & 1) && j == seg_end(s) - 1) {
      const int sq = seq0 + s, tl = (kv - 1) % PS;
      const int64_t new_slot = __builtin_amdgcn_readlane(lane_slot, s);
      const bool pt = (patch >> s) & 1;
      const unsigned char* kn = reinterpret_cast<const unsigned char*>(k_new + sq * row);
      const unsigned char* vn = reinterpret_cast<const unsigned char*>(v_new + sq * row);
      unsigned char* kd = reinterpret_cast<unsigned char*>(kpool + new_slot * row);
      unsigned char* vd = reinterpret_cast<unsigned char*>(vpool + new_slot * row);
#pragma unroll
      for (int k = 0; k < CPL; ++k) {
        if (lrow[k] == tl) {
          const uint32_t col = goff[k] - (uint32_t)tl * frow;
          const vec8 kx = *reinterpret_cast<const vec8*>(kn + col);
          const vec8 vx = *reinterpret_cast<const vec8*>(vn + col);
          *reinterpret_cast<vec8*>(kd + col) = kx;
          *reinterpret_cast<vec8*>(vd + col) = vx;
          if (pt) {
            kr[k] = kx;
            vr[k] = vx;
          }
        }
      }
    } else if (!PACK && ((patch >> s) & 1) && j == seg_end(s) - 1) {
      const int sq = seq0 + s, tl = (kv - 1) % PS;
      const unsigned char* kn = reinterpret_cast<const unsigned char*>(k_new + sq * row);
      const unsigned char* vn = reinterpret_cast<const unsigned char*>(v_new + sq * row);
#pragma unroll
      for (int k = 0; k < CPL; ++k) {
        if (lrow[k] == tl) {
          const uint32_t col = goff[k] - (uint32_t)tl * frow;
          kr[k] = *reinterpret_cast<const vec8*>(kn + col);
          vr[k] = *reinterpret_cast<const vec8*>(vn + col);
        }
      }
    }
    const int tp = page_tok(j, s);  // first token of the page
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      *reinterpret_cast<vec8*>(kl + loff[k]) = kr[k];
      // rows past kv_len are zeroed so stale bits never reach the PV sum
      *reinterpret_cast<vec8*>(vl + loff[k]) = tp + lrow[k] < kv ? vr[k] : vec8{};
    }
  };
  // lane (dim column n, group g) holds heads 4g..4g+3 of dims 16b + n.
  auto write_out = [&]() {
#pragma unroll
    for (int hh = 0; hh < HPW; ++hh) {
      const int h = hg * HGW + wave + hh * NW;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * g + i;
        const float li = __shfl(l_run[hh], r, 64);  // lane r holds head r's sum
        if (r < G) {
#pragma unroll
          for (int b = 0; b < NDB; ++b)
            out[((int64_t)seq * Hq + h * G + r) * D + 16 * b + n] = (T)(o[hh][b][i] / li);
        }
      }
    }
  };
  auto compute = [&](int j) {
    const unsigned char* kl = smem + (j & 1) * 2 * PS * RS;
    const unsigned char* vl = kl + PS * RS;
    const int sg = seg_of(j);
    const int kv = seg_kv(sg);
    const int tp = page_tok(j, sg);
#pragma unroll
    for (int hh = 0; hh < HPW; ++hh) {
      const int h = wave + hh * NW;  // the head's column in the group's LDS rows
      // S^T: lane (n, g) gets the scores of tokens 4g..4g+3 for head n.
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      const unsigned char* kp = kl + n * RS + (h * D + g * 8) * (int)sizeof(T);
#pragma unroll
      for (int c = 0; c < NCH; ++c)
        acc = Mma<T>::qk(*reinterpret_cast<const vec8*>(kp + c * 32 * sizeof(T)), qb[hh][c], acc);
      float sc[4];
      float mx = -INFINITY;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sc[i] = tp + 4 * g + i < kv ? acc[i] * scale_log2 : -INFINITY;
        mx = fmaxf(mx, sc[i]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      // Lazy rescale: the reference max moves only when some head's max
      // grows by more than 2^8, so p <= 256 and o / l is unchanged.
      if (__builtin_amdgcn_ballot_w64(mx > m_run[hh] + 8.f)) {
        const float m_new = fmaxf(m_run[hh], mx);  // finite: every page has a live token
        const float alpha = __builtin_amdgcn_exp2f(m_run[hh] - m_new);
        l_run[hh] *= alpha;
        m_run[hh] = m_new;
        // lane (n, g) holds output rows 4g+i, whose factor lives in lane 4g+i
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float a = __shfl(alpha, 4 * g + i, 64);
#pragma unroll
          for (int b = 0; b < NDB; ++b) o[hh][b][i] *= a;
        }
      }
      vec4 p;
      float ls = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = __builtin_amdgcn_exp2f(sc[i] - m_run[hh]);
        ls += e;
        p[i] = (T)e;
      }
      ls += __shfl_xor(ls, 16, 64);
      ls += __shfl_xor(ls, 32, 64);
      l_run[hh] += ls;
      const unsigned char* vp =
          vl + (4 * g + (n >> 2)) * RS + (h * D + 4 * (n & 3)) * (int)sizeof(T);
#pragma unroll
      for (int b = 0; b < NDB; ++b) {
        const i16x4 raw = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_i16x4*)(vp + 16 * b * sizeof(T)));
        o[hh][b] = Mma<T>::pv(p, __builtin_bit_cast(vec4, raw), o[hh][b]);
      }
    }
    if constexpr (PACK) {
      // the segment's last page: write its output and start the next
      // sequence (the last segment leaves through the common exit)
      if (sg + 1 < nseq && j == seg_end(sg) - 1) {
        write_out();
#pragma unroll
        for (int hh = 0; hh < HPW; ++hh) {
          m_run[hh] = -INFINITY;
          l_run[hh] = 0.f;
#pragma unroll
          for (int b = 0; b < NDB; ++b) o[hh][b] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        seq = seq0 + sg + 1;
#pragma unroll
        for (int hh = 0; hh < HPW; ++hh) {
#pragma unroll
          for (int c = 0; c < NCH; ++c) qb[hh][c] = qn[hh][c];
        }
        if (sg + 2 < nseq) load_q(qn, seq + 1);
      }
    }
  };
  // Registers: set A holds the even pages, set B the odd ones.
  stage(0, kA, vA);
  if (npp > 2) load_page(2, kA, vA);
  __syncthreads();
  for (int j = 0; j < npp; j += 2) {  // two register sets, so unrolled by two
    if (j + 1 < npp) stage(j + 1, kB, vB);
    if (j + 3 < npp) load_page(j + 3, kB, vB);
    compute(j);
    __syncthreads();
    if (j + 1 < npp) {
      if (j + 2 < npp) stage(j + 2, kA, vA);
      if (j + 4 < npp) load_page(j + 4, kA, vA);
      compute(j + 1);
      __syncthreads();
    }
  }

  if (PACK || slot < 0) {
    write_out();
    return;
  }

  // ---- split sequence: publish, count, and the last arrival merges --------
  const __amdgpu_buffer_rsrc_t ro = ws_rsrc(part_o, o_bytes);
  const __amdgpu_buffer_rsrc_t rm = ws_rsrc(part_ml, ml_bytes);
#pragma unroll
  for (int hh = 0; hh < HPW; ++hh) {
    const int h = hg * HGW + wave + hh * NW;
    const uint32_t head_off = (uint32_t)(((int64_t)slot * n_kv_heads + h) * PL::FLOATS * 4);
    if (g < NGR) {
#pragma unroll
      for (int b = 0; b < NDB; ++b)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o[hh][b]), ro,
                                               head_off + ((g * NDB + b) * 16 + n) * 16, 0, kSc1);
    }
    if (lane < G)
      __builtin_amdgcn_raw_buffer_store_b64(
          __builtin_bit_cast(u32x2, f32x2{m_run[hh], l_run[hh]}), rm,
          (uint32_t)(((int64_t)slot * Hq + h * G + lane) * 8), 0, kSc1);
  }
  // Every partial store of every wave has completed at the coherence point
  // before the workgroup counts its arrival.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  int32_t* cnt = counters + (int64_t)seq * n_groups + hg;
  if (tid == 0)
    *s_flag = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (*s_flag != nparts - 1) return;

  // Last arrival for seq: each wave merges its heads, using its share of
  // the (now free) page tile as scratch for the weights.
  float* wts = reinterpret_cast<float*>(smem) + wave * 64 * (4 * NGR);
#pragma unroll
  for (int hh = 0; hh < HPW; ++hh)
    merge_head<T, D, G>(out, wts, seq, hg * HGW + wave + hh * NW, n_kv_heads, nparts, slot0,
                        ro, rm);
  if (tid == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Dynamic LDS of a decode workgroup: two padded K+V page buffers plus the
// arrival flag. The merge reuses the tiles as 64 x 4*ceil(G/4) floats per wave.
static size_t decode_lds_bytes(int32_t Hkv, int32_t D, int32_t G) {
  const size_t tiles = 2 * 2 * 16 * (size_t)(Hkv * D * 2 + 16);  // two K+V page buffers
  const size_t merge = (size_t)std::min(Hkv, kMaxWaves) * 64 * 4 * ((G + 3) / 4) * 4;
  return std::max(tiles, merge) + 16;  // + the arrival flag
}

template <typename T, int D, int G, int HPW>
static void launch(const void* q, void* out, void* kp, void* vp, int64_t nb,
                   const int32_t* indices, const int32_t* indptr, const int32_t* kv_lens,
                   bool pack, const int32_t* work, int32_t n_work, int32_t Hkv,
                   float sl2, const void* kn, const void* vn, const int32_t* slots, float* po,
                   float* pml, uint32_t o_bytes, uint32_t ml_bytes, int32_t* cnt,
                   int32_t* status, hipStream_t s) {
  const int hgw = std::min<int>(Hkv, kGroupHeads);  // KV heads per workgroup
  const int nw = hgw / HPW;
  const dim3 grid((unsigned)(n_work * (Hkv / hgw))), block(nw * 64);
  const size_t lds = decode_lds_bytes(hgw, D, G);
  if (pack)
    hipLaunchKernelGGL((decode_kernel<T, D, G, HPW, true>), grid, block, lds, s, (const T*)q,
                       (T*)out, (T*)kp, (T*)vp, nb, indices, indptr, kv_lens, work, Hkv, sl2,
                       (const T*)kn, (const T*)vn, slots, po, pml, o_bytes, ml_bytes, cnt, status);
  else
    hipLaunchKernelGGL((decode_kernel<T, D, G, HPW, false>), grid, block, lds, s, (const T*)q,
                       (T*)out, (T*)kp, (T*)vp, nb, indices, indptr, kv_lens, work, Hkv, sl2,
                       (const T*)kn, (const T*)vn, slots, po, pml, o_bytes, ml_bytes, cnt, status);
}

typedef void (*LaunchFn)(const void*, void*, void*, void*, int64_t, const int32_t*,
                         const int32_t*, const int32_t*, bool, const int32_t*, int32_t, int32_t,
                         float, const void*, const void*, const int32_t*, float*, float*,
                         uint32_t, uint32_t, int32_t*, int32_t*, hipStream_t);

template <typename T, int D, int HPW>
static LaunchFn pick_g(int G) {
  switch (G) {
    case 1: return launch<T, D, 1, HPW>;
    case 2: return launch<T, D, 2, HPW>;
    case 4: return launch<T, D, 4, HPW>;
    case 8: return launch<T, D, 8, HPW>;
    case 16: return launch<T, D, 16, HPW>;
    default: return nullptr;
  }
}

// Heads per wave: the workgroup has one wave per KV head of its group, up to
// kMaxWaves.
static int heads_per_wave(int Hkv) {
  const int hgw = std::min(Hkv, kGroupHeads);
  return hgw <= kMaxWaves ? 1 : hgw / kMaxWaves;
}

template <typename T>
static LaunchFn pick(int Hkv, int D, int G) {
  // Whole-row staging needs rows of at most 2 KiB and Hkv a power of two up
  // to 2 * kMaxWaves (so that waves x heads per wave covers every head).
  const int hgw = std::min(Hkv, kGroupHeads);
  if (Hkv < 1 || (Hkv & (Hkv - 1)) || hgw > 2 * kMaxWaves || hgw * D * 2 > 2048) return nullptr;
  const int hpw = heads_per_wave(Hkv);
  switch (D) {
    case 64: return hpw == 1 ? pick_g<T, 64, 1>(G) : pick_g<T, 64, 2>(G);
    case 128: return hpw == 1 ? pick_g<T, 128, 1>(G) : nullptr;
    default: return nullptr;
  }
}

static LaunchFn fast_decode(int32_t dtype, int32_t Hkv, int32_t D, int32_t G,
                            int32_t page_size, int32_t pp) {
  if (page_size != 16 || pp < 1 || pp > kMaxPartPages) return nullptr;
  if (dtype == PKV_DTYPE_F16) return pick<_Float16>(Hkv, D, G);
  if (dtype == PKV_DTYPE_BF16) return pick<__bf16>(Hkv, D, G);
  return nullptr;
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

extern "C" int pkv_plan_decode(const int32_t* kv_indptr, const int32_t* kv_lens,
                               const int32_t* kv_last_page_len, int32_t n_seqs,
                               int32_t page_size, int32_t part_pages, int32_t* plan,
                               int64_t plan_capacity, int32_t* n_work_out,
                               int32_t* n_slots_out) {
  if (n_seqs <= 0 || page_size <= 0 || part_pages <= 0 || part_pages > kMaxPartPages)
    return fail(PKV_ERR_INVALID, "n_seqs and page_size must be positive and part_pages in "
                "[1, %d]", kMaxPartPages);
  if (kv_indptr[0] != 0) return fail(PKV_ERR_INVALID, "kv_indptr must start at 0");
  struct Item { int32_t v[kWorkInts]; };
  std::vector<Item> items;
  items.reserve(n_seqs);
  int32_t slots = 0;
  for (int32_t i = 0; i < n_seqs; ++i) {
    const int32_t np = kv_indptr[i + 1] - kv_indptr[i];
    int rc = check_seq_pages(i, np, kv_lens[i], kv_last_page_len[i], page_size);
    if (rc) return rc;
    const int32_t parts = (np + part_pages - 1) / part_pages;
    const int32_t slot0 = parts > 1 ? slots : -1;
    for (int32_t p = 0; p < parts; ++p) {
      const int32_t first = p * part_pages;
      items.push_back({{i, kv_indptr[i] + first, std::min(part_pages, np - first),
                        parts > 1 ? slots + p : -1, kv_lens[i], first * page_size, parts,
                        slot0}});
    }
    if (parts > 1) slots += parts;
  }
  if (slots == 0) {
    // No sequence is split: runs of consecutive sequences (their pages are
    // consecutive in kv_indices) share a partition, up to part_pages pages
    // and kMaxPackSeqs sequences, so a workgroup's start-up latency is paid
    // once per pack instead of once per short sequence. Entry: {first seq,
    // its first page index, pages of the pack, -1, sequences in the pack, 0,
    // 1, -1}.
    items.clear();
    for (int32_t i = 0; i < n_seqs;) {
      int32_t j = i, pages = 0;
      while (j < n_seqs && j - i < kMaxPackSeqs) {
        const int32_t np = kv_indptr[j + 1] - kv_indptr[j];
        if (j > i && pages + np > part_pages) break;
        pages += np;
        ++j;
      }
      items.push_back({{i, kv_indptr[i], pages, -1, j - i, 0, 1, -1}});
      i = j;
    }
  }
  // Longest partitions first, so the short tail items fill in behind them;
  // among equals, longer sequences first so their merges start early.
  std::stable_sort(items.begin(), items.end(), [](const Item& a, const Item& b) {
    return a.v[2] != b.v[2] ? a.v[2] > b.v[2] : a.v[4] > b.v[4];
  });
  const int64_t need = (int64_t)kWorkInts * items.size();
  if (need > plan_capacity)
    return fail(PKV_ERR_CAPACITY, "plan needs %lld entries, capacity %lld", (long long)need,
                (long long)plan_capacity);
  int64_t o = 0;
  for (const Item& it : items)
    for (int k = 0; k < kWorkInts; ++k) plan[o++] = it.v[k];
  *n_work_out = (int32_t)items.size();
  *n_slots_out = slots;
  return PKV_OK;
}

extern "C" int64_t pkv_decode_workspace_bytes(int32_t n_seqs, int32_t n_slots,
                                              int32_t n_heads, int32_t n_kv_heads,
                                              int32_t head_dim) {
  if (n_seqs <= 0 || n_kv_heads <= 0 || n_slots <= 0) return 0;
  if (n_heads % n_kv_heads) return 0;
  const int64_t counters = ((int64_t)n_seqs * n_kv_heads * 4 + 255) / 256 * 256;
  const int64_t po = (int64_t)n_slots * n_kv_heads * part_floats(n_heads / n_kv_heads, head_dim);
  return counters + (po + (int64_t)n_slots * n_heads * 2) * 4;
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
                         int32_t n_work, int32_t n_slots, int32_t part_pages, const void* k_new,
                         const void* v_new, const int32_t* slot_mapping, void* workspace,
                         int64_t workspace_bytes, bool zero_counters, int32_t* status_word,
                         void* stream) {
  int rc = check_geometry(n_heads, n_kv_heads, head_dim, page_size, dtype);
  if (rc) return rc;
  if (n_seqs <= 0) return PKV_OK;
  hipStream_t s = (hipStream_t)stream;
  const int32_t G = n_heads / n_kv_heads;
  LaunchFn fn = fast_decode(dtype, n_kv_heads, head_dim, G, page_size, part_pages);
  if (!fn) {
    if (k_new)
      return fail(PKV_ERR_INVALID, "a fused append needs the fast decode path "
                                   "(see pkv_decode_fast_path)");
    return generic_decode(q, out, k_pool, v_pool, num_blocks, kv_indptr, kv_indices, kv_lens,
                          n_seqs, n_heads, n_kv_heads, head_dim, page_size, scale, dtype,
                          status_word, s);
  }
  if (!plan || n_work <= 0) return fail(PKV_ERR_INVALID, "decode needs a plan");
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
    // [arrival counters, n_seqs * n_kv_heads, zero before the first launch and
    //  left zero by every launch][n_slots][Hkv][part_floats] partial outputs,
    //  then [n_slots][Hq][2] (m, l)
    const int64_t pf = (int64_t)n_slots * n_kv_heads * part_floats(G, head_dim);
    const int64_t mlf = (int64_t)n_slots * n_heads * 2;
    if ((pf + mlf) * 4 > 0x7fffffffLL)
      return fail(PKV_ERR_INVALID, "split-K partials exceed 2 GiB; use larger partitions");
    cnt = (int32_t*)workspace;
    po = (float*)((char*)workspace + ((int64_t)n_seqs * n_kv_heads * 4 + 255) / 256 * 256);
    pml = po + pf;
    o_bytes = (uint32_t)(pf * 4);
    ml_bytes = (uint32_t)(mlf * 4);
    if (zero_counters) {
      const int64_t words = (int64_t)n_seqs * n_kv_heads;
      hipLaunchKernelGGL(zero_words, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, s,
                         cnt, words);
      PKV_LAUNCH_CHECK();
    }
  }
  // A plan without partial slots splits no sequence; its partitions are packs
  // of whole consecutive sequences (pkv_plan_decode).
  fn(q, out, k_pool, v_pool, num_blocks, kv_indices, kv_indptr, kv_lens, n_slots == 0, plan,
     n_work, n_kv_heads, scale * kLog2e, k_new, v_new, slot_mapping, po, pml, o_bytes, ml_bytes,
     cnt, status_word, s);
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
                                 int32_t n_slots, int32_t part_pages, const void* k_new,
                                 const void* v_new, const int32_t* slot_mapping,
                                 void* workspace, int64_t workspace_bytes,
                                 int32_t* status_word, void* stream) {
  return attend_decode(q, out, k_pool, v_pool, num_blocks, kv_indptr, kv_indices, kv_lens,
                       n_seqs, n_heads, n_kv_heads, head_dim, page_size, scale, dtype, plan,
                       n_work, n_slots, part_pages, k_new, v_new, slot_mapping, workspace,
                       workspace_bytes, false, status_word, stream);
}

extern "C" int pkv_attend_decode_noalloc(const void* q, void* out, void* k_pool, void* v_pool,
                                         int64_t num_blocks, const int32_t* kv_indptr,
                                         const int32_t* kv_indices, const int32_t* kv_lens,
                                         int32_t n_seqs, int32_t n_heads, int32_t n_kv_heads,
                                         int32_t head_dim, int32_t page_size, float scale,
                                         int32_t dtype, const int32_t* plan, int32_t n_work,
                                         int32_t n_slots, int32_t part_pages,
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
                       n_work, n_slots, part_pages, k_new, v_new, slot_mapping, ws,
                       (int64_t)PKV_DECODE_SCRATCH_BYTES, true, status_word, stream);
}
