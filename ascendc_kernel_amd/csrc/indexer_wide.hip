// Task2 lightning indexer, wide configuration: 64 index heads x 128 channels,
// up to 8192 candidates, top-k up to 2048 (the DSA layer of DeepSeek-V3.2).
//
// Semantics are those of Model.forward of reference/task2_v0_ref.py:123-144
// after the two projections, with the rounding torch-ROCm applies at these
// shapes (established on the MI355X with planted inputs):
//   RoPE  (:131)  as in the 16-head kernel (rope_pair, slot rule on the flat index)
//   w     (:132)  bf16(fp32(wl) * fp32(scale))
//   S     (:133)  bf16(q . k), fp32 accumulation over channels 0..127 in order
//   score (:134)  bf16(sum_h bf16(relu(S_h) * w_h)), fp32 sum in the order of
//                 torch's reduction kernel for a 64-long middle dimension: Y threads
//                 split the heads (thread y takes heads y, y + Y, ...), each keeps
//                 four accumulators over its heads (accumulator i of thread y gets
//                 heads y + Y i + 4 Y m in order) combined as ((a0 + a1) + a2) + a3,
//                 and the thread totals meet in a halving tree (Y = 2: t0 + t1;
//                 Y = 4: (t0 + t2) + (t1 + t3)). Y follows from the candidate count
//                 T and the output size N = b s T (torch_head_split below; measured
//                 on the MI355X for T up to 8192 and N up to 132 K).
//   mask / top-k / fill (:135-143) as in the 16-head kernel; ties by index.
//
// Workgroup = 4 consecutive tokens x 2 waves (32 heads each). The candidates go
// in tiles of 32 keys (8 KB), copied into a 4-buffer LDS ring by buffer_load ... lds
// and shared by the 8 waves. A wave computes
//   S[32 heads x 32 candidates] = Q[32 x 128] . K^T   (8 x mfma 32x32x16)
// with its 32 head rows permuted (head_of) so that the 16 heads a lane holds for
// one candidate form whole accumulator chains of the order above: Y = 2, wave y =
// thread y, lane half hf = its accumulators 2hf, 2hf+1; Y = 4, lane half hf of wave
// y = thread y + 2hf; Y = 1, lane half hf of wave y = accumulator 2(1 - y) + hf. The
// relu/w/bf16 chain and the sums are lane-local (relu with v_pk_max_i16 on the
// packed bf16 scores, exact fp32 products, IEEE fp32 adds), one v_permlane32_swap
// joins the lane halves, and the two waves' totals meet in LDS. Scores become 16-bit
// order keys in LDS; per token a two-pass 8-bit radix select finds the k-th key,
// the picks are compacted ([> k-th] then [== k-th] in index order) and put in
// (key descending, index ascending) order by a stable two-pass LSD radix sort
// before the int64 indices are written.
#include "dsa_common.h"

using namespace dsa;

namespace {

constexpr int kWH = 64;      // index heads
constexpr int kWD = 128;     // channels per head
constexpr int kTok = 4;      // tokens per workgroup
constexpr int kTileC = 32;   // candidates per tile
constexpr int kRingW = 4;    // LDS tile buffers
constexpr int kMaxT = 8192;
constexpr int kMaxK = 2048;

typedef short s16v2 __attribute__((ext_vector_type(2)));

struct WideParams {
  const uint16_t* q;    // [B, S, 64, 128] projected queries (before RoPE)
  const uint16_t* kv;   // row k of batch b at kv + b*kvbs + k*128
  int64_t kvbs;
  const uint16_t* wl;   // [B, S, 64]
  float wscale;
  const float* freqs;   // [S, rd/2, 2] (rows from start_pos) or nullptr
  int32_t rope_mode;
  int64_t* out;         // [B, S, K]
  uint16_t* gkeys;      // if set: per-candidate results go to this [B*S, T] buffer instead of
                        // LDS and the kernel ends after the scores (no top-k)
  int32_t graw;         // 1: gkeys gets the bf16 scores (masked -inf); 0: 16-bit order keys
  int64_t gstride;      // gkeys row length: T for the scores, T rounded up to 4 for keys
  int32_t B, S, rd, T, K, ratio, causal;
  int64_t offset;
  int32_t groups;       // ceil(S / kTok)
  int32_t csplit;       // candidate chunks per token group (1 unless the keys go to gkeys)
  int32_t ctiles;       // candidate tiles per chunk
  int32_t tpad;         // key row length in LDS (T rounded up to 32)
  int32_t psort;        // power of two >= K (pick buffer length)
};

__device__ __forceinline__ int swz(int r, int c) { return r * 16 + (c ^ (r & 15)); }

// Head held in accumulator register r (0..15) of lane half hf of wave y, for the
// head split KY (register pair m = r/2 is one packed bf16 pair in the score loop):
//  KY = 2: thread y, accumulator i = 2hf + r%2, term m       -> y + 2i + 8m
//  KY = 4: thread y + 2hf, accumulator i = 2(m%2) + r%2, term m/2
//                                                           -> y + 2hf + 4i + 16(m/2)
//  KY = 1: accumulator i = 2(1 - y) + hf, term r            -> i + 4r
template <int KY>
__device__ __forceinline__ int head_of(int y, int hf, int r) {
  const int m = r >> 1;
  if constexpr (KY == 2) return y + 2 * (2 * hf + (r & 1)) + 8 * m;
  else if constexpr (KY == 4) return y + 2 * hf + 4 * (2 * (m & 1) + (r & 1)) + 16 * (m >> 1);
  else return 2 * (1 - y) + hf + 4 * r;
}
// MFMA row R of the 32x32 accumulator sits in lane half (R/4)%2, register 4(R/8) + R%4.
template <int KY>
__device__ __forceinline__ int head_of_row(int R, int y) {
  return head_of<KY>(y, (R >> 2) & 1, 4 * (R >> 3) + (R & 3));
}

__device__ __forceinline__ int n_valid_w(const WideParams& p, int t) {
  if (t >= p.S) return 0;
  if (!p.causal) return p.T;
  const int n = (t + 1) / p.ratio;
  return n < p.T ? n : p.T;
}


// Full wave over a 256-bin histogram (bins ascending in key) kept as NC copies
// kCopyStride words apart and summed here: the bin b with count(bins > b) < need <=
// count(bins >= b); gt = count(bins > b).
constexpr int kCopyStride = 260;  // 16-byte aligned; copy c's bin b is 4c banks off
template <int NC = 1>
__device__ __forceinline__ int find_bin64(const uint32_t* hist, int lane, uint32_t need, uint32_t& gt) {
  u32x4 v = *reinterpret_cast<const u32x4*>(hist + 4 * lane);
#pragma unroll
  for (int c = 1; c < NC; ++c) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(hist + c * kCopyStride + 4 * lane);
    v[0] += w[0];
    v[1] += w[1];
    v[2] += w[2];
    v[3] += w[3];
  }
  const uint32_t local = v[0] + v[1] + v[2] + v[3];
  uint32_t incl = local;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t o = __shfl(incl, (lane + off) & 63, 64);
    if (lane + off < 64) incl += o;
  }
  uint32_t cum = incl - local;
  int fb = -1;
  uint32_t fgt = 0;
#pragma unroll
  for (int i = 3; i >= 0; --i) {
    const uint32_t nc = cum + v[i];
    if (cum < need && nc >= need) {
      fb = 4 * lane + i;
      fgt = cum;
    }
    cum = nc;
  }
  const uint64_t m = __ballot(fb >= 0);
  const int src = m ? (int)__builtin_ctzll(m) : 0;
  gt = __shfl(fgt, src, 64);
  return __shfl(fb, src, 64);
}

// The occupied bins (non-zero total over NC copies) at or above lo_bin of a 256-bin
// histogram, ranked from the top, by one wave: byte b of map (64 words of LDS) becomes
// 255 - #(occupied bins above b) for every such bin b (other bytes: 0). Returns the
// number of those bins.
template <int NC>
__device__ __forceinline__ int rank_map64(const uint32_t* hist, int lane, int lo_bin, uint32_t* map) {
  u32x4 v = *reinterpret_cast<const u32x4*>(hist + 4 * lane);
#pragma unroll
  for (int c = 1; c < NC; ++c) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(hist + c * kCopyStride + 4 * lane);
    v[0] += w[0];
    v[1] += w[1];
    v[2] += w[2];
    v[3] += w[3];
  }
  uint32_t occ = 0u;  // bit i: bin 4 lane + i
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (v[i] != 0u && 4 * lane + i >= lo_bin) occ |= 1u << i;
  const uint32_t local = (uint32_t)__builtin_popcount(occ);
  uint32_t incl = local;  // occupied bins in lanes >= lane
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t o = __shfl(incl, (lane + off) & 63, 64);
    if (lane + off < 64) incl += o;
  }
  uint32_t above = incl - local;
  uint32_t word = 0u;
#pragma unroll
  for (int i = 3; i >= 0; --i)
    if ((occ >> i) & 1u) {
      word |= (255u - above) << (8 * i);
      ++above;
    }
  map[lane] = word;
  return __shfl((int)incl, 0, 64);
}

// hist[bin] += 1 for the active lanes of a wave, one LDS atomic per distinct bin
// (the high bytes of a row's order keys fall into a handful of bins).
__device__ __forceinline__ void hist_add_grouped(uint32_t* hist, uint32_t bin, bool active, int lane) {
  uint64_t m = __ballot(active);
  while (m) {
    const int leader = (int)__builtin_ctzll(m);
    const uint32_t lb = (uint32_t)__shfl((int)bin, leader, 64);
    const uint64_t same = __ballot(active && bin == lb);
    if (lane == leader) atomicAdd(&hist[lb], (uint32_t)__builtin_popcountll(same));
    m &= ~same;
  }
}

// m & ~(b ^ s): the lanes of m whose ballot bit b equals the lane's own bit (s = 0
// or ~0). One v_bitop3 (truth table 0x90) per call: the empty asm keeps the result
// in a register, so that a chain of calls is not regrouped into xors and ors. (The
// operation itself stays in C: the compiler inserts the wait states that a VALU
// read of a ballot just written by a VALU compare needs, which it does not do for
// inline assembly.)
__device__ __forceinline__ uint32_t keep_equal(uint32_t m, uint32_t b, uint32_t s) {
  uint32_t r = m & ~(b ^ s);
  asm("" : "+v"(r));
  return r;
}

// Stable sort, descending on the 8-bit digit (v >> sh) & 255, of the n values
// src[0..n) into dst, by the NW waves (thread index tt) of a workgroup whose every
// thread calls this. Wave w takes the w-th contiguous chunk in rounds of 64; per
// round the lanes holding the same digit are found with one ballot per digit bit
// (a lane keeps the ballot where its own bit is set, its complement where not:
// m &= ~(ballot ^ sext(bit)), one v_bitop3 per half), which gives each value its
// rank among equal digits of the chunk so far (a per-wave running count per digit
// in wr). The digit totals of all waves then give every (wave, digit) its output
// start. Inlined so that src, dst and wr are addressed as LDS. src and dst may be the
// same buffer (every value is read into registers before the first barrier).
// NB < 8: every value's digit has its bits NB..7 equal, so NB ballots tell the
// digits apart. kRemap: each value's byte 3 is replaced, as it is read, by
// remap[byte 3] (bytes of LDS); the values then carry it to dst.
// wr: NW * 256 words, wt: NW words of LDS.
template <int NW, int NB = 8, bool kRemap = false>
__device__ __forceinline__ void radix_pass_desc(const uint32_t* src, uint32_t* dst, int n, int sh,
                                                uint32_t* wr, uint32_t* wt, int tt,
                                                const uint8_t* remap = nullptr) {
  static_assert(NB >= 1 && NB <= 8, "digit bits");
  constexpr int kR = kMaxK / (64 * NW);  // rounds per wave at most
  const int lane = tt & 63, wv = tt >> 6;
  const int chunk = ((n + NW - 1) / NW + 63) & ~63;
  const int c_beg = wv * chunk;
  const int c_end = min(n, c_beg + chunk);
  for (int i = tt; i < NW * 256; i += 64 * NW) wr[i] = 0u;
  __syncthreads();
  uint32_t* myw = wr + wv * 256;
  uint32_t vals[kR], rk[kR];
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    const int c = c_beg + 64 * r + lane;
    const bool act = c < c_end;
    uint32_t v = act ? src[c] : 0u;
    if constexpr (kRemap) v = (v & 0x00ffffffu) | ((uint32_t)remap[v >> 24] << 24);
    const uint32_t d = 255u - ((v >> sh) & 255u);
    const uint64_t am = __ballot(act);
    uint32_t mlo = (uint32_t)am, mhi = (uint32_t)(am >> 32);
    // equal digits <=> equal bits sh .. sh+NB-1 of v; the ballots are all taken
    // before they are used
    uint32_t sx[NB];
    uint64_t bb[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      sx[b] = (uint32_t)__builtin_amdgcn_sbfe((int)v, sh + b, 1);  // 0 or ~0
      asm("" : "+v"(sx[b]));  // the ballot tests sx itself (one compare)
      bb[b] = __ballot(sx[b] != 0u);
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      mlo = keep_equal(mlo, (uint32_t)bb[b], sx[b]);
      mhi = keep_equal(mhi, (uint32_t)(bb[b] >> 32), sx[b]);
    }
    const uint32_t rank = __builtin_amdgcn_mbcnt_hi(mhi, __builtin_amdgcn_mbcnt_lo(mlo, 0u));
    uint32_t old = 0u;
    if (act) old = myw[d];
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    if (act && rank == 0u) myw[d] = old + (uint32_t)(__builtin_popcount(mlo) + __builtin_popcount(mhi));
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    vals[r] = v;
    rk[r] = old + rank;
  }
  __syncthreads();
  // Exclusive scan of the digit totals (digit order = output order), then the
  // start of every (wave, digit) block, written over the counts. Threads
  // 0 .. 64 kSW - 1 take kQ digits each (with more than 256 threads, the first 256
  // take one and the others only meet the barriers).
  constexpr int kQ = (256 / (64 * NW)) > 0 ? 256 / (64 * NW) : 1;  // digits per scan thread
  constexpr int kSW = 256 / (64 * kQ);                            // waves that scan
  const bool scans = wv < kSW;
  uint32_t cnt[kQ][NW];
  uint32_t loc = 0u;
#pragma unroll
  for (int i = 0; i < kQ; ++i)
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      cnt[i][w] = scans ? wr[w * 256 + kQ * tt + i] : 0u;
      loc += cnt[i][w];
    }
  uint32_t incl = loc;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t o = (uint32_t)__shfl_up((int)incl, off, 64);
    if (lane >= off) incl += o;
  }
  if (lane == 63 && scans) wt[wv] = incl;
  __syncthreads();
  if (scans) {
    uint32_t run = incl - loc;
    for (int w = 0; w < wv; ++w) run += wt[w];
#pragma unroll
    for (int i = 0; i < kQ; ++i)
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        wr[w * 256 + kQ * tt + i] = run;
        run += cnt[i][w];
      }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    const int c = c_beg + 64 * r + lane;
    if (c < c_end) {
      const uint32_t d = 255u - ((vals[r] >> sh) & 255u);
      dst[myw[d] + rk[r]] = vals[r];
    }
  }
  __syncthreads();
}

// Top-K of one row of 16-bit order keys held in LDS (keys[0..nv) are the valid
// candidates), by the NW waves (thread index tt) of a workgroup whose every thread
// calls this (it contains __syncthreads): two-pass 8-bit radix select of the K-th
// key, compaction of the picks ([keys > k-th] then the first [== k-th], each in
// index order) as (key << 16 | ~index) composites, a stable radix sort of the
// picks on the key, descending (equal keys keep index order), and the int64
// output (index + offset; -1 for picks beyond the valid candidates).
// hist: max(512, NW * 256) words, sel: 4 words, sb and tmp: K words of LDS each.
template <int NW>
__device__ __forceinline__ void select_topk_row(const uint16_t* keys, int nv, int K, uint32_t* hist,
                                                int32_t* sel, uint32_t* sb, uint32_t* tmp, int tt,
                                                int64_t* out_row, int64_t offset) {
  constexpr int nthr = 64 * NW;
  const int lane = tt & 63;
  const int nw = NW, wv = tt >> 6;
  const bool selecting = nv > K;
  uint32_t* h1 = hist;
  uint32_t* h2 = hist + 256;
  for (int i = tt; i < 512; i += nthr) h1[i] = 0u;
  __syncthreads();
  if (selecting)
    for (int c0 = wv * 64; c0 < nv; c0 += nthr) {
      const int c = c0 + lane;
      hist_add_grouped(h1, c < nv ? (uint32_t)keys[c] >> 8 : 0u, c < nv, lane);
    }
  __syncthreads();
  if (selecting && tt < 64) {
    uint32_t gt;
    const int b1 = find_bin64(h1, lane, (uint32_t)K, gt);
    if (lane == 0) {
      sel[0] = b1;
      sel[1] = (int32_t)gt;
    }
  }
  __syncthreads();
  const int b1 = sel[0];
  if (selecting)
    for (int c = tt; c < nv; c += nthr) {
      const uint32_t u = keys[c];
      if ((int)(u >> 8) == b1) atomicAdd(&h2[u & 255u], 1u);
    }
  __syncthreads();
  if (selecting && tt < 64) {
    uint32_t gt;
    const uint32_t above = (uint32_t)sel[1];
    const int b0 = find_bin64(h2, lane, (uint32_t)K - above, gt);
    if (lane == 0) {
      sel[2] = b0;
      sel[3] = (int32_t)(above + gt);
    }
  }
  __syncthreads();
  const int count = selecting ? K : nv;  // picks that are real candidates
  // Compaction: wave wv scans candidates [wv * chunk, (wv + 1) * chunk) twice, first
  // counting its picks (h1 is free again) and then writing them after the picks of
  // the lower waves, in index order.
  const uint32_t kth = ((uint32_t)b1 << 8) | (uint32_t)sel[2];
  const uint32_t n_gt = (uint32_t)sel[3];
  const int chunk = (nv + 64 * nw - 1) / (64 * nw) * 64;
  const int c_beg = wv * chunk, c_end = min(nv, c_beg + chunk);
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  __syncthreads();  // everyone has read sel before h1 is reused
  if (selecting) {
    uint32_t ng = 0, ne = 0;
    for (int c0 = c_beg; c0 < c_end; c0 += 64) {
      const int c = c0 + lane;
      const uint32_t u = c < c_end ? (uint32_t)keys[c] : 0u;
      ng += __builtin_popcountll(__ballot(c < c_end && u > kth));
      ne += __builtin_popcountll(__ballot(c < c_end && u == kth));
    }
    if (lane == 0) {
      h1[wv] = ng;
      h1[8 + wv] = ne;
    }
  }
  __syncthreads();
  if (selecting) {
    uint32_t run_gt = 0, run_eq = 0;
    for (int w = 0; w < wv; ++w) {
      run_gt += h1[w];
      run_eq += h1[8 + w];
    }
    const uint32_t need_eq = (uint32_t)K - n_gt;
    for (int c0 = c_beg; c0 < c_end; c0 += 64) {
      const int c = c0 + lane;
      const uint32_t u = c < c_end ? (uint32_t)keys[c] : 0u;
      const bool g = c < c_end && u > kth;
      const bool e = c < c_end && u == kth;
      const uint64_t mg = __ballot(g), me = __ballot(e);
      const uint32_t comp = (u << 16) | (0xffffu - (uint32_t)c);
      if (g) sb[run_gt + __builtin_popcountll(mg & below)] = comp;
      if (e) {
        const uint32_t r = run_eq + __builtin_popcountll(me & below);
        if (r < need_eq) sb[n_gt + r] = comp;
      }
      run_gt += __builtin_popcountll(mg);
      run_eq += __builtin_popcountll(me);
    }
  } else {
    for (int c = tt; c < nv; c += nthr) sb[c] = ((uint32_t)keys[c] << 16) | (0xffffu - (uint32_t)c);
  }
  __syncthreads();
  // Stable LSD radix sort on the key: low byte, then high byte.
  radix_pass_desc<NW>(sb, tmp, count, 16, hist, reinterpret_cast<uint32_t*>(sel), tt);
  radix_pass_desc<NW>(tmp, sb, count, 24, hist, reinterpret_cast<uint32_t*>(sel), tt);
  if (out_row != nullptr)
    for (int j = tt; j < K; j += nthr) {
      const uint32_t comp = sb[j];
      const int64_t c = (int64_t)(0xffffu - (comp & 0xffffu));
      out_row[j] = (j < count) ? c + offset : (int64_t)-1;
    }
}

// kFused: the keys of the 4 tokens stay in LDS and each token's two waves run
// the top-k (select_topk_row) at the end. Otherwise the per-candidate results go
// to p.gkeys and the kernel ends after the scores; that instantiation carries no
// select code, which keeps its register count low enough for two workgroups per CU.
template <bool kFused, int KY>
__global__ __launch_bounds__(512) void ix_wide_kernel(WideParams p) {
  static_assert(KY == 1 || KY == 2 || KY == 4, "torch splits 64 heads over 1, 2 or 4 threads");
  extern __shared__ __align__(16) uint8_t smem[];
  uint16_t* keys = reinterpret_cast<uint16_t*>(smem);                                   // [kTok][tpad]
  u32x4* ring = reinterpret_cast<u32x4*>(smem + (size_t)kTok * p.tpad * 2);           // [kRingW][512]
  float* xbuf = reinterpret_cast<float*>(ring + kRingW * 512);                         // [2][kTok][32]
  uint32_t* hist = reinterpret_cast<uint32_t*>(xbuf + 2 * kTok * kTileC);             // [kTok][2][256]
  int32_t* sel = reinterpret_cast<int32_t*>(hist + kTok * 512);                       // [kTok][4]
  uint32_t* sortbuf = reinterpret_cast<uint32_t*>(ring);  // [kTok][psort], after the scores
  uint32_t* tmpbuf = reinterpret_cast<uint32_t*>(sel + kTok * 4);                     // [kTok][psort]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wi = tid >> 6;
  const int tl = wi >> 1;  // token slot
  const int y = wi & 1;    // head parity
  const int hf = lane >> 5;
  const int col = lane & 31;
  // Longest causal rows first: the last token groups of every batch start first.
  // With p.csplit > 1 (few token groups, e.g. decode) a workgroup scores the run of
  // p.ctiles candidate tiles `chunk` of its group; the tile index n below counts
  // from that run's first tile nbase.
  const int b = blockIdx.x % p.B;
  const int rest = (int)(blockIdx.x / p.B);
  const int chunk = rest % p.csplit;
  const int grp = p.groups - 1 - rest / p.csplit;
  const int t0 = grp * kTok;
  const int t = t0 + tl;
  const bool tok_ok = t < p.S;
  const int nv = n_valid_w(p, t);
  const int nv_max = n_valid_w(p, min(t0 + kTok - 1, p.S - 1));
  const int nbase = chunk * p.ctiles;
  const int ntiles = max(0, min((nv_max + kTileC - 1) / kTileC, nbase + p.ctiles) - nbase);
  if (!kFused && ntiles == 0 && !p.graw) return;  // a chunk past this group's last tile
  const int64_t row_bt = (int64_t)b * p.S + (tok_ok ? t : 0);
  uint16_t* mykeys = keys + tl * p.tpad;

  // Q fragments (A operand): row col -> head hq; channels 16ks + 8hf .. +7, RoPE'd on the fly.
  const int hq = head_of_row<KY>(col, y);
  bf16x8 qa[8];
  {
    const uint16_t* qrow = p.q + (row_bt * kWH + hq) * kWD + 8 * hf;
    const int half_rd = p.rd >> 1;
    const int rbase = kWD - p.rd;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      u32x4 v = tok_ok ? *reinterpret_cast<const u32x4*>(qrow + 16 * ks) : u32x4{0u, 0u, 0u, 0u};
      if (p.freqs != nullptr && tok_ok) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int d0 = 16 * ks + 8 * hf + 2 * w;
          if (d0 >= rbase) {
            const int pj = (d0 - rbase) >> 1;
            const int64_t n = (row_bt * kWH + hq) * half_rd + pj;
            const float c = p.freqs[((int64_t)t * half_rd + pj) * 2];
            const float d = p.freqs[((int64_t)t * half_rd + pj) * 2 + 1];
            float re, im;
            rope_pair(bf_lo(v[w]), bf_hi(v[w]), c, d, p.rope_mode, n, re, im);
            v[w] = pack_bf2(re, im);
          }
        }
      }
      qa[ks] = __builtin_bit_cast(bf16x8, v);
    }
  }
  // Head weights of the lane's 16 heads (bf16 bits): wlo[m] = w of register 2m's head
  // in the low half, whi[m] = w of register 2m+1's head in the high half.
  uint32_t wlo[8], whi[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    uint32_t w0 = 0, w1 = 0;
    if (tok_ok) {
      w0 = f2bf(bf2f(p.wl[row_bt * kWH + head_of<KY>(y, hf, 2 * m)]) * p.wscale);
      w1 = f2bf(bf2f(p.wl[row_bt * kWH + head_of<KY>(y, hf, 2 * m + 1)]) * p.wscale);
    }
    wlo[m] = w0;
    whi[m] = w1 << 16;
  }

  // Tile copies: wave wi moves unit wi (rows 4wi .. 4wi+3 of the tile).
  const i32x4 rsrc = make_rsrc(p.kv + (int64_t)b * p.kvbs, (uint32_t)p.T * (uint32_t)(kWD * 2));
  const uint32_t ring_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) u32x4*)ring;
  const int wis = __builtin_amdgcn_readfirstlane(wi);
  const int urow = 4 * wis + (lane >> 4);
  const uint32_t uoff = 16u * (uint32_t)((lane & 15) ^ (urow & 15));
  const uint32_t ulds = ring_lds + 1024u * (uint32_t)wis;
  auto issue = [&](int n) {
    lds_dma16(rsrc, (uint32_t)(kTileC * (nbase + n) + urow) * (uint32_t)(kWD * 2) + uoff,
              ulds + 8192u * (uint32_t)(n % kRingW));
  };
#pragma unroll
  for (int j = 0; j < kRingW - 1; ++j)
    if (j < ntiles) issue(j);
  // Consume the compiler-tracked loads here (their vmcnt(0) also covers the copies).
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) asm volatile("" ::"v"(qa[ks]));
#pragma unroll
  for (int m = 0; m < 8; ++m) asm volatile("" ::"v"(wlo[m]), "v"(whi[m]));

  uint16_t* gdst = (p.gkeys != nullptr && tok_ok) ? p.gkeys + row_bt * p.gstride : nullptr;
  // Wave 0's part of the previous tile (upper lanes): KY = 2, 4 its total (t0, or
  // t0 + t2); KY = 1 accumulators a2 (t0val) and a3 (t0val2).
  float t0val = 0.f, t0val2 = 0.f;
  // Keys of tile n-1: wave 0's part + wave 1's (from LDS) -> bf16 -> order key (or
  // raw bits when dumping).
  auto finalize = [&](int n) {
    if (y == 0 && hf == 1) {
      const float x1 = xbuf[((n & 1) * kTok + tl) * kTileC + col];
      const float t4 = KY == 1 ? (x1 + t0val) + t0val2 : t0val + x1;
      // The reference adds the 0 / -inf mask in bf16: bf16(bf16(x) + 0) = bf16(x + 0),
      // which only turns -0 into +0.
      const float tot = p.causal ? t4 + 0.0f : t4;
      const uint32_t sc = f2bf(tot);
      const int c = kTileC * (nbase + n) + col;
      if (c < nv) {
        // order key: the bf16's sign is tot's (NaN aside), one arithmetic shift
        const uint32_t neg = (uint32_t)((int32_t)__builtin_bit_cast(uint32_t, tot) >> 31);
        const uint16_t key = __builtin_isnan(tot) ? (uint16_t)0xffffu : (uint16_t)(sc ^ (neg | 0x8000u));
        const uint16_t v = (uint16_t)(p.graw ? sc : key);
        if constexpr (kFused) mykeys[c] = v;
        else if (gdst != nullptr) gdst[c] = v;
      }
    }
  };

  // Software pipeline: iteration n issues the products of tile n + 1 one k-step at a
  // time, each followed by one step of tile n's rounding chain (plain VALU work, which
  // the SIMD can issue while the matrix core runs). One 16-byte operand read at a
  // time keeps the register count low enough for two workgroups per CU. Iteration n
  // waits for tile n + 1 and refills the slot of tile n - 1, whose products ran two
  // iterations ago. Tiles go in groups of kRingW so every ring slot is a constant.
  // The scores of consecutive tiles alternate between two accumulator sets (sA, sB),
  // so no register copy is needed between iterations.
  f32x16 sA = {}, sB = {};
  if (ntiles > 0) {
    if (ntiles > 2) wait_vmcnt<2>();
    else if (ntiles > 1) wait_vmcnt<1>();
    else wait_vmcnt<0>();
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
      sA = mfma32x32x16(qa[ks], __builtin_bit_cast(bf16x8, ring[swz(col, 2 * ks + hf)]), sA);
  }
  // Iteration n: s_cur holds S of tile n, s_nx receives S of tile n + 1.
  auto step = [&](const int n, const int j, const f32x16& s_cur, f32x16& s_nx) {
    if (n + 2 < ntiles) wait_vmcnt<1>();
    else wait_vmcnt<0>();
    __syncthreads();  // tile n+1 is in LDS; tile n-1's slot and odd totals are consumed/visible
    if (n > 0) finalize(n - 1);
    if (n + kRingW - 1 < ntiles) issue(n + kRingW - 1);
    // (after the last tile this reads a stale slot; the result is not used)
    const u32x4* kt = ring + ((j + 1) % kRingW) * 512;
    s_nx = f32x16{};
    // acc[i]: the lane's accumulators in the order of head_of (KY = 2: 0, 1; KY = 4:
    // 0..3; KY = 1: the one chain in acc[0]).
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      s_nx = mfma32x32x16(qa[m], __builtin_bit_cast(bf16x8, kt[swz(col, 2 * m + hf)]), s_nx);
      s16v2 pk = __builtin_bit_cast(s16v2, pack_bf2(s_cur[2 * m], s_cur[2 * m + 1]));
      pk = __builtin_elementwise_max(pk, (s16v2){0, 0});  // relu on the bf16 bit patterns
      // bf16 x bf16 products are exact in fp32; each is rounded to bf16 and added
      // with an IEEE fp32 add (v_dot2c's accumulation does not always round like one).
      const uint32_t pv = __builtin_bit_cast(uint32_t, pk);
      const float p0 = bf16_as_f32(bf_lo(pv) * bf_lo(wlo[m]));
      const float p1 = bf16_as_f32(bf_hi(pv) * bf_hi(whi[m]));
      if constexpr (KY == 2) {
        acc[0] = acc[0] + p0;
        acc[1] = acc[1] + p1;
      } else if constexpr (KY == 4) {
        acc[2 * (m & 1)] = acc[2 * (m & 1)] + p0;
        acc[2 * (m & 1) + 1] = acc[2 * (m & 1) + 1] + p1;
      } else {
        acc[0] = acc[0] + p0;
        acc[0] = acc[0] + p1;
      }
    }
    float ty;
    if constexpr (KY == 2) {
      // Lower lanes hold accumulators 0, 1; upper lanes 2, 3 of the same thread.
      const float a01 = acc[0] + acc[1];
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(a01), __float_as_uint(a01), false, false);
      ty = (__uint_as_float(sw[0]) + acc[0]) + acc[1];  // valid in the upper lanes
    } else if constexpr (KY == 4) {
      // Each lane half is one thread: t = ((a0 + a1) + a2) + a3; upper lanes add the
      // lower half's (thread y) to their own (thread y + 2).
      const float tt4 = ((acc[0] + acc[1]) + acc[2]) + acc[3];
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(tt4), __float_as_uint(tt4), false, false);
      ty = __uint_as_float(sw[0]) + tt4;
    } else {
      // Wave 1 holds accumulators 0 (lower) and 1 (upper), wave 0 holds 2 and 3.
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[0]), __float_as_uint(acc[0]), false, false);
      ty = __uint_as_float(sw[0]) + acc[0];  // wave 1: a0 + a1
      if (y == 0) t0val2 = acc[0];           // wave 0: a3 (a2 is sw[0], kept in t0val)
      if (y == 0) ty = __uint_as_float(sw[0]);
    }
    if (y == 1) {
      if (hf == 1) xbuf[((n & 1) * kTok + tl) * kTileC + col] = ty;
    } else {
      t0val = ty;
    }
  };
  static_assert(kRingW % 2 == 0, "the accumulator sets alternate within a ring group");
  for (int n0 = 0; n0 < ntiles; n0 += kRingW) {
#pragma unroll
    for (int j = 0; j < kRingW; ++j) {
      const int n = n0 + j;
      if (n >= ntiles) break;
      if ((j & 1) == 0) step(n, j, sA, sB);
      else step(n, j, sB, sA);
    }
  }
  __syncthreads();
  if (ntiles > 0) finalize(ntiles - 1);
  __syncthreads();

  const int tt = y * 64 + lane;  // thread of the token (0..127)
  if constexpr (!kFused) {
    if (p.graw && gdst != nullptr)  // score dump: never-valid candidates are -inf
      for (int c = nv + tt; c < p.T; c += 128) gdst[c] = (uint16_t)0xff80u;
  } else {
    select_topk_row<2>(mykeys, nv, p.K, hist + tl * 512, sel + tl * 4, sortbuf + tl * p.psort,
                       tmpbuf + tl * p.psort, tt, tok_ok ? p.out + row_bt * p.K : nullptr, p.offset);
  }
}

// Top-K of rows of 16-bit order keys written by ix_wide_kernel: one workgroup
// (256 threads, or 1024 for few rows) per token row. Thread tt holds keys
// [KPT tt, KPT tt + KPT) of the row in registers (index order = thread order, then
// register order):
//   1. high-byte histogram (LDS atomics into 4 lane-interleaved copies), the bin of
//      the K-th key; low-byte histogram of that bin, the K-th key itself (kth) and
//      n_gt = #(keys > kth);
//   2. one workgroup scan of the per-thread counts (#(> kth) | #(== kth) << 16)
//      places every pick: [> kth] at [0, n_gt) and the first K - n_gt [== kth]
//      after them, each in index order;
//   3. stable two-pass LSD radix sort of the picks on the key (descending), in place:
//      the low byte, then the high byte's rank among the bins that hold picks (from
//      the high-byte histogram, which every row takes), in as many ballots per round
//      as that number of bins needs; int64 out.
struct SelParams {
  const uint16_t* keys;  // [B*S, kstride], kstride = T rounded up to a multiple of 4
  int64_t kstride;
  int64_t* out;          // [B*S, K]
  int32_t S, T, K, ratio, causal, psort;
  int64_t offset;
};

// NT threads per workgroup: 256 (32 keys per thread) for many rows, 1024 (8 keys per
// thread) when there are too few rows to fill the CUs (decode), where the row's
// latency is the step's.
// The high-byte histogram is kept in kH1Copies copies (lane l adds to copy l % 4, so
// that the lanes of one atomic instruction that hit the same bin, as the high bytes
// of a row mostly do, are spread over 4 addresses), then the low-byte histogram.
constexpr int kH1Copies = 4;
constexpr int kH2 = kH1Copies * kCopyStride;  // offset of the low-byte histogram
template <int NT>
constexpr int sel_hist_words() { return (NT / 64) * 256 > kH2 + 256 ? (NT / 64) * 256 : kH2 + 256; }

template <int NT>
__global__ __launch_bounds__(NT) void ix_select_kernel(SelParams p) {
  constexpr int NW = NT / 64;
  constexpr int KPT = kMaxT / NT;  // keys per thread
  constexpr int KW = KPT / 4;      // 8-byte words per thread
  // The second sort pass on the high byte's rank (below) saves VALU work where rows
  // share the CU (256 threads); for one row per workgroup of 1024 threads (decode),
  // whose latency is the step's, the rank map's extra serial steps cost more than
  // the ballots they save, so that instantiation sorts on both bytes in full.
  constexpr bool kNarrow = NT <= 256;
  extern __shared__ __align__(16) uint8_t smem[];
  uint32_t* hist = reinterpret_cast<uint32_t*>(smem);     // h1 | h2, then the radix counts
  uint32_t* wt = hist + sel_hist_words<NT>();              // [NW] wave totals
  int32_t* sel = reinterpret_cast<int32_t*>(wt + NW);     // [8]
  uint32_t* hmap = reinterpret_cast<uint32_t*>(sel + 8);  // [64]: 256 bytes, the high bytes' ranks
  uint32_t* sortbuf = hmap + 64;                           // [psort]
  const int tt = threadIdx.x;
  const int lane = tt & 63, wv = tt >> 6;
  const int64_t row = blockIdx.x;
  const int t = (int)(row % p.S);
  int nv = p.T;
  if (p.causal) {
    nv = (t + 1) / p.ratio;
    if (nv > p.T) nv = p.T;
  }
  const int K = p.K;
  const bool selecting = nv > K;
  // Keys of this thread (8-byte loads: rows start 8-byte aligned, kstride % 4 == 0).
  const uint2* src = reinterpret_cast<const uint2*>(p.keys + row * p.kstride) + KW * tt;
  const int c0 = KPT * tt;
  // Order keys are >= 0x007f (-inf), so 0 marks the positions past nv.
  uint2 kw[KW];
#pragma unroll
  for (int i = 0; i < KW; ++i) {
    const int rem = nv - (c0 + 4 * i);  // valid keys in this piece
    kw[i] = rem > 0 ? src[i] : uint2{0u, 0u};
    if (rem == 1) kw[i] = uint2{kw[i].x & 0xffffu, 0u};
    if (rem == 2) kw[i].y = 0u;
    if (rem == 3) kw[i].y &= 0xffffu;
  }
  auto key_of = [&](int e) -> uint32_t {
    const uint32_t w = (e & 2) ? kw[e >> 2].y : kw[e >> 2].x;
    return (e & 1) ? (w >> 16) : (w & 0xffffu);
  };
  // The histograms take whole 4-key pieces that start below nv: the 0 to 3 zero keys
  // past nv in the last such piece fall into bin 0 of the high-byte histogram (and
  // of the low-byte one when that bin is selected), which start at minus their
  // number. (Every zero key past nv in one bin would serialise its atomics.)
  const int npiece = min(max((nv - c0 + 3) >> 2, 0), KW);  // pieces of this thread
  const uint32_t pad = (uint32_t)(((nv + 3) & ~3) - nv);
  for (int i = tt; i < kH2 + 256; i += NT) hist[i] = (i == 0) ? 0u - pad : 0u;
  __syncthreads();
  uint32_t kth = 0u, n_gt = (uint32_t)nv, need_eq = 0u;
  // A wave whose keys all lie past nv (causal rows) skips the per-key loops.
  const bool wlive = __builtin_amdgcn_readfirstlane(wv) * (64 * KPT) < nv;
  if ((kNarrow || selecting) && wlive) {
    uint32_t* h1 = hist + (lane & (kH1Copies - 1)) * kCopyStride;
#pragma unroll
    for (int e = 0; e < KPT; ++e)
      if ((e >> 2) < npiece) atomicAdd(&h1[key_of(e) >> 8], 1u);
  }
  __syncthreads();
  // Wave 0: the high-byte bin of the K-th key (when selecting), and the ranks of the
  // bins that hold picks: every occupied bin at or above that one (above bin 0
  // without selection).
  if (wv == 0) {
    uint32_t gt = 0u;
    const int b1 = selecting ? find_bin64<kH1Copies>(hist, lane, (uint32_t)K, gt) : 0;
    const int nocc = kNarrow ? rank_map64<kH1Copies>(hist, lane, b1, hmap) : 256;
    if (lane == 0) {
      sel[0] = b1;
      sel[1] = (int32_t)gt;
      sel[4] = nocc;
    }
  }
  __syncthreads();
  if (selecting) {
    const uint32_t b1 = (uint32_t)sel[0];
    if (b1 == 0u && tt == 0) atomicSub(&hist[kH2], pad);
    if (wlive) {
#pragma unroll
      for (int e = 0; e < KPT; ++e) {
        const uint32_t u = key_of(e);
        if ((e >> 2) < npiece && (u >> 8) == b1) atomicAdd(&hist[kH2 + (u & 255u)], 1u);
      }
    }
    __syncthreads();
    if (wv == 0) {
      uint32_t gt;
      const uint32_t above = (uint32_t)sel[1];
      const int b0 = find_bin64(hist + kH2, lane, (uint32_t)K - above, gt);
      if (lane == 0) {
        sel[2] = b0;
        sel[3] = (int32_t)(above + gt);
      }
    }
    __syncthreads();
    kth = (b1 << 8) | (uint32_t)sel[2];
    n_gt = (uint32_t)sel[3];
    need_eq = (uint32_t)K - n_gt;
  }
  // Per-thread pick counts, packed (> kth) | (== kth) << 16, and their exclusive
  // scan over the workgroup.
  // Without selection every key > 0 is a pick; kth >= 0x007f when selecting, so
  // the 0 marks never count.
  const uint32_t kth_e = selecting ? kth : 0xffffffffu;
  uint32_t cnt = 0u, incl = 0u;
  if (wlive) {
#pragma unroll
    for (int e = 0; e < KPT; ++e) {
      const uint32_t u = key_of(e);
      cnt += (u > kth ? 1u : 0u) + (u == kth_e ? 0x10000u : 0u);
    }
    incl = cnt;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t o = (uint32_t)__shfl_up((int)incl, off, 64);
      if (lane >= off) incl += o;
    }
  }
  if (lane == 63) wt[wv] = incl;
  __syncthreads();
  uint32_t base = incl - cnt;
  for (int w = 0; w < wv; ++w) base += wt[w];
  uint32_t og = base & 0xffffu, oe = n_gt + (base >> 16);  // next slots of each kind
  const uint32_t oe_end = n_gt + need_eq;
  const uint32_t ibase = 0xffffu - (uint32_t)c0;
  // The comparisons are recomputed below rather than kept from the count loop (64
  // lane masks of it would not fit in the scalar registers).
  if (wlive) {
#pragma unroll
    for (int i = 0; i < KW; ++i) asm volatile("" : "+v"(kw[i]));
#pragma unroll
    for (int e = 0; e < KPT; ++e) {
      const uint32_t u = key_of(e);
      const bool g = u > kth, q = u == kth_e;
      const bool ok = g | (q & (oe < oe_end));
      const uint32_t pos = g ? og : oe;
      // (u << 16) | (index bits): one v_perm of the key's 16-bit half and ibase - e
      const uint32_t w = (e & 2) ? kw[e >> 2].y : kw[e >> 2].x;
      const uint32_t comp = __builtin_amdgcn_perm(w, ibase - (uint32_t)e, (e & 1) ? 0x07060100u : 0x05040100u);
      if (ok) sortbuf[pos] = comp;
      og += g ? 1u : 0u;
      oe += q ? 1u : 0u;
    }
  }
  const int count = selecting ? K : nv;
  const int nocc = __builtin_amdgcn_readfirstlane(sel[4]);
  __syncthreads();
  // Stable LSD radix sort of the picks on the key, descending, in place: the low byte,
  // then the high byte's rank among the nocc bins that hold picks (the first pass
  // writes it over the high byte as 255 - rank), which takes ceil(log2 nocc) ballots
  // per round instead of 8 (one bin: no second pass).
  radix_pass_desc<NW, 8, kNarrow>(sortbuf, sortbuf, count, 16, hist, wt, tt,
                                  reinterpret_cast<const uint8_t*>(hmap));
  switch (!kNarrow ? 8 : nocc <= 1 ? 0 : 32 - __builtin_clz((uint32_t)(nocc - 1))) {
    case 0: break;
    case 1: radix_pass_desc<NW, 1>(sortbuf, sortbuf, count, 24, hist, wt, tt); break;
    case 2: radix_pass_desc<NW, 2>(sortbuf, sortbuf, count, 24, hist, wt, tt); break;
    case 3: radix_pass_desc<NW, 3>(sortbuf, sortbuf, count, 24, hist, wt, tt); break;
    case 4: radix_pass_desc<NW, 4>(sortbuf, sortbuf, count, 24, hist, wt, tt); break;
    case 5: radix_pass_desc<NW, 5>(sortbuf, sortbuf, count, 24, hist, wt, tt); break;
    case 6: radix_pass_desc<NW, 6>(sortbuf, sortbuf, count, 24, hist, wt, tt); break;
    case 7: radix_pass_desc<NW, 7>(sortbuf, sortbuf, count, 24, hist, wt, tt); break;
    default: radix_pass_desc<NW, 8>(sortbuf, sortbuf, count, 24, hist, wt, tt); break;
  }
  int64_t* out_row = p.out + row * K;
  for (int j = tt; j < K; j += NT) {
    const uint32_t comp = sortbuf[j];
    out_row[j] = (j < count) ? (int64_t)(0xffffu - (comp & 0xffffu)) + p.offset : (int64_t)-1;
  }
}

}  // namespace

// Called by the indexer entry points for h == 64, d == 128 (checks common to both
// configurations are done by the caller).
int64_t dsa_indexer_wide_workspace_bytes(int64_t b, int64_t s, int64_t n_cand) {
  return b * s * ((n_cand + 3) & ~INT64_C(3)) * 2;  // a 16-bit order key per (token, candidate)
}

// The number of threads torch-ROCm's reduction kernel splits the 64 heads over when it
// sums the bf16 [b, s, 64, T] products over the heads (reference/task2_v0_ref.py:134),
// from its launch configuration for a reduction over a non-innermost dimension: the
// output [b, s, T] is vectorised by 4 (T % 4 == 0), 2 (T % 2 == 0) or 1; a block
// is min(pow2(N / vec), 64) threads wide (N = b s T outputs, 512 / vec threads in all)
// and as many tall as fit, up to 64; the heads are split over the block's height only
// when each of those threads still sums at least 16 of them. Measured on the MI355X
// for T in 2 .. 8192 and N up to 132 K (T = 1, a single candidate, is reduced
// differently, but its top-1 does not depend on the score).
int torch_head_split(int64_t n_out, int64_t T) {
  const int vec = (T % 4 == 0) ? 4 : (T % 2 == 0) ? 2 : 1;
  const int64_t max_thr = 512 / vec;
  const int64_t dim0 = n_out / vec;
  int64_t p2 = 1;
  while (p2 * 2 <= dim0 && p2 < max_thr) p2 *= 2;
  const int64_t width = p2 < 64 ? p2 : 64;
  int64_t height = max_thr / width;
  if (height > 64) height = 64;
  return (64 >= 16 * height) ? (int)height : 1;
}

// With a workspace of at least dsa_indexer_wide_workspace_bytes: the score kernel
// writes order keys to it and ix_select_kernel ranks them (one workgroup per
// token). Without: one fused kernel keeps the keys of 4 tokens in LDS. With
// `scores`: the score kernel writes the bf16 scores there and nothing is ranked.
int dsa_indexer_wide_launch(const void* q, const void* kv_cache, int64_t kv_batch_stride,
                            const void* wl, float w_scale, const void* freqs_cis,
                            int32_t rope_mode, int64_t* out, uint16_t* scores, int64_t b,
                            int64_t s, int64_t rd, int64_t n_cand, int64_t k_out,
                            int64_t ratio, int32_t causal, int64_t offset, void* workspace,
                            int64_t workspace_bytes, hipStream_t stream) {
  if (n_cand > kMaxT) return DSA_ERR_UNSUPPORTED;
  if (k_out > kMaxK) return DSA_ERR_UNSUPPORTED;
  // torch reduces a single candidate's heads another way; its score (not its top-1) differs.
  if (scores != nullptr && n_cand == 1) return DSA_ERR_UNSUPPORTED;
  const int ky = torch_head_split(b * s * n_cand, n_cand);
  const bool two_pass = scores == nullptr && workspace != nullptr &&
                        workspace_bytes >= dsa_indexer_wide_workspace_bytes(b, s, n_cand);
  if (workspace != nullptr && ((uintptr_t)workspace & 15u)) return DSA_ERR_ALIGN;
  WideParams p;
  p.q = (const uint16_t*)q;
  p.kv = (const uint16_t*)kv_cache;
  p.kvbs = kv_batch_stride;
  p.wl = (const uint16_t*)wl;
  p.wscale = w_scale;
  p.freqs = (const float*)freqs_cis;
  p.rope_mode = rope_mode;
  p.out = out;
  p.gkeys = scores != nullptr ? scores : (two_pass ? (uint16_t*)workspace : nullptr);
  p.graw = scores != nullptr ? 1 : 0;
  p.gstride = scores != nullptr ? n_cand : ((n_cand + 3) & ~INT64_C(3));
  p.B = (int32_t)b;
  p.S = (int32_t)s;
  p.rd = (int32_t)rd;
  p.T = (int32_t)n_cand;
  p.K = (int32_t)k_out;
  p.ratio = (int32_t)(ratio > (1 << 30) ? (1 << 30) : ratio);
  p.causal = causal ? 1 : 0;
  p.offset = offset;
  p.groups = (int32_t)((s + kTok - 1) / kTok);
  // Candidate split for the two-pass path when the token groups alone would leave
  // most CUs idle (decode: one group scoring every candidate on one CU): chunks of
  // at least two tiles, about two workgroups per CU in all.
  const int64_t ntile_all = (n_cand + kTileC - 1) / kTileC;
  p.csplit = 1;
  p.ctiles = (int32_t)(ntile_all > 0 ? ntile_all : 1);
  if (two_pass) {
    int cu = 0;
    if (dsa_host::device_cu_count(&cu) != DSA_OK) return DSA_ERR_DEVICE;
    const int64_t base = b * (int64_t)p.groups;
    if (base < 2 * (int64_t)cu && ntile_all >= 4) {
      int64_t want = (2 * (int64_t)cu + base - 1) / base;
      if (want > ntile_all / 2) want = ntile_all / 2;
      const int64_t ct = (ntile_all + want - 1) / want;
      p.ctiles = (int32_t)ct;
      p.csplit = (int32_t)((ntile_all + ct - 1) / ct);
    }
  }
  int ps = 1;
  while (ps < k_out) ps <<= 1;
  p.psort = ps;
  size_t smem;
  if (p.gkeys != nullptr) {
    p.tpad = 0;  // no key rows in LDS
    smem = (size_t)kRingW * 8192 + 2 * kTok * kTileC * 4 + kTok * 512 * 4 + kTok * 4 * 4;
  } else {
    p.tpad = (int32_t)((n_cand + kTileC - 1) / kTileC * kTileC);
    smem = (size_t)kTok * p.tpad * 2 + (size_t)kRingW * 8192 + 2 * kTok * kTileC * 4 +
           kTok * 512 * 4 + kTok * 4 * 4 + (size_t)kTok * ps * 4;
  }
  if (smem > 160 * 1024) return DSA_ERR_UNSUPPORTED;
  const bool fused = p.gkeys == nullptr;
  const void* kfns[2][3] = {
      {(const void*)ix_wide_kernel<false, 1>, (const void*)ix_wide_kernel<false, 2>,
       (const void*)ix_wide_kernel<false, 4>},
      {(const void*)ix_wide_kernel<true, 1>, (const void*)ix_wide_kernel<true, 2>,
       (const void*)ix_wide_kernel<true, 4>}};
  const int kyi = ky == 1 ? 0 : ky == 2 ? 1 : 2;
  const void* kfn = kfns[fused ? 1 : 0][kyi];
  if (dsa_host::ensure_dyn_lds(kfn, (int)smem) != DSA_OK) return DSA_ERR_LAUNCH;
  const int64_t blocks = b * p.groups * (int64_t)p.csplit;
  if (blocks > INT32_MAX || b * s > INT32_MAX) return DSA_ERR_SHAPE;
  void* kargs[] = {&p};
  if (hipLaunchKernel(kfn, dim3((unsigned)blocks), dim3(512), kargs, smem, stream) != hipSuccess)
    return DSA_ERR_LAUNCH;
  if (hipGetLastError() != hipSuccess) return DSA_ERR_LAUNCH;
  if (two_pass) {
    SelParams sp;
    sp.keys = (const uint16_t*)workspace;
    sp.kstride = p.gstride;
    sp.out = out;
    sp.S = p.S;
    sp.T = p.T;
    sp.K = p.K;
    sp.ratio = p.ratio;
    sp.causal = p.causal;
    sp.psort = p.psort;
    sp.offset = offset;
    // Fewer rows than CUs (decode): 1024 threads per row; otherwise 256.
    int cu = 0;
    if (dsa_host::device_cu_count(&cu) != DSA_OK) return DSA_ERR_DEVICE;
    const bool wide_rows = b * s < (int64_t)cu;
    void (*sfn)(SelParams) = wide_rows ? ix_select_kernel<1024> : ix_select_kernel<256>;
    const int snt = wide_rows ? 1024 : 256;
    const size_t smem2 = (size_t)(wide_rows ? sel_hist_words<1024>() : sel_hist_words<256>()) * 4 +
                         (size_t)(snt / 64) * 4 + 32 + 256 + (size_t)ps * 4;
    if (dsa_host::ensure_dyn_lds((const void*)sfn, (int)smem2) != DSA_OK) return DSA_ERR_LAUNCH;
    hipLaunchKernelGGL(sfn, dim3((unsigned)(b * s)), dim3(snt), smem2, stream, sp);
    if (hipGetLastError() != hipSuccess) return DSA_ERR_LAUNCH;
  }
  return DSA_OK;
}
