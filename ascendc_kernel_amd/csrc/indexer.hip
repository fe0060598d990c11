// Task2: lightning indexer (RoPE + relu-weighted multi-head score + causal
// mask + top-k) on gfx950 (MI355X).
//
// Semantics follow Model.forward of reference/task2_v0_ref.py:123-144 after the
// two projections, reproducing the rounding torch applies on the same GPU:
//   RoPE   (:93-104,131)  q[..., d-rd:] *= freqs_cis as complex, rounded to bf16
//   w      (:132)         bf16(fp32(wl) * w_scale)
//   S      (:133)         bf16(q . k), fp32 accumulate in channel order 0..d-1
//   score  (:134)         bf16(sum_h bf16(relu(S_h) * w_h)); the fp32 head sum uses
//                         four accumulators (heads j, j+4, j+8, j+12 for j = 0..3)
//                         combined as ((a0 + a1) + a2) + a3
//   mask   (:135-137)     k >= (t+1)//ratio -> -inf
//   top-k  (:138)         value descending, ties by index ascending
//   fill   (:139-143)     masked picks -> -1, others + offset
// The rounding rules were established on the MI355X against torch 2.10-ROCm
// with planted inputs (GEMM: MFMA in channel order; head sum: the accumulator
// pattern above; RoPE: see rope_pair).
//
// One wave owns two consecutive tokens of one batch. Their 2 x 16 head rows
// form the A operand of v_mfma_f32_32x32x16_bf16 against 32 candidate keys per
// tile, in a row order that leaves every lane all 16 head scores of one
// (token, candidate), so the epilogue and the head sum are lane-local. Scores
// become 16-bit order keys in LDS; a two-pass 8-bit radix select per half-wave
// finds the k-th key, ties are taken in index order with ballots, and the k
// winners are bitonic-sorted on a (key, ~index) composite before the int64
// indices are written. Waves take token pairs from the end of the sequence
// first, so the longest causal rows start first.
#include "dsa_common.h"

#include <atomic>
#include <type_traits>
#include <mutex>

using namespace dsa;

namespace {

typedef short s16v2 __attribute__((ext_vector_type(2)));

constexpr int kH = 16;  // index heads handled by the fused kernel
constexpr int kD = 64;  // index head dim handled by the fused kernel

// ---------------------------------------------------------------------------
// Standalone in-place RoPE: one thread per complex pair.
struct RopeParams {
  uint16_t* q;
  const float* freqs;  // [s, rd/2, 2]
  int64_t rows;        // b * s * h
  int32_t S, H, D, rd, mode;
};

__global__ __launch_bounds__(256) void rope_kernel(RopeParams p) {
  const int half_rd = p.rd >> 1;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= p.rows * half_rd) return;
  const int64_t row = gid / half_rd;
  const int j = (int)(gid - row * half_rd);
  const int t = (int)((row / p.H) % p.S);
  uint32_t* w = reinterpret_cast<uint32_t*>(p.q + row * p.D + (p.D - p.rd) + 2 * j);
  const uint32_t x = *w;
  const float c = p.freqs[((int64_t)t * half_rd + j) * 2];
  const float d = p.freqs[((int64_t)t * half_rd + j) * 2 + 1];
  float re, im;
  rope_pair(bf_lo(x), bf_hi(x), c, d, p.mode, gid, re, im);
  *w = pack_bf2(re, im);
}

// ---------------------------------------------------------------------------
// Fused score + top-k.
struct IxParams {
  const uint16_t* q;    // [B, S, 16, 64]
  const uint16_t* kv;   // row k of batch b at kv + b*kvbs + k*64
  int64_t kvbs;
  const uint16_t* wl;   // [B, S, 16]
  float wscale;
  const float* freqs;   // [S, rd/2, 2] or nullptr
  int32_t rope_mode;
  int64_t* out;         // [B, S, K]
  uint16_t* scores;     // optional [B, S, T] bf16 score dump (masked entries -inf)
  int32_t B, S, rd, T, K, ratio, causal;
  int64_t offset;
  int32_t npairs;       // ceil(S / 2)
  int32_t keys_bytes;   // LDS bytes of the key area of one wave (16-byte multiple)
  int32_t wave_bytes;   // LDS bytes per wave
};

__device__ __forceinline__ int n_valid(const IxParams& p, int t) {
  if (t >= p.S) return 0;
  if (!p.causal) return p.T;
  const int n = (t + 1) / p.ratio;
  return n < p.T ? n : p.T;
}

// The middle of three unsigned values: med3(x, y, ~0) = max(x, y), med3(x, y, 0) =
// min(x, y). The compiler turns this form into one v_med3_u32 (and, being its own
// instruction, keeps the wait states a following DPP read of the result needs).
__device__ __forceinline__ uint32_t med3_u32(uint32_t x, uint32_t y, uint32_t z) {
  return max(min(x, y), min(max(x, y), z));
}

// v from lane (lane ^ m) within each 32-lane half (m in 1, 2, 4, 8, 16): DPP quad
// permutations for 1 and 2, a row rotation by 8 for 8, ds_swizzle otherwise.
__device__ __forceinline__ uint32_t xor_lanes(uint32_t v, int m) {
  const int x = (int)v;
  if (m == 1) return (uint32_t)__builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false);  // [1,0,3,2]
  if (m == 2) return (uint32_t)__builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false);  // [2,3,0,1]
  if (m == 8) return (uint32_t)__builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, false); // row_ror:8
  if (m == 4) return (uint32_t)__builtin_amdgcn_ds_swizzle(x, (4 << 10) | 0x1F);
  return (uint32_t)__builtin_amdgcn_ds_swizzle(x, (16 << 10) | 0x1F);
}

__device__ __forceinline__ void lds_fence() { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront"); }

// Per half-wave: the bin b of a 256-bin histogram (bins ascending in key) with
// count(bins > b) < need <= count(bins >= b); returns -1 when the half holds
// fewer than `need` entries. `gt` receives count(bins > b).
__device__ __forceinline__ int find_bin(const uint32_t* hist, int lane, uint32_t need, uint32_t& gt) {
  const int hl = lane & 31, half = lane >> 5;
  const u32x4 lo4 = *reinterpret_cast<const u32x4*>(hist + 8 * hl);
  const u32x4 hi4 = *reinterpret_cast<const u32x4*>(hist + 8 * hl + 4);
  const uint32_t bins[8] = {lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
  uint32_t local = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) local += bins[i];
  uint32_t incl = local;
#pragma unroll
  for (int off = 1; off < 32; off <<= 1) {
    const uint32_t o = __shfl(incl, (lane + off) & 63, 64);
    if (hl + off < 32) incl += o;
  }
  uint32_t cum = incl - local;
  int fb = -1;
  uint32_t fgt = 0;
#pragma unroll
  for (int i = 7; i >= 0; --i) {
    const uint32_t nc = cum + bins[i];
    if (cum < need && nc >= need) {
      fb = 8 * hl + i;
      fgt = cum;
    }
    cum = nc;
  }
  const uint32_t hm = (uint32_t)(__ballot(fb >= 0) >> (32 * half));
  const int src = hm ? (int)(__builtin_ctz(hm)) + 32 * half : lane;
  const int b = __shfl(fb, src, 64);
  gt = __shfl(fgt, src, 64);
  return hm ? b : -1;
}

// kDump: the bf16 scores are written to p.scores (the score-stage entry point);
// the top-k build carries no dump code in its tile loop.
template <int E, bool kDump>
__global__ __launch_bounds__(256) void ix_score_topk_kernel(IxParams p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int KP = 32 * E;  // sort size per half-wave
  const int lane = threadIdx.x & 63;
  const int wi = threadIdx.x >> 6;
  // A workgroup = 4 consecutive token pairs (8 tokens) of one batch, so that its
  // waves share the candidate tiles; groups from the end of the sequence (the
  // longest causal rows) start first. Waves past the last pair still take part in
  // the tile copies and barriers (their tokens are >= S and produce nothing).
  const int ngroups = (p.npairs + 3) >> 2;
  const int b = (int)(blockIdx.x % (unsigned)p.B);
  const int grp = ngroups - 1 - (int)(blockIdx.x / (unsigned)p.B);
  const int pr = 4 * grp + wi;
  const int t0 = 2 * pr;
  const int half = lane >> 5, hl = lane & 31;
  const int t = t0 + half;

  unsigned char* wbase = smem + (size_t)wi * p.wave_bytes;
  uint16_t* keys = reinterpret_cast<uint16_t*>(wbase) ;                // [2][NT][32]
  uint32_t* hist = reinterpret_cast<uint32_t*>(wbase + p.keys_bytes);   // [2][256]
  uint32_t* myhist = hist + 256 * half;

  const int nv = n_valid(p, t);
  // Tiles of the workgroup: up to the valid candidates of its last token (the
  // count grows with t).
  const int tg_last = min(2 * (4 * grp + 3) + 1, p.S - 1);
  const int ntile = (n_valid(p, tg_last) + 31) >> 5;
  const int ntile_all = (p.keys_bytes / 128);
  // Candidate tiles (32 rows x 128 B) in a 3-slot LDS ring after the wave areas.
  uint8_t* ring = smem + 4 * (size_t)p.wave_bytes;

  // Head weights of this half's token, bf16(fp32(wl) * w_scale), fp32 copies.
  float w[kH];
  if (t < p.S) {
    const u32x4* wp = reinterpret_cast<const u32x4*>(p.wl + ((int64_t)b * p.S + t) * kH);
    const u32x4 w0 = wp[0], w1 = wp[1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      w[2 * i] = bf2f(f2bf(bf_lo(w0[i]) * p.wscale));
      w[2 * i + 1] = bf2f(f2bf(bf_hi(w0[i]) * p.wscale));
      w[8 + 2 * i] = bf2f(f2bf(bf_lo(w1[i]) * p.wscale));
      w[8 + 2 * i + 1] = bf2f(f2bf(bf_hi(w1[i]) * p.wscale));
    }
  } else {
#pragma unroll
    for (int i = 0; i < kH; ++i) w[i] = 0.f;
  }

  // A operand: row i = lane % 32 is token t0 + (i/4)%2, head i%4 + 4(i/8); lane
  // holds channels 16ks + 8(lane/32) .. +7 of that row, RoPE applied when asked.
  // The 32x32 product leaves rows 8(r/4) + 4(lane/32) + r%4 in accumulator r of a
  // lane, so with this row order accumulator r of lanes 0..31 is head r of token t0
  // and of lanes 32..63 head r of token t0 + 1, for candidate lane % 32: every lane
  // holds all 16 heads of one (token, candidate) without an exchange of halves.
  bf16x8 qa[4];
  {
    const int tq = t0 + ((lane >> 2) & 1);
    const int hq = (lane & 3) | (((lane & 31) >> 3) << 2);
    const int hsel = lane >> 5;
    if (tq < p.S) {
      const int64_t row = ((int64_t)b * p.S + tq) * kH + hq;
      const uint16_t* src = p.q + row * kD;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        u32x4 v = *reinterpret_cast<const u32x4*>(src + 16 * ks + 8 * hsel);
        if (p.freqs != nullptr) {
          const int half_rd = p.rd >> 1;
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int dch = 16 * ks + 8 * hsel + 2 * jj;
            const int pj = (dch - (kD - p.rd)) >> 1;
            if (dch >= kD - p.rd) {
              const float c = p.freqs[((int64_t)tq * half_rd + pj) * 2];
              const float d = p.freqs[((int64_t)tq * half_rd + pj) * 2 + 1];
              const int64_t n = row * half_rd + pj;
              float re, im;
              rope_pair(bf_lo(v[jj]), bf_hi(v[jj]), c, d, p.rope_mode, n, re, im);
              v[jj] = pack_bf2(re, im);
            }
          }
        }
        qa[ks] = __builtin_bit_cast(bf16x8, v);
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) qa[ks] = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
    }
  }

  // Zero this half's histogram (8 bins per lane).
  *reinterpret_cast<u32x4*>(myhist + 8 * hl) = u32x4{0u, 0u, 0u, 0u};
  *reinterpret_cast<u32x4*>(myhist + 8 * hl + 4) = u32x4{0u, 0u, 0u, 0u};
  lds_fence();

  // Tile n is copied by buffer_load ... lds into ring slot n % 3: wave wi moves rows
  // 8wi .. 8wi+7 (lane l: row 8wi + l/8, 16-byte chunk (l%8) ^ (row%8), so chunk c of
  // row r sits at position 8r + (c ^ (r%8)) and the fragment reads below spread over
  // all banks). Rows >= T read as zero through the resource's range.
  const i32x4 krs = make_rsrc(p.kv + (int64_t)b * p.kvbs, (uint32_t)p.T * (uint32_t)(kD * 2));
  const uint32_t ring_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)ring;
  const int wis = __builtin_amdgcn_readfirstlane(wi);
  const int crow = 8 * wis + (lane >> 3);
  const uint32_t coff = (uint32_t)(crow * kD + 8 * ((lane & 7) ^ (crow & 7))) * 2u;
  auto issue = [&](int n, int slot) {
    lds_dma16(krs, (uint32_t)(32 * n * kD * 2) + coff, ring_lds + 4096u * (uint32_t)slot + 1024u * (uint32_t)wis);
  };
#pragma unroll
  for (int j = 0; j < 2; ++j)
    if (j < ntile) issue(j, j);
  // Consume the compiler-tracked loads here: its own vmcnt(0) for them (which also
  // covers the copies just issued) then stays out of the loop.
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) asm volatile("" ::"v"(qa[ks]));
#pragma unroll
  for (int i = 0; i < kH; ++i) asm volatile("" ::"v"(w[i]));
  // B operand: candidate 32*tile + lane%32, channels 16ks + 8(lane/32) .. +7.
  const int kcol = lane & 31;
  const int khalf = lane >> 5;
  // Lane offsets of the four B fragments inside a ring slot (the slot is a constant in
  // each unrolled step below, so it becomes the LDS instructions' immediate offset).
  uint32_t boff[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    boff[ks] = ring_lds + 16u * (uint32_t)(8 * kcol + ((2 * ks + khalf) ^ (kcol & 7)));
  // The smaller of the two tokens' valid candidate counts (wave-uniform).
  const int nv_min = min(__builtin_amdgcn_readfirstlane(nv), __builtin_amdgcn_readlane(nv, 32));
  auto step = [&](auto slot_c, const int tile) {
    constexpr int kSlot = decltype(slot_c)::value;  // tile % 3
    if (tile + 1 < ntile) wait_vmcnt<1>();
    else wait_vmcnt<0>();
    __syncthreads();  // tile `tile` is in LDS for every wave; the slot of tile-1 is free
    if (tile + 2 < ntile) issue(tile + 2, (kSlot + 2) % 3);  // (tile + 2) % 3 == (tile - 1) % 3
    f32x16 acc = {};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const auto* src = (__attribute__((address_space(3))) const u32x4*)(uintptr_t)(boff[ks] + 4096u * kSlot);
      acc = mfma32x32x16(qa[ks], __builtin_bit_cast(bf16x8, *src), acc);
    }

    // The einsum's bf16 rounding, then relu on the bf16 bit patterns (both heads
    // of a word at once): word k holds heads 2k, 2k+1.
    uint32_t pk[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      s16v2 h = __builtin_bit_cast(s16v2, pack_bf2(acc[2 * k], acc[2 * k + 1]));
      pk[k] = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(h, (s16v2){0, 0}));
    }
    // * w -> bf16 (the products are exact in fp32), as fp32 values: one
    // v_cvt_pk_bf16_f32 with a zero low operand leaves bf16(x) in the high half and
    // zeros below it, which is bf16(x) as an fp32 value.
    float v[16];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      v[2 * k] = bf16_as_f32(bf_lo(pk[k]) * w[2 * k]);
      v[2 * k + 1] = bf16_as_f32(bf_hi(pk[k]) * w[2 * k + 1]);
    }
    // IEEE fp32 adds in torch's order (accumulator j sums heads j, j+4, j+8, j+12).
    // torch's four accumulators start at +0; adding the +0 once to the total instead
    // gives the same value (x + 0 == x except for the sign of a zero, and a -0 can
    // only reach the total when every term is -0).
    float a4[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) a4[j] = ((v[j] + v[j + 4]) + v[j + 8]) + v[j + 12];
    const float tot = (((a4[0] + a4[1]) + a4[2]) + a4[3]) + 0.0f;
    // The reference adds the 0/-inf mask, bf16(x + 0), which only turns -0 into +0.
    // Here sc is never -0: tot is +0 (the + 0 above) or a sum of bf16 values, all
    // multiples of 2^-133, so |tot| >= 2^-133 rounds to a nonzero bf16 (the conversion
    // keeps fp32 denormals: it matches IEEE round-to-nearest-even on them).
    const uint16_t sc = f2bf(tot);
    const int c = 32 * tile + hl;
    const bool valid = c < nv;
    // Order key: sign set -> all bits flipped, else the sign bit flipped; the sign of
    // the bf16 is that of tot (NaN aside), taken from tot's bits with one shift.
    const uint32_t neg = (uint32_t)((int32_t)__builtin_bit_cast(uint32_t, tot) >> 31);
    uint16_t u = (uint16_t)(sc ^ (neg | 0x8000u));
    if (__builtin_isnan(tot)) u = 0xffffu;  // NaN ranks above everything
    if constexpr (kDump) {
      if (t < p.S && c < p.T)
        p.scores[((int64_t)b * p.S + t) * p.T + c] = valid ? sc : (uint16_t)0xff80u;
    }
    if (32 * tile + 32 <= nv_min) {  // (wave-uniform) every lane's candidate is valid
      keys[(half * ntile_all + tile) * 32 + hl] = u;
      atomicAdd(&myhist[u >> 8], 1u);
    } else {
      keys[(half * ntile_all + tile) * 32 + hl] = valid ? u : (uint16_t)0;
      if (valid) atomicAdd(&myhist[u >> 8], 1u);
    }
  };
  for (int tile0 = 0; tile0 < ntile; tile0 += 3) {
    step(std::integral_constant<int, 0>{}, tile0);
    if (tile0 + 1 < ntile) step(std::integral_constant<int, 1>{}, tile0 + 1);
    if (tile0 + 2 < ntile) step(std::integral_constant<int, 2>{}, tile0 + 2);
  }
  if constexpr (kDump) {  // score dump only: fill the never-valid tail with -inf
    if (t < p.S)
      for (int c = 32 * ntile + hl; c < p.T; c += 32)
        p.scores[((int64_t)b * p.S + t) * p.T + c] = (uint16_t)0xff80u;
    return;
  }
  lds_fence();

  // The picks of the select go to ring slots no wave reads any more: every wave
  // has passed the barrier of the last tile, so only the last tile's slot may
  // still be read; the other two held tiles whose reads and copies are done
  // (256 E bytes per wave; E = 8 takes both slots).
  constexpr int kWavesPerSlot = (16 / E) < 4 ? (16 / E) : 4;
  const int sslot = (((ntile > 0 ? ntile - 1 : 0) + 1 + wi / kWavesPerSlot) % 3);
  uint32_t* mysbuf = reinterpret_cast<uint32_t*>(ring + 4096 * sslot + (wi % kWavesPerSlot) * (256 * E)) +
                     KP * half;

  // The reference ranks all T candidates; masked ones carry -inf (order key
  // 0x007f). Their count is known, so they enter the histograms analytically.
  constexpr uint32_t kNegInfKey = 0x007fu;
  const uint32_t K = (uint32_t)p.K;
  const uint32_t nmask = (t < p.S) ? (uint32_t)(p.T - nv) : 0u;
  if (hl == 0 && nmask > 0) atomicAdd(&myhist[kNegInfKey >> 8], nmask);
  lds_fence();

  // Radix select of the K-th largest key: two 8-bit passes.
  uint32_t gt1 = 0, gt2 = 0;
  const int b1 = find_bin(myhist, lane, K, gt1);
  lds_fence();
  *reinterpret_cast<u32x4*>(myhist + 8 * hl) = u32x4{0u, 0u, 0u, 0u};
  *reinterpret_cast<u32x4*>(myhist + 8 * hl + 4) = u32x4{0u, 0u, 0u, 0u};
  lds_fence();
  // Four tiles' keys are read before their atomics so the LDS reads overlap (reads
  // past the last tile stay inside the workgroup's LDS and are not used).
  for (int tile0 = 0; tile0 < ntile; tile0 += 4) {
    uint32_t u4[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) u4[j] = keys[(half * ntile_all + tile0 + j) * 32 + hl];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = 32 * (tile0 + j) + hl;
      if (c < nv && (int)(u4[j] >> 8) == b1) atomicAdd(&myhist[u4[j] & 255u], 1u);
    }
  }
  if (hl == 0 && nmask > 0 && b1 == (int)(kNegInfKey >> 8)) atomicAdd(&myhist[kNegInfKey & 255u], nmask);
  lds_fence();
  const int b0 = find_bin(myhist, lane, K - gt1, gt2);
  const bool real = (t < p.S) && b1 >= 0 && b0 >= 0;
  const uint32_t V = real ? (((uint32_t)b1 << 8) | (uint32_t)b0) : 0x10000u;  // 0x10000: nothing matches
  const uint32_t n_gt = real ? gt1 + gt2 : 0u;   // picks strictly above the k-th key
  const uint32_t need_eq = real ? K - n_gt : 0u; // picks equal to it, lowest index first

  // Gather the K picks in torch's order: [keys > V in index order] then
  // [keys == V in index order], masked -inf candidates counting as index >= nv.
  // E > 1: entry = (key << 16) | ~index, later sorted as a whole (stable order).
  // E = 1: entry = (float-order key << 16) | valid << 15 | index, in gather order.
  auto entry = [&](uint32_t u, uint32_t c) -> uint32_t {
    if (E == 1) {
      const uint32_t fk = (u == 0x7fffu) ? 0x8000u : u;  // -0 == +0 for the comparator
      return (fk << 16) | 0x8000u | c;
    }
    return (u << 16) | (0xffffu - c);
  };
  // One token at a time over all 64 lanes (64 candidates a step), so the ranks come
  // straight from the 64-bit ballots: mbcnt gives the lanes below, and the running
  // counts stay wave-uniform.
  uint32_t* const sbuf0 = mysbuf - KP * half;  // the wave's pick buffers, token t0 first
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t Vh = (uint32_t)__builtin_amdgcn_readlane((int)V, 32 * h);
    const uint32_t ngt = (uint32_t)__builtin_amdgcn_readlane((int)n_gt, 32 * h);
    const uint32_t need = (uint32_t)__builtin_amdgcn_readlane((int)need_eq, 32 * h);
    const int nvh = __builtin_amdgcn_readlane(nv, 32 * h);
    const uint16_t* kh = keys + h * ntile_all * 32;
    uint32_t* sb = sbuf0 + KP * h;
    uint32_t gt_run = 0, eq_run = 0;
    for (int c0 = 0; c0 < nvh; c0 += 64) {
      const int c = c0 + lane;
      const bool valid = c < nvh;
      const uint32_t u = valid ? (uint32_t)kh[c] : 0u;
      const bool gt = valid && u > Vh;
      // Lane masks straight from the compares (a ballot of a combined condition is
      // rebuilt from a 0/1 vector value first).
      const uint64_t vb = __builtin_amdgcn_sicmp(c, nvh, 40);           // c < nvh (signed)
      const uint64_t gb = __builtin_amdgcn_uicmp(u, Vh, 34) & vb;       // u > Vh
      if (gt) {
        const uint32_t pos = __builtin_amdgcn_mbcnt_hi((uint32_t)(gb >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)gb, gt_run));
        if (pos < (uint32_t)KP) sb[pos] = entry(u, (uint32_t)c);
      }
      gt_run += (uint32_t)__builtin_popcountll(gb);
      const bool eq = valid && u == Vh;
      const uint64_t eb = __builtin_amdgcn_uicmp(u, Vh, 32) & vb;       // u == Vh
      if (eb != 0) {  // ties with the k-th key are rare: skip the step otherwise
        if (eq) {
          const uint32_t er = __builtin_amdgcn_mbcnt_hi((uint32_t)(eb >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)eb, eq_run));
          const uint32_t pos = ngt + er;
          if (er < need && pos < (uint32_t)KP) sb[pos] = entry(u, (uint32_t)c);
        }
        eq_run += (uint32_t)__builtin_popcountll(eb);
      }
    }
    const uint32_t eq_taken = eq_run < need ? eq_run : need;
    if (Vh == kNegInfKey) {
      // the remaining ties are masked candidates nv, nv+1, ...
      for (uint32_t j = (uint32_t)lane; j < need - eq_taken; j += 64) {
        const uint32_t pos = ngt + eq_taken + j;
        if (pos < (uint32_t)KP) sb[pos] = entry(kNegInfKey, (uint32_t)nvh + j);
      }
    }
  }
  const uint32_t nsel = real ? K : 0u;
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const uint32_t e = (uint32_t)(hl * E + i);
    if (e >= nsel) mysbuf[e] = 0u;  // E > 1: sorts last; E = 1: invalid slot
  }
  lds_fence();

  uint32_t sv[E];
#pragma unroll
  for (int i = 0; i < E; ++i) sv[i] = mysbuf[hl * E + i];

  if (E > 1) {
    // k > 32: torch sorts the gathered picks stably by value, i.e. value
    // descending then index ascending = descending order of the entries (all
    // distinct but for the zero fill, so any correct sort gives the same order).
    // Bitonic sort (descending) of KP entries, E per lane, element e = hl*E + i.
    // A compare-exchange is one med3 against a per-lane bound (all ones keeps the
    // larger entry, zero the smaller); lanes exchange through DPP or ds_swizzle.
#pragma unroll
    for (int k = 2; k <= KP; k <<= 1) {
#pragma unroll
      for (int j = k >> 1; j > 0; j >>= 1) {
        if (j >= E) {
          // (e & j) and (e & k) only depend on hl here (j, k >= E and E a power of 2).
          const int lj = j / E;
          const bool lower = (hl & lj) == 0;
          const bool desc = (hl & (k / E)) == 0;
          const uint32_t bound = (lower == desc) ? 0xffffffffu : 0u;
#pragma unroll
          for (int i = 0; i < E; ++i) sv[i] = med3_u32(sv[i], xor_lanes(sv[i], lj), bound);
        } else {
#pragma unroll
          for (int i = 0; i < E; ++i) {
            if ((i & j) == 0) {
              const uint32_t x = sv[i], y = sv[i + j];
              if (k < E) {  // direction fixed by i
                const bool desc = (i & k) == 0;
                sv[i] = desc ? max(x, y) : min(x, y);
                sv[i + j] = desc ? min(x, y) : max(x, y);
              } else {
                const uint32_t bound = (hl & (k / E)) == 0 ? 0xffffffffu : 0u;
                sv[i] = med3_u32(x, y, bound);
                sv[i + j] = med3_u32(x, y, ~bound);
              }
            }
          }
        }
      }
    }
  } else {
    // k <= 32: torch's 32-slot bitonic network on the gathered list. A slot pair
    // (lower A, upper B) at stride st belongs to comparator thread
    // tid = lower slot with bit st removed; stages of size 2..16 use the direction
    // flag (tid & size/2) != 0, the final merge uses false. The pair exchanges when
    // ((A > B and A valid) or B invalid) == flag, which also moves equal values.
    uint32_t x = sv[0];
    auto stage = [&](int size, int st, bool final_merge) {
      const uint32_t o = (uint32_t)__shfl_xor((int)x, st, 64);
      const bool lower = (hl & st) == 0;
      const uint32_t A = lower ? x : o, B = lower ? o : x;
      const int lo = lower ? hl : (hl ^ st);
      const int tid = ((lo >> 1) & ~(st - 1)) | (lo & (st - 1));
      const bool flag = final_merge ? false : ((tid & (size >> 1)) != 0);
      const bool va = (A >> 15) & 1u, vb = (B >> 15) & 1u;
      const bool sw = (((A >> 16) > (B >> 16)) && va) || !vb;
      if (sw == flag) x = lower ? B : A;
    };
#pragma unroll
    for (int size = 2; size < 32; size <<= 1)
#pragma unroll
      for (int st = size >> 1; st > 0; st >>= 1) stage(size, st, false);
#pragma unroll
    for (int st = 16; st > 0; st >>= 1) stage(32, st, true);
    sv[0] = x;
  }

  if (t < p.S) {
    int64_t* dst = p.out + ((int64_t)b * p.S + t) * p.K;
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const uint32_t e = (uint32_t)(hl * E + i);
      if (e < K) {
        const uint32_t c = (E == 1) ? (sv[i] & 0x7fffu) : (0xffffu - (sv[i] & 0xffffu));
        dst[e] = (p.causal && c >= (uint32_t)nv) ? (int64_t)-1 : (int64_t)c + p.offset;
      }
    }
  }
}

}  // namespace

extern "C" int dsa_indexer_rope(void* q, const void* freqs_cis, int64_t b, int64_t s, int64_t h,
                                int64_t d, int64_t rd, int32_t rope_mode, void* stream) {
  if (b < 0 || s < 0 || h <= 0 || d <= 0 || rd <= 0 || rd > d || (rd & 1) || (d & 1))
    return DSA_ERR_SHAPE;
  if (rope_mode != DSA_ROPE_CPU && rope_mode != DSA_ROPE_TORCH_ROCM) return DSA_ERR_UNSUPPORTED;
  if (b * s * h * d > (INT64_C(1) << 40)) return DSA_ERR_SHAPE;
  if (b == 0 || s == 0) return DSA_OK;
  if (!q || !freqs_cis) return DSA_ERR_NULL;
  if (((uintptr_t)q & 3u) || ((uintptr_t)freqs_cis & 7u)) return DSA_ERR_ALIGN;
  RopeParams p;
  p.q = (uint16_t*)q;
  p.freqs = (const float*)freqs_cis;
  p.rows = b * s * h;
  p.S = (int32_t)s;
  p.H = (int32_t)h;
  p.D = (int32_t)d;
  p.rd = (int32_t)rd;
  p.mode = rope_mode;
  const int64_t n = p.rows * (rd / 2);
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(rope_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, p);
  return hipGetLastError() == hipSuccess ? DSA_OK : DSA_ERR_LAUNCH;
}

int64_t dsa_indexer_wide_workspace_bytes(int64_t b, int64_t s, int64_t n_cand);
int dsa_indexer_wide_launch(const void* q, const void* kv_cache, int64_t kv_batch_stride,
                            const void* wl, float w_scale, const void* freqs_cis,
                            int32_t rope_mode, int64_t* out, uint16_t* scores, int64_t b,
                            int64_t s, int64_t rd, int64_t n_cand, int64_t k_out,
                            int64_t ratio, int32_t causal, int64_t offset, void* workspace,
                            int64_t workspace_bytes, hipStream_t stream);

namespace {

int launch_ix(const void* q, const void* kv_cache, int64_t kv_batch_stride, const void* wl,
              float w_scale, const void* freqs_cis, int32_t rope_mode, int64_t* out,
              uint16_t* scores, int64_t b, int64_t s, int64_t h, int64_t d, int64_t rd,
              int64_t n_cand, int64_t k_out, int64_t ratio, int32_t causal, int64_t offset,
              void* workspace, int64_t workspace_bytes, void* stream) {
  if (b < 0 || s < 0 || h <= 0 || d <= 0 || n_cand < 1 || k_out < 1 || ratio < 1)
    return DSA_ERR_SHAPE;
  if (k_out > n_cand) return DSA_ERR_SHAPE;
  const bool wide = (h == 64 && d == 128);
  if (!wide && (h != kH || d != kD)) return DSA_ERR_UNSUPPORTED;
  if (!wide && (n_cand > 2048 || k_out > 256)) return DSA_ERR_UNSUPPORTED;
  if (freqs_cis != nullptr) {
    if (rd <= 0 || rd > d || (rd & 1)) return DSA_ERR_SHAPE;
    if (rope_mode != DSA_ROPE_CPU && rope_mode != DSA_ROPE_TORCH_ROCM) return DSA_ERR_UNSUPPORTED;
  }
  if (kv_batch_stride < n_cand * d) return DSA_ERR_SHAPE;
  if (b > (1 << 20) || s > (1 << 24)) return DSA_ERR_SHAPE;
  if (b == 0 || s == 0) return DSA_OK;
  if (!q || !kv_cache || !wl || (!out && !scores)) return DSA_ERR_NULL;
  if (!dsa_host::aligned16(q) || !dsa_host::aligned16(kv_cache) || !dsa_host::aligned16(wl) ||
      ((uintptr_t)out & 7u) || ((uintptr_t)scores & 1u) || (kv_batch_stride % 8) != 0 ||
      (freqs_cis != nullptr && ((uintptr_t)freqs_cis & 7u)))
    return DSA_ERR_ALIGN;

  if (workspace_bytes < 0) return DSA_ERR_SHAPE;
  if (wide)
    return dsa_indexer_wide_launch(q, kv_cache, kv_batch_stride, wl, w_scale, freqs_cis, rope_mode,
                                   out, scores, b, s, rd, n_cand, k_out, ratio, causal, offset,
                                   workspace, workspace_bytes, (hipStream_t)stream);

  IxParams p;
  p.q = (const uint16_t*)q;
  p.kv = (const uint16_t*)kv_cache;
  p.kvbs = kv_batch_stride;
  p.wl = (const uint16_t*)wl;
  p.wscale = w_scale;
  p.freqs = (const float*)freqs_cis;
  p.rope_mode = rope_mode;
  p.out = out;
  p.scores = scores;
  p.B = (int32_t)b;
  p.S = (int32_t)s;
  p.rd = (int32_t)rd;
  p.T = (int32_t)n_cand;
  p.K = (int32_t)k_out;
  p.ratio = (int32_t)(ratio > (1 << 30) ? (1 << 30) : ratio);
  p.causal = causal ? 1 : 0;
  p.offset = offset;
  p.npairs = (int32_t)((s + 1) / 2);
  const int ntile = (int)((n_cand + 31) / 32);
  p.keys_bytes = ntile * 128;  // 2 halves x 32 lanes x uint16 per tile
  int E = 1;
  while (32 * E < k_out) E <<= 1;
  // Per wave: its key rows and two 256-bin histograms; then the 3-slot tile ring,
  // which also holds the picks after the tile loop (256 E bytes per wave). At
  // configs[2] (T 650, k 128) this is 31,232 bytes: five workgroups per CU.
  p.wave_bytes = p.keys_bytes + 2048;
  const size_t smem = (size_t)p.wave_bytes * 4 + 3 * 4096;
  if (smem > 64 * 1024) return DSA_ERR_UNSUPPORTED;
  const int64_t blocks = (int64_t)b * ((p.npairs + 3) / 4);  // 4 token pairs of one batch each
  if (blocks > INT32_MAX) return DSA_ERR_SHAPE;
  hipStream_t st = (hipStream_t)stream;
  if (scores != nullptr) {  // score stage: out == nullptr, k == 1
    if (out != nullptr || E != 1) return DSA_ERR_UNSUPPORTED;
    hipLaunchKernelGGL((ix_score_topk_kernel<1, true>), dim3((unsigned)blocks), dim3(256), smem, st, p);
    return hipGetLastError() == hipSuccess ? DSA_OK : DSA_ERR_LAUNCH;
  }
  switch (E) {
    case 1: hipLaunchKernelGGL((ix_score_topk_kernel<1, false>), dim3((unsigned)blocks), dim3(256), smem, st, p); break;
    case 2: hipLaunchKernelGGL((ix_score_topk_kernel<2, false>), dim3((unsigned)blocks), dim3(256), smem, st, p); break;
    case 4: hipLaunchKernelGGL((ix_score_topk_kernel<4, false>), dim3((unsigned)blocks), dim3(256), smem, st, p); break;
    case 8: hipLaunchKernelGGL((ix_score_topk_kernel<8, false>), dim3((unsigned)blocks), dim3(256), smem, st, p); break;
    default: return DSA_ERR_UNSUPPORTED;
  }
  return hipGetLastError() == hipSuccess ? DSA_OK : DSA_ERR_LAUNCH;
}

}  // namespace

extern "C" int dsa_indexer_score_topk(const void* q, const void* kv_cache, int64_t kv_batch_stride,
                                      const void* wl, float w_scale, const void* freqs_cis,
                                      int32_t rope_mode, int64_t* out, int64_t b, int64_t s,
                                      int64_t h, int64_t d, int64_t rd, int64_t n_cand,
                                      int64_t k_out, int64_t ratio, int32_t causal,
                                      int64_t offset, void* stream) {
  if (out == nullptr && b > 0 && s > 0) return DSA_ERR_NULL;
  return launch_ix(q, kv_cache, kv_batch_stride, wl, w_scale, freqs_cis, rope_mode, out, nullptr,
                   b, s, h, d, rd, n_cand, k_out, ratio, causal, offset, nullptr, 0, stream);
}

extern "C" int64_t dsa_indexer_workspace_bytes(int64_t b, int64_t s, int64_t h, int64_t d,
                                               int64_t n_cand) {
  if (b < 0 || s < 0 || n_cand < 0 || b > (1 << 20) || s > (1 << 24) || n_cand > (1 << 24))
    return DSA_ERR_SHAPE;
  if (h == 64 && d == 128) return dsa_indexer_wide_workspace_bytes(b, s, n_cand);
  return 0;
}

extern "C" int dsa_indexer_score_topk_ws(const void* q, const void* kv_cache, int64_t kv_batch_stride,
                                         const void* wl, float w_scale, const void* freqs_cis,
                                         int32_t rope_mode, int64_t* out, int64_t b, int64_t s,
                                         int64_t h, int64_t d, int64_t rd, int64_t n_cand,
                                         int64_t k_out, int64_t ratio, int32_t causal,
                                         int64_t offset, void* workspace, int64_t workspace_bytes,
                                         void* stream) {
  if (out == nullptr && b > 0 && s > 0) return DSA_ERR_NULL;
  return launch_ix(q, kv_cache, kv_batch_stride, wl, w_scale, freqs_cis, rope_mode, out, nullptr,
                   b, s, h, d, rd, n_cand, k_out, ratio, causal, offset, workspace, workspace_bytes,
                   stream);
}

namespace {

// Scratch of dsa_indexer_score_topk_noalloc: the 16-bit order keys of the 64-head
// path, one per (token, candidate), written by the score kernel and read by the
// select kernel (every key read was written by the same call). Each device that
// runs the library holds one copy of this array from module load until the
// process ends; its device address comes from hipGetSymbolAddress (the array's
// name in host code is not a device address).
constexpr int64_t kScratchBytes = DSA_INDEXER_NOALLOC_MAX_BYTES;
__device__ __align__(256) uint8_t scratch[kScratchBytes];

// Device address of `scratch` on the current device, looked up on the first call
// from each device and kept.
int scratch_address(void** out) {
  static std::atomic<void*> addr[dsa_host::kMaxDevices];
  static std::mutex mu;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= dsa_host::kMaxDevices)
    return DSA_ERR_DEVICE;
  void* ptr = addr[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    std::lock_guard<std::mutex> lock(mu);
    ptr = addr[dev].load(std::memory_order_relaxed);
    if (ptr == nullptr) {
      if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr)
        return DSA_ERR_DEVICE;
      addr[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return DSA_OK;
}

}  // namespace

extern "C" int dsa_indexer_score_topk_noalloc(const void* q, const void* kv_cache,
                                              int64_t kv_batch_stride, const void* wl,
                                              float w_scale, const void* freqs_cis,
                                              int32_t rope_mode, int64_t* out, int64_t b,
                                              int64_t s, int64_t h, int64_t d, int64_t rd,
                                              int64_t n_cand, int64_t k_out, int64_t ratio,
                                              int32_t causal, int64_t offset, void* stream) {
  if (out == nullptr && b > 0 && s > 0) return DSA_ERR_NULL;
  const int64_t need = dsa_indexer_workspace_bytes(b, s, h, d, n_cand);
  if (need < 0) return DSA_ERR_SHAPE;
  if (need > kScratchBytes) return DSA_ERR_SCRATCH;
  void* ws = nullptr;
  if (need > 0 && b > 0 && s > 0) {
    const int rc = scratch_address(&ws);
    if (rc != DSA_OK) return rc;
  }
  return launch_ix(q, kv_cache, kv_batch_stride, wl, w_scale, freqs_cis, rope_mode, out, nullptr,
                   b, s, h, d, rd, n_cand, k_out, ratio, causal, offset, ws, need, stream);
}

extern "C" int dsa_indexer_scores(const void* q, const void* kv_cache, int64_t kv_batch_stride,
                                  const void* wl, float w_scale, const void* freqs_cis,
                                  int32_t rope_mode, void* scores, int64_t b, int64_t s, int64_t h,
                                  int64_t d, int64_t rd, int64_t n_cand, int64_t ratio,
                                  int32_t causal, void* stream) {
  if (scores == nullptr && b > 0 && s > 0) return DSA_ERR_NULL;
  return launch_ix(q, kv_cache, kv_batch_stride, wl, w_scale, freqs_cis, rope_mode, nullptr,
                   (uint16_t*)scores, b, s, h, d, rd, n_cand, 1, ratio, causal, 0, nullptr, 0, stream);
}
