// Task2 query projection with RoPE: q = qr . W^T (F.linear of the indexer's wq_b,
// reference/task2_v0_ref.py:129-130 through Linear.forward :81-83) followed by
// apply_rotary_emb on the last rd channels of every head (:131, :93-104).
//
// Rounding reproduced: F.linear of bf16 inputs on torch-ROCm accumulates in fp32
// over k in ascending order with matrix-core products and rounds once to bf16
// (measured at the indexer's shapes, see the equality tests); RoPE then works on
// the bf16 q, in torch-ROCm's rounding (rope_pair), and rounds to bf16 again.
//
// Workgroup = 4 waves, tile = 128 tokens x 256 output channels. K goes in chunks
// of 32 through a 3-stage LDS ring filled by buffer_load ... lds (the W rows of
// the tile and the qr rows of the tile, 24 KB per stage). A wave computes 64
// channels x 128 tokens as q^T = W . qr^T with mfma 32x32x16 (A = W rows, B =
// qr rows), so each lane ends up with 4 consecutive channels of one token per
// register group: the RoPE pairs are lane-local. The bf16 tile is transposed
// through LDS and written as whole 512-byte row segments.
#include "dsa_common.h"

using namespace dsa;

namespace {

constexpr int kTM = 128;                      // tokens per tile
constexpr int kTN = 256;                      // output channels per tile (4 waves x 64)
constexpr int kKC = 32;                       // k per stage
constexpr int kStages = 3;
constexpr int kWUnits = kTN * kKC * 2 / 1024;  // 16 copy units of 1 KB (W rows)
constexpr int kXUnits = kTM * kKC * 2 / 1024;  // 8 copy units (qr rows)
constexpr int kUnits = kWUnits + kXUnits;      // 24 per stage
constexpr int kUnitsW = kUnits / 4;            // 6 per wave
constexpr int kStageBytes = kUnits * 1024;     // 24 KB
constexpr uint32_t kOob = 0xfffffff0u;         // a copy offset beyond any resource: reads zeros

struct ProjParams {
  const uint16_t* x;    // [M, K] qr
  const uint16_t* w;    // [N, K] wq_b.weight
  uint16_t* q;          // [M, N]
  const float* freqs;   // [S, rd/2, 2] (row t = position start_pos + t) or nullptr
  int64_t M;
  int32_t N, K, D, H, rd, S, rope_mode;
};

// Position P (16-byte chunk) of a stage region holds row P/4, k chunk
// (P%4) ^ ((row/4)%4) of that row: a fragment read (32 rows, one k chunk) then
// touches 16 different chunk positions in every 256 bytes.
__device__ __forceinline__ int pos_of(int row, int c) { return row * 4 + (c ^ ((row >> 2) & 3)); }

__global__ __launch_bounds__(256) void ix_proj_kernel(ProjParams p) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wi = tid >> 6;
  const int wis = __builtin_amdgcn_readfirstlane(wi);
  const int ntn = p.N / kTN;
  const int64_t m0 = (int64_t)(blockIdx.x / ntn) * kTM;
  const int n0 = (int)(blockIdx.x % ntn) * kTN;
  const int nk = p.K / kKC;

  const i32x4 wrs = make_rsrc(p.w, (uint32_t)p.N * (uint32_t)p.K * 2u);
  const i32x4 xrs = make_rsrc(p.x, (uint32_t)(p.M * p.K * 2));
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;
  // Copy unit u of a stage: 64 chunk positions; wave wi moves units wi, wi+4, ...
  // Per unit and lane the source row / chunk are fixed; only k0 moves.
  uint32_t src_off[kUnitsW];
  bool from_w[kUnitsW];
#pragma unroll
  for (int i = 0; i < kUnitsW; ++i) {
    const int u = wis + 4 * i;
    const bool isw = u < kWUnits;
    const int P = 64 * (isw ? u : u - kWUnits) + lane;
    const int row = P >> 2;
    const int c = (P & 3) ^ ((row >> 2) & 3);
    from_w[i] = isw;
    if (isw) {
      src_off[i] = ((uint32_t)(n0 + row) * (uint32_t)p.K + 8u * (uint32_t)c) * 2u;
    } else {
      const int64_t m = m0 + row;
      src_off[i] = m < p.M ? (uint32_t)((m * p.K + 8 * c) * 2) : kOob;
    }
  }
  auto issue = [&](int kc) {
    const uint32_t base = lds0 + (uint32_t)(kc % kStages) * kStageBytes;
#pragma unroll
    for (int i = 0; i < kUnitsW; ++i) {
      const int u = wis + 4 * i;
      const uint32_t kb = (uint32_t)(kc * kKC) * 2u;
      const uint32_t off = src_off[i] == kOob ? kOob : src_off[i] + kb;
      lds_dma16(from_w[i] ? wrs : xrs, off, base + 1024u * (uint32_t)u);
    }
  };

  f32x16 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

  if (nk > 0) issue(0);
  if (nk > 1) issue(1);
  const int r32 = lane & 31, g = lane >> 5;
  for (int kc = 0; kc < nk; ++kc) {
    if (kc + 1 < nk) wait_vmcnt<kUnitsW>();
    else wait_vmcnt<0>();
    __syncthreads();  // chunk kc is in LDS; the stage of chunk kc - 1 is free
    if (kc + 2 < nk) issue(kc + 2);
    const u32x4* st = reinterpret_cast<const u32x4*>(smem + (kc % kStages) * kStageBytes);
    const u32x4* xs = st + kWUnits * 64;
#pragma unroll
    for (int ks = 0; ks < kKC / 16; ++ks) {
      const int c = 2 * ks + g;
      bf16x8 af[2], bf[4];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = __builtin_bit_cast(bf16x8, st[pos_of(64 * wi + 32 * i + r32, c)]);
#pragma unroll
      for (int j = 0; j < 4; ++j) bf[j] = __builtin_bit_cast(bf16x8, xs[pos_of(32 * j + r32, c)]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma32x32x16(af[i], bf[j], acc[i][j]);
    }
  }
  __syncthreads();  // the ring becomes the output staging area

  // Epilogue. acc[i][j] register r of lane (r32, g): token 32j + r32 of the tile,
  // channel 64wi + 32i + 8(r/4) + 4g + r%4 of the tile. Register group q4 of tile i
  // holds the channel pairs (c0, c0+1), (c0+2, c0+3) with c0 = 64wi + 32i + 8q4 + 4g;
  // whether they are rotated is the same for the whole group ((D - rd) % 8 == 0), and
  // their two table entries are one 16-byte load.
  const int half_rd = p.rd >> 1;
  const int head = (n0 + 64 * wi) / p.D;  // the wave's 64 channels lie in one head
  uint8_t* ob = smem;  // [128 tokens][256 channels] bf16, 16-byte chunk c of row t at t*512 + (c ^ (t%32))*16
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int tt = 32 * j + r32;
    const int64_t m = m0 + tt;
    const bool mok = m < p.M;
    const int tpos = (int)(m % p.S);
    const int64_t nbase = (m * p.H + head) * half_rd;  // flat complex index of pair 0
    float4 cs[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d0 = (n0 + 64 * wi + 32 * i + 8 * q4 + 4 * g) % p.D;
        cs[i][q4] = float4{1.f, 0.f, 1.f, 0.f};
        if (p.freqs != nullptr && d0 >= p.D - p.rd && mok) {
          const int pj = (d0 - (p.D - p.rd)) >> 1;
          cs[i][q4] = *reinterpret_cast<const float4*>(p.freqs + ((int64_t)tpos * half_rd + pj) * 2);
        }
      }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d0 = (n0 + 64 * wi + 32 * i + 8 * q4 + 4 * g) % p.D;
        const bool rot = p.freqs != nullptr && d0 >= p.D - p.rd && mok;
        const int pj = (d0 - (p.D - p.rd)) >> 1;
        uint32_t wv[2];
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          const int r = 4 * q4 + 2 * h2;
          uint32_t u = pack_bf2(acc[i][j][r], acc[i][j][r + 1]);
          if (rot) {
            float re, im;
            const float c = h2 ? cs[i][q4].z : cs[i][q4].x;
            const float sn = h2 ? cs[i][q4].w : cs[i][q4].y;
            rope_pair(bf_lo(u), bf_hi(u), c, sn, p.rope_mode, nbase + pj + h2, re, im);
            u = pack_bf2(re, im);
          }
          wv[h2] = u;
        }
        const int cidx = 8 * wi + 4 * i + q4;  // 16-byte chunk of the row (8 channels); g picks the half
        *reinterpret_cast<uint2*>(ob + tt * 512 + ((cidx ^ (tt & 31)) * 16) + 8 * g) = uint2{wv[0], wv[1]};
      }
    }
  }
  __syncthreads();
  // Rows: thread tid stores chunk tid%32 of rows tid/32 + 8k.
  const int cc = tid & 31;
#pragma unroll 4
  for (int rr = tid >> 5; rr < kTM; rr += 8) {
    const int64_t m = m0 + rr;
    if (m < p.M) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(ob + rr * 512 + ((cc ^ (rr & 31)) * 16));
      *reinterpret_cast<u32x4*>(p.q + m * p.N + n0 + 8 * cc) = v;
    }
  }
}

// ---------------------------------------------------------------------------
// k = 256 (the configs[2] wq_b): W-stationary persistent kernel.
//
// With k = 256 a wave's share of W (64 channels x 256 k, 32 KB) fits in 128
// VGPRs as the A operand of all 16 k-steps, so W is read from L2 once per wave
// and only the token side streams. Workgroup = 4 waves = 256 channels; two
// workgroups per CU. A workgroup walks a contiguous run of 32-token tiles: each
// tile's qr rows (16 KB) and, with RoPE, the tile's table rows (32 x rd/2
// complex) are copied by buffer_load ... lds into a 3-slot ring two tiles ahead;
// a wave computes q^T[64 ch x 32 tok] with 2 x 16 mfma 32x32x16 (k ascending, as
// the streaming kernel above), rounds, rotates, and writes its 32 x 128-byte row
// pieces through a wave-private LDS transpose with buffer stores (rows past M
// are dropped by the range check, so every wave issues the same number of
// vector-memory operations per tile, which the explicit waits count).
// The workgroups that share a token run (one per 256-channel group) are given
// ids on the same XCD, so the run's qr rows come from HBM once.

constexpr int kSK = 256;                       // k of this kernel
constexpr int kSTok = 32;                      // tokens per tile
constexpr int kSCh = 256;                      // channels per workgroup
constexpr int kSRing = 3;
constexpr int kSXUnits = kSTok * kSK * 2 / 1024;  // 16 copy units of 1 KB (qr rows)
constexpr int kSStoresW = 4;                   // 16-byte stores per lane and tile
constexpr int kSStageBytes = 4 * kSTok * 128;  // per-wave 32 x 128 B output staging

// s_waitcnt lgkmcnt(0), other counters untouched.
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

template <int RD>
struct SCfg {
  static constexpr int kFUnits = kSTok * RD * 4 / 1024;  // table rows: 32 x rd/2 x 8 B
  static constexpr int kUnits = kSXUnits + kFUnits;
  static constexpr int kUnitsW = kUnits / 4;             // copies per wave and tile
  static constexpr int kSlotBytes = kUnits * 1024;
  static constexpr int kLds = kSRing * kSlotBytes + kSStageBytes;
  static_assert(kUnits % 4 == 0, "copy units split evenly over the 4 waves");
};

struct SProjParams {
  const uint16_t* x;    // [M, 256] qr
  const uint16_t* w;    // [N, 256]
  uint16_t* q;          // [M, N]
  const float* freqs;   // [S, rd/2, 2]
  int32_t M, N, D, H, S;
  int32_t ngroups;      // N / 256
  int32_t nstreams;     // token runs; grid = ngroups * nstreams
  int32_t ntiles;       // ceil(M / 32)
  int32_t xcd_map;      // grid is a multiple of 8 * ngroups
  int32_t tail16;       // q_role part 2 takes the last tail16 / 16 of each run's tiles
};

// rope_pair with the mode fixed at compile time and torch-ROCm's unroll-slot
// choice made by selects instead of a branch (the same operations and roundings).
template <int RM>
__device__ __forceinline__ void rope_pair_sel(float a, float b, float c, float d, uint32_t n, float& re,
                                              float& im) {
  if constexpr (RM == DSA_ROPE_CPU) {
    re = __fsub_rn(__fmul_rn(a, c), __fmul_rn(b, d));
    im = __fadd_rn(__fmul_rn(a, d), __fmul_rn(b, c));
  } else {
    const bool s3 = ((n >> 7) & 3u) == 3u;
    const float ac = __fmul_rn(a, c), bd = __fmul_rn(b, d), ad = __fmul_rn(a, d), bc = __fmul_rn(b, c);
    re = s3 ? __fmaf_rn(-b, d, ac) : __fmaf_rn(a, c, -bd);
    im = s3 ? __fadd_rn(ad, bc) : __fmaf_rn(b, c, ad);
  }
}

// Token run and channel group of q-role block `blk`: the workgroups of one run get ids
// on one XCD when the run count is a multiple of 8 (p.xcd_map).
__device__ __forceinline__ void q_run(const SProjParams& p, int blk, int& cg, int& t0, int& t1) {
  int st;
  if (p.xcd_map) {
    const int j = blk >> 3;
    cg = j % p.ngroups;
    st = (j / p.ngroups) * 8 + (blk & 7);
  } else {
    cg = blk % p.ngroups;
    st = blk / p.ngroups;
  }
  t0 = (int)((int64_t)st * p.ntiles / p.nstreams);
  t1 = (int)((int64_t)(st + 1) * p.ntiles / p.nstreams);
}

// Copies of a 32-token tile into a ring slot by buffer_load ... lds. Copy unit u of a
// slot covers 64 16-byte positions. qr region: position P holds row P/32, chunk
// (P%32) ^ (row%16) (16 lanes reading one k chunk of 16 rows hit 16 different bank
// groups; k-steps ks and ks + 8 are 256 bytes apart). Table region: position P holds
// row P/(RD/4), chunk (P%(RD/4)) ^ (row % (RD/4)) of that token's RD*4-byte table row.
// Each wave moves units wi, wi + 4, ...: with RD = 32 its last unit (16 + wi) is table
// rows. Tiles must be issued in order (the table position follows them).
template <int RD>
struct QTileCopier {
  static constexpr int kXW = kSXUnits / 4;   // qr units per wave
  static constexpr int kCpr = RD > 0 ? RD / 4 : 1;  // 16-byte chunks per table row
  i32x4 xrs, frs;
  uint32_t lds0;
  int M, S, wis;
  int frow, fpos;  // table unit: tile row, and its position (m % S)
  uint32_t fcol;

  __device__ __forceinline__ void init(const SProjParams& p, uint8_t* smem, int wis_, int lane, int t0) {
    xrs = make_rsrc(p.x, (uint32_t)p.M * (uint32_t)(kSK * 2));
    frs = make_rsrc(p.freqs, RD > 0 ? (uint32_t)p.S * (uint32_t)(RD * 4) : 0u);
    lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;
    M = p.M;
    S = p.S;
    wis = wis_;
    frow = 0;
    fpos = 0;
    fcol = 0;
    if constexpr (RD > 0) {
      static_assert(SCfg<RD>::kFUnits == 4, "one table unit per wave");
      const int P = 64 * wis + lane;
      frow = P / kCpr;
      fcol = 16u * (uint32_t)((P % kCpr) ^ (frow % kCpr));
      fpos = (int)((uint32_t)(t0 * kSTok + frow) % (uint32_t)S);
    }
  }
  // The per-lane source offsets are recomputed at each issue from an opaque copy of the
  // lane id: held across the tile loop they would take registers the products need.
  __device__ __forceinline__ void issue(int t, int slot) {
    const uint32_t base = lds0 + (uint32_t)slot * SCfg<RD>::kSlotBytes;
    const int lim = M - t * kSTok;  // rows of the tile below M
    const uint32_t mb = (uint32_t)(t * kSTok) * (uint32_t)(kSK * 2);
    int ln = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    asm volatile("" : "+v"(ln));
#pragma unroll
    for (int i = 0; i < kXW; ++i) {
      const int P = 64 * (wis + 4 * i) + ln;
      const int row = P >> 5;
      const uint32_t off = (uint32_t)row * (uint32_t)(kSK * 2) + 16u * (uint32_t)((P & 31) ^ (row & 15));
      lds_dma16(xrs, row < lim ? mb + off : kOob, base + 1024u * (uint32_t)(wis + 4 * i));
    }
    if constexpr (RD > 0) {
      lds_dma16(frs, frow < lim ? (uint32_t)fpos * (uint32_t)(RD * 4) + fcol : kOob,
                base + 1024u * (uint32_t)(kSXUnits + wis));
      fpos += kSTok;
      if (fpos >= S) {
        fpos -= S;
        if (fpos >= S) fpos = (int)((uint32_t)fpos % (uint32_t)S);
      }
    }
  }
};

// The q tiles of q-role block `blk`. kPacked: W comes as fragments pre-packed by
// dsa_indexer_pack_projection_weights (wave slice r = n / 64, tile i, k-step ks, lane:
// 16 B), loaded straight into registers with 1 KB coalesced loads after the first two
// tiles' copies are issued; otherwise W is staged through LDS from its [N, 256] rows.
// part: 0 = every tile of the block's token run, 1 = all but its tail, 2 = the tail only
// (tail16 / 16 of the run's tiles).
template <int RD, int RM, bool kPacked>
__device__ __forceinline__ void q_role(const SProjParams& p, int blk, uint8_t* smem, int part) {
  using C = SCfg<RD>;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wi = tid >> 6;
  const int wis = __builtin_amdgcn_readfirstlane(wi);
  const int r32 = lane & 31, g = lane >> 5;
  int cg, t0, t1;
  q_run(p, blk, cg, t0, t1);
  if (part != 0) {
    const int tail = ((t1 - t0) * p.tail16) >> 4;
    if (part == 1)
      t1 -= tail;
    else
      t0 = t1 - tail;
  }
  const int n0 = cg * kSCh;
  const __amdgpu_buffer_rsrc_t qrs = buf_rsrc(p.q, (uint32_t)p.M * (uint32_t)p.N * 2u);
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;

  // This wave's W in MFMA A-operand layout: wf[i][ks] of lane (r32, g) holds row
  // n0 + 64 wi + 32 i + r32, k 16 ks + 8 g .. + 7. Loaded straight from global
  // memory every instruction would touch 32 rows (32 cache lines); instead each
  // wave copies its 32 rows of tile i (16 KB, contiguous in W) into LDS with 1 KB
  // copies, position P holding row P/32, chunk (P%32) ^ (row%16), and reads the
  // fragments from there (two passes through the first 64 KB of LDS).
  bf16x8 wf[2][16];
  if constexpr (!kPacked) {
    static_assert(4 * 16 * 1024 <= C::kLds, "W staging fits the workgroup's LDS");
    const i32x4 wrs = make_rsrc(p.w, (uint32_t)p.N * (uint32_t)(kSK * 2));
    const uint32_t wbase = lds0 + (uint32_t)wis * 16384u;
    const u32x4* wl = reinterpret_cast<const u32x4*>(smem + wi * 16384);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t rbase = (uint32_t)(n0 + 64 * wis + 32 * i) * (uint32_t)(kSK * 2);
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int P = 64 * u + lane, row = P >> 5;
        lds_dma16(wrs, rbase + (uint32_t)row * (uint32_t)(kSK * 2) + 16u * (uint32_t)((P & 31) ^ (row & 15)),
                  wbase + 1024u * (uint32_t)u);
      }
      wait_vmcnt<0>();
      __syncthreads();
#pragma unroll
      for (int ks = 0; ks < 16; ++ks) wf[i][ks] = __builtin_bit_cast(bf16x8, wl[r32 * 32 + ((2 * ks + g) ^ (r32 & 15))]);
      wait_lgkmcnt0();  // the reads are done before the region is copied over again
      __syncthreads();
    }
  }
  if (t0 >= t1) return;  // (workgroup-uniform)

  QTileCopier<RD> cp;
  cp.init(p, smem, wis, lane, t0);
  cp.issue(t0, 0);
  if (t0 + 1 < t1) cp.issue(t0 + 1, 1);
  constexpr int kWLoads = 32;  // packed W: 1 KB loads per wave, counted by the first tile's wait
  if constexpr (kPacked) {
    const u32x4* wsrc = reinterpret_cast<const u32x4*>(p.w) + (size_t)((n0 >> 6) + wis) * (2 * 16 * 64);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int ks = 0; ks < 16; ++ks) wf[i][ks] = __builtin_bit_cast(bf16x8, wsrc[(i * 16 + ks) * 64 + lane]);
  }
  uint8_t* wst = smem + kSRing * C::kSlotBytes + wi * (kSTok * 128);  // this wave's staging
  const int D = p.D;
  // With rd = 32 at most one of the wave's two 32-channel tiles is rotated (the last 32
  // channels of a head): irot, or -1. hd: the head of the wave's 64 channels.
  int irot = -1;
  if constexpr (RD > 0) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
      if ((n0 + 64 * wis + 32 * i) % D >= D - RD) irot = i;
  }
  const uint32_t hd = (uint32_t)((n0 + 64 * wis) / D);
  for (int t = t0; t < t1; ++t) {
    const int it = t - t0;
    // Operations issued after this tile's copies: the stores of tile t - 2 (when
    // it >= 2; waiting for them too is harmless), the copies of tile t + 1 and the
    // stores of tile t - 1; at the first tile with packed W the copies of tile t0 + 1
    // and the 32 W loads (which tile t0's products wait for, so they are done later).
    if (t + 1 < t1) {
      if (it >= 1) wait_vmcnt<C::kUnitsW + kSStoresW>();
      else if (kPacked) wait_vmcnt<C::kUnitsW + kWLoads>();
      else wait_vmcnt<C::kUnitsW>();
    } else {
      if (it >= 1) wait_vmcnt<kSStoresW>();
      else if (kPacked) wait_vmcnt<kWLoads>();
      else wait_vmcnt<0>();
    }
    __syncthreads();  // tile t is in LDS; every wave is done with the slot of tile t - 1
    if (t + 2 < t1) cp.issue(t + 2, (it + 2) % kSRing);
    const uint8_t* slot = smem + (it % kSRing) * C::kSlotBytes;
    const u32x4* xs = reinterpret_cast<const u32x4*>(slot);

    // B fragments are read kPre k-steps ahead of their products (one LDS read per
    // two MFMAs in the issue order, pinned below; fewer with the RoPE epilogue's
    // registers).
    constexpr int kPre = RD > 0 ? 4 : 8;
    f32x16 acc0 = f32x16{}, acc1 = f32x16{};
    bf16x8 bq[16];
#pragma unroll
    for (int ks = 0; ks < kPre; ++ks) bq[ks] = __builtin_bit_cast(bf16x8, xs[r32 * 32 + ((2 * ks + g) ^ (r32 & 15))]);
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) {
      if (ks + kPre < 16)
        bq[ks + kPre] = __builtin_bit_cast(bf16x8, xs[r32 * 32 + ((2 * (ks + kPre) + g) ^ (r32 & 15))]);
      acc0 = mfma32x32x16(wf[0][ks], bq[ks], acc0);
      acc1 = mfma32x32x16(wf[1][ks], bq[ks], acc1);
    }
#pragma unroll
    for (int ks = 0; ks < kPre; ++ks) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) {
      if (ks + kPre < 16) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);                      // 2 MFMA
    }

    // Epilogue: lane (r32, g), register r of tile i is channel
    // n0 + 64 wi + 32 i + 8 (r/4) + 4 g + r%4 of token m0 + r32. The rotated tile's
    // four table entries (complex pairs 4 q4 + 2 g, + 1 of the token) are read together,
    // while the last products finish.
    const int m = t * kSTok + r32;
    float4 cs[4];
    if constexpr (RD > 0) {
      constexpr int kCpr = RD / 4;
      const uint8_t* fr = slot + kSXUnits * 1024;
      if (irot >= 0) {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const int pj = 4 * q4 + 2 * g;
          cs[q4] = *reinterpret_cast<const float4*>(fr + (r32 * kCpr + ((pj >> 1) ^ (r32 % kCpr))) * 16);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const f32x16& a = i ? acc1 : acc0;
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        uint32_t u0 = pack_bf2(a[4 * q4], a[4 * q4 + 1]);
        uint32_t u1 = pack_bf2(a[4 * q4 + 2], a[4 * q4 + 3]);
        if constexpr (RD > 0) {
          if (i == irot) {
            const int pj = 4 * q4 + 2 * g;  // complex index of (u0); (u1) is pj + 1
            // Only (n / 128) % 4 of the flat complex index n matters: 32-bit wrap is exact.
            const uint32_t nb = ((uint32_t)m * (uint32_t)p.H + hd) * (uint32_t)(RD / 2) + (uint32_t)pj;
            float re, im;
            rope_pair_sel<RM>(bf_lo(u0), bf_hi(u0), cs[q4].x, cs[q4].y, nb, re, im);
            u0 = pack_bf2(re, im);
            rope_pair_sel<RM>(bf_lo(u1), bf_hi(u1), cs[q4].z, cs[q4].w, nb + 1, re, im);
            u1 = pack_bf2(re, im);
          }
        }
        const int ck = 4 * i + q4;  // 16-byte chunk of the wave's 128-byte row piece
        *reinterpret_cast<uint2*>(wst + r32 * 128 + ((ck ^ (r32 & 7)) * 16) + 8 * g) = uint2{u0, u1};
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int k = 0; k < kSStoresW; ++k) {
      const int row = 8 * k + (lane >> 3), ch = lane & 7;
      const u32x4 v = *reinterpret_cast<const u32x4*>(wst + row * 128 + ((ch ^ (row & 7)) * 16));
      const uint32_t mm = (uint32_t)(t * kSTok + row);
      // Rows at or past M are beyond the resource and dropped.
      const uint32_t off = mm < (uint32_t)p.M ? (mm * (uint32_t)p.N + (uint32_t)(n0 + 64 * wis + 8 * ch)) * 2u
                                              : 0xfffffff0u;
      __builtin_amdgcn_raw_buffer_store_b128(v, qrs, (int)off, 0, 0);
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
  }
}

template <int RD, int RM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void ix_proj_k256_kernel(
    SProjParams p) {
  extern __shared__ __align__(16) uint8_t smem[];
  q_role<RD, RM, false>(p, blockIdx.x, smem, 0);
}

// ---------------------------------------------------------------------------
// Both projections of the indexer in one launch: q = RoPE(qr . wq_b^T) and the head
// weights wl = x . weights_proj^T (reference/task2_v0_ref.py:129-132). The Ascend
// submission overlaps them by running weights_proj on a second stream beside the
// query path (src/task2_indexer.py:805-839, go_c2_ovl); here the overlap happens
// inside one grid with no stream or event calls: workgroups of the q role (q_role on
// packed W) and workgroups of the w role (w_role) share the CUs, the first mostly
// matrix-core and LDS work, the second a stream of x from HBM.

constexpr int kWDim = 1024;           // x row length (the model dim) of the w role
constexpr int kWHeads = 16;           // weights_proj outputs
constexpr int kWSteps = kWDim / 32;   // 16x16x32 k-steps per chain
constexpr int kWTok = 16;             // tokens per chain
constexpr uint32_t kWChainBytes = kWTok * kWDim * 2;

struct WProjParams {
  const uint16_t* x;  // [M, 1024]
  const u32x4* wp;    // packed weights_proj fragments [32 k-steps][64 lanes]
  uint16_t* wl;       // [M, 16]
  int32_t M;
  int32_t nwaves;     // waves of the w role in the grid
};

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// wl for chains of 16 tokens: acc = W (16 heads x 32 k, A operand) . x^T (32 k x 16
// tokens, B operand) over the k-steps 0..31 in order, one accumulator per chain, rounded
// once to bf16: the natural k order, which is F.linear's on torch-ROCm where hipBLASLt
// runs a kernel without split-k for this shape. W's fragments sit in LDS (32 KB); all 32
// x fragments of the next chain (16 B per lane and k-step) are in flight while the
// current chain's products run. Rows at or past M read as zero and are not stored.
__device__ __forceinline__ void w_role(const WProjParams& p, int wblk, uint8_t* smem) {
  const int tid = threadIdx.x, lane = tid & 63, wi = tid >> 6;
  u32x4* wls = reinterpret_cast<u32x4*>(smem);
#pragma unroll
  for (int i = 0; i < kWSteps * 64 / 256; ++i) wls[tid + 256 * i] = p.wp[tid + 256 * i];
  __syncthreads();
  const int gw = wblk * 4 + wi;
  const int nch = (p.M + kWTok - 1) / kWTok;
  const int c0 = (int)((int64_t)gw * nch / p.nwaves);
  const int c1 = (int)((int64_t)(gw + 1) * nch / p.nwaves);
  if (c0 >= c1) return;
  const __amdgpu_buffer_rsrc_t xr = buf_rsrc(p.x, (uint32_t)p.M * (uint32_t)(kWDim * 2));
  const __amdgpu_buffer_rsrc_t orr = buf_rsrc(p.wl, (uint32_t)p.M * (uint32_t)(kWHeads * 2));
  const uint32_t lo = (uint32_t)(lane & 15) * (uint32_t)(kWDim * 2) + (uint32_t)(lane >> 4) * 16u;
  u32x4 xf[kWSteps];
  {
    const uint32_t b0 = (uint32_t)c0 * kWChainBytes + lo;
#pragma unroll
    for (int ks = 0; ks < kWSteps; ++ks) xf[ks] = __builtin_amdgcn_raw_buffer_load_b128(xr, (int)(b0 + 64u * ks), 0, 0);
  }
  for (int c = c0; c < c1; ++c) {
    const bool more = c + 1 < c1;
    const uint32_t nb = (uint32_t)(c + 1) * kWChainBytes + lo;
    // W fragments are read kWPre k-steps ahead of their products; the issue order (LDS
    // read, product, next chain's load) is pinned so that only a few W fragments are
    // live beside the 32 x fragments.
    constexpr int kWPre = 4;
    f32x4 acc = f32x4{};
    bf16x8 wa[kWSteps];
#pragma unroll
    for (int ks = 0; ks < kWPre; ++ks) wa[ks] = __builtin_bit_cast(bf16x8, wls[ks * 64 + lane]);
#pragma unroll
    for (int ks = 0; ks < kWSteps; ++ks) {
      if (ks + kWPre < kWSteps) wa[ks + kWPre] = __builtin_bit_cast(bf16x8, wls[(ks + kWPre) * 64 + lane]);
      acc = mfma16x16x32(wa[ks], __builtin_bit_cast(bf16x8, xf[ks]), acc);
      // The next chain's fragment ks (beyond the resource, i.e. no memory access, after the last chain).
      xf[ks] = __builtin_amdgcn_raw_buffer_load_b128(xr, more ? (int)(nb + 64u * ks) : (int)0xfffffff0u, 0, 0);
    }
#pragma unroll
    for (int ks = 0; ks < kWPre; ++ks) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
#pragma unroll
    for (int ks = 0; ks < kWSteps; ++ks) {
      if (ks + kWPre < kWSteps) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                            // MFMA
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                            // VMEM read
    }
    // Lane (n = lane % 16, g = lane / 16) holds heads 4g .. 4g + 3 of token 16c + n.
    const uint32_t t = (uint32_t)c * kWTok + (uint32_t)(lane & 15);
    const uint32_t off = t < (uint32_t)p.M ? t * (uint32_t)(kWHeads * 2) + (uint32_t)(lane >> 4) * 8u : 0xfffffff0u;
    __builtin_amdgcn_raw_buffer_store_b64(u32x2{pack_bf2(acc[0], acc[1]), pack_bf2(acc[2], acc[3])}, orr, (int)off,
                                          0, 0);
  }
}

struct Proj2Params {
  SProjParams q;
  WProjParams w;
  int32_t nq;     // blocks [0, nq) run the q role; blocks [nq, 2 nq) the w role
  int32_t wtail;  // w-role block j then takes the tail of q-role block j's token run
};

// The q-role blocks come first in the grid: they are dispatched first (one per CU), and
// their W loads reach the memory system ahead of the w role's stream of x (dispatched
// the other way round the q role's first tile came ~5 us later). Each w-role block,
// once its chains are done, computes the last tail16/16 of the q tiles of the run with
// its own index (on the same XCD), so that both roles end together.
template <int RD, int RM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void ix_proj2_kernel(Proj2Params p) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int b = blockIdx.x;
  if (b < p.nq) {
    q_role<RD, RM, true>(p.q, b, smem, p.wtail ? 1 : 0);
  } else {
    w_role(p.w, b - p.nq, smem);
    if (p.wtail) {
      __syncthreads();  // the w role's LDS (W fragments) becomes the q role's ring
      q_role<RD, RM, true>(p.q, b - p.nq, smem, 2);
    }
  }
}

// q-role plan: ngroups channel groups of 256, `blocks_target` workgroups in all; the
// workgroups of one token run get ids on one XCD (ids i, i + 8, ... when the run count
// is a multiple of 8).
void plan_q(SProjParams& p, int64_t M, int32_t N, int blocks_target) {
  p.M = (int32_t)M;
  p.N = N;
  p.ngroups = N / kSCh;
  p.ntiles = (int32_t)((M + kSTok - 1) / kSTok);
  int streams = blocks_target / p.ngroups;
  if (streams < 1) streams = 1;
  if (streams >= 8) streams -= streams % 8;
  if (streams > p.ntiles) streams = p.ntiles;
  p.nstreams = streams;
  p.xcd_map = streams % 8 == 0 ? 1 : 0;
}

template <int RD, int RM>
int launch_k256(const ProjParams& a, void* stream) {
  using C = SCfg<RD>;
  int cus = 0;
  if (dsa_host::device_cu_count(&cus) != DSA_OK) return DSA_ERR_DEVICE;
  SProjParams p;
  p.x = a.x;
  p.w = a.w;
  p.q = a.q;
  p.freqs = a.freqs;
  p.D = a.D;
  p.H = a.H;
  p.S = a.S;
  p.tail16 = 0;
  // Two workgroups per CU; the token runs of one XCD's workgroups share qr tiles.
  plan_q(p, a.M, a.N, 2 * cus);
  const int64_t blocks = (int64_t)p.nstreams * p.ngroups;
  void (*fn)(SProjParams) = ix_proj_k256_kernel<RD, RM>;
  if (dsa_host::ensure_dyn_lds((const void*)fn, C::kLds) != DSA_OK) return DSA_ERR_LAUNCH;
  hipLaunchKernelGGL(fn, dim3((unsigned)blocks), dim3(256), (size_t)C::kLds,
                     (hipStream_t)stream, p);
  return hipGetLastError() == hipSuccess ? DSA_OK : DSA_ERR_LAUNCH;
}

// Combined launch: q-role workgroups per CU (as many w-role ones), and the share of
// each token run's q tiles (in sixteenths) that the paired w-role workgroup takes.
constexpr int kProj2QPerCu = 1;
constexpr int kProj2Tail16 = 4;

template <int RD, int RM>
int launch_proj2(SProjParams q, WProjParams w, void* stream) {
  using C = SCfg<RD>;
  int cus = 0;
  if (dsa_host::device_cu_count(&cus) != DSA_OK) return DSA_ERR_DEVICE;
  plan_q(q, q.M, q.N, kProj2QPerCu * cus);
  q.tail16 = kProj2Tail16;
  const int64_t qblocks = (int64_t)q.nstreams * q.ngroups;
  // One w-role block per q-role block (block nq + j runs on the XCD of block j when nq
  // is a multiple of 8, as it is whenever the q role's XCD map is on).
  const int64_t wblocks = qblocks;
  w.nwaves = (int32_t)(4 * wblocks);
  Proj2Params p;
  p.q = q;
  p.w = w;
  p.nq = (int32_t)qblocks;
  p.wtail = kProj2Tail16 > 0 ? 1 : 0;
  void (*fn)(Proj2Params) = ix_proj2_kernel<RD, RM>;
  if (dsa_host::ensure_dyn_lds((const void*)fn, C::kLds) != DSA_OK) return DSA_ERR_LAUNCH;
  hipLaunchKernelGGL(fn, dim3((unsigned)(qblocks + wblocks)), dim3(256), (size_t)C::kLds, (hipStream_t)stream, p);
  return hipGetLastError() == hipSuccess ? DSA_OK : DSA_ERR_LAUNCH;
}

// Fragment packing of the projection weights, one thread per 16-byte fragment.
//  wq [n, 256]:        fragment f = ((r * 2 + i) * 16 + ks) * 64 + lane holds
//                      wq[64 r + 32 i + lane % 32][16 ks + 8 (lane / 32) .. + 7]
//  wproj [n_w, dim]:   fragment e = (hg * (dim / 32) + ks) * 64 + lane holds
//                      wproj[16 hg + lane % 16][32 ks + 8 (lane / 16) .. + 7]
__global__ __launch_bounds__(256) void ix_pack_kernel(const uint16_t* wq, int64_t nq_frag, u32x4* wq_packed,
                                                      const uint16_t* wp, int64_t nw_frag, int32_t dim,
                                                      u32x4* wp_packed) {
  const int64_t f = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (f < nq_frag) {
    const int lane = (int)(f & 63), ks = (int)((f >> 6) & 15), i = (int)((f >> 10) & 1);
    const int64_t row = 64 * (f >> 11) + 32 * i + (lane & 31);
    wq_packed[f] = *reinterpret_cast<const u32x4*>(wq + row * kSK + 16 * ks + 8 * (lane >> 5));
  } else if (f < nq_frag + nw_frag) {
    const int64_t e = f - nq_frag;
    const int lane = (int)(e & 63);
    const int steps = dim / 32;
    const int ks = (int)((e >> 6) % steps);
    const int64_t row = 16 * ((e >> 6) / steps) + (lane & 15);
    wp_packed[e] = *reinterpret_cast<const u32x4*>(wp + row * dim + 32 * ks + 8 * (lane >> 4));
  }
}

}  // namespace

extern "C" int dsa_indexer_q_proj(const void* qr, const void* wq, const void* freqs_cis,
                                  int32_t rope_mode, void* q, int64_t m, int64_t n, int64_t k,
                                  int64_t head_dim, int64_t rd, int64_t s_len, void* stream) {
  if (m < 0 || n <= 0 || k <= 0 || head_dim <= 0 || s_len <= 0) return DSA_ERR_SHAPE;
  if (n % head_dim != 0) return DSA_ERR_SHAPE;
  if (freqs_cis != nullptr) {
    if (rd <= 0 || rd > head_dim || (rd & 1)) return DSA_ERR_SHAPE;
    if (rope_mode != DSA_ROPE_CPU && rope_mode != DSA_ROPE_TORCH_ROCM) return DSA_ERR_UNSUPPORTED;
    // Rotated channels start on an 8-channel boundary (whole register groups).
    if ((head_dim - rd) % 8 != 0) return DSA_ERR_UNSUPPORTED;
  }
  if (k % kKC != 0 || n % kTN != 0 || (head_dim != 64 && head_dim != 128)) return DSA_ERR_UNSUPPORTED;
  // Buffer offsets are 32-bit byte counts.
  if (m * k * 2 > (int64_t)UINT32_MAX - 4096 || n * k * 2 > (int64_t)UINT32_MAX) return DSA_ERR_UNSUPPORTED;
  if (m % s_len != 0) return DSA_ERR_SHAPE;  // tokens are [b, s_len] rows
  if (m == 0) return DSA_OK;
  if (!qr || !wq || !q) return DSA_ERR_NULL;
  if (!dsa_host::aligned16(qr) || !dsa_host::aligned16(wq) || !dsa_host::aligned16(q) ||
      (freqs_cis != nullptr && ((uintptr_t)freqs_cis & 15u)))
    return DSA_ERR_ALIGN;
  ProjParams p;
  p.x = (const uint16_t*)qr;
  p.w = (const uint16_t*)wq;
  p.q = (uint16_t*)q;
  p.freqs = (const float*)freqs_cis;
  p.M = m;
  p.N = (int32_t)n;
  p.K = (int32_t)k;
  p.D = (int32_t)head_dim;
  p.H = (int32_t)(n / head_dim);
  p.rd = (int32_t)rd;
  p.S = (int32_t)s_len;
  p.rope_mode = rope_mode;
  // k = 256 with a table of at most 32 rotated channels per head: W-stationary kernel.
  if (k == kSK && m <= INT32_MAX / 2 && m * n <= (int64_t)UINT32_MAX / 2) {
    if (freqs_cis == nullptr) return launch_k256<0, 0>(p, stream);
    if (rd == 32)
      return rope_mode == DSA_ROPE_CPU ? launch_k256<32, DSA_ROPE_CPU>(p, stream)
                                       : launch_k256<32, DSA_ROPE_TORCH_ROCM>(p, stream);
  }
  const int64_t blocks = (m + kTM - 1) / kTM * (n / kTN);
  if (blocks > INT32_MAX) return DSA_ERR_SHAPE;
  const size_t smem = (size_t)kStages * kStageBytes;
  if (dsa_host::ensure_dyn_lds((const void*)ix_proj_kernel, (int)smem) != DSA_OK) return DSA_ERR_LAUNCH;
  hipLaunchKernelGGL(ix_proj_kernel, dim3((unsigned)blocks), dim3(256), smem, (hipStream_t)stream, p);
  return hipGetLastError() == hipSuccess ? DSA_OK : DSA_ERR_LAUNCH;
}

extern "C" int dsa_indexer_pack_projection_weights(const void* wq, int64_t n, int64_t k, const void* wproj,
                                                   int64_t n_w, int64_t dim, void* wq_packed,
                                                   void* wproj_packed, void* stream) {
  int64_t nq_frag = 0, nw_frag = 0;
  if (wq != nullptr || wq_packed != nullptr) {
    if (!wq || !wq_packed) return DSA_ERR_NULL;
    if (n <= 0 || k <= 0) return DSA_ERR_SHAPE;
    if (k != kSK || n % 64 != 0) return DSA_ERR_UNSUPPORTED;
    if (!dsa_host::aligned16(wq) || !dsa_host::aligned16(wq_packed)) return DSA_ERR_ALIGN;
    nq_frag = n * k / 8;
  }
  if (wproj != nullptr || wproj_packed != nullptr) {
    if (!wproj || !wproj_packed) return DSA_ERR_NULL;
    if (n_w <= 0 || dim <= 0) return DSA_ERR_SHAPE;
    if (n_w % 16 != 0 || dim % 32 != 0 || dim > (1 << 20)) return DSA_ERR_UNSUPPORTED;
    if (!dsa_host::aligned16(wproj) || !dsa_host::aligned16(wproj_packed)) return DSA_ERR_ALIGN;
    nw_frag = n_w * dim / 8;
  }
  const int64_t total = nq_frag + nw_frag;
  if (total == 0) return DSA_OK;
  if ((total + 255) / 256 > INT32_MAX) return DSA_ERR_SHAPE;
  hipLaunchKernelGGL(ix_pack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)wq, nq_frag, (u32x4*)wq_packed, (const uint16_t*)wproj, nw_frag,
                     (int32_t)dim, (u32x4*)wproj_packed);
  return hipGetLastError() == hipSuccess ? DSA_OK : DSA_ERR_LAUNCH;
}

extern "C" int dsa_indexer_projections(const void* qr, const void* wq_packed, const void* freqs_cis,
                                       int32_t rope_mode, void* q, const void* x, const void* wproj_packed,
                                       void* wl, int64_t m, int64_t n, int64_t k, int64_t dim, int64_t n_w,
                                       int64_t head_dim, int64_t rd, int64_t s_len, void* stream) {
  if (m < 0 || n <= 0 || k <= 0 || dim <= 0 || n_w <= 0 || head_dim <= 0 || s_len <= 0) return DSA_ERR_SHAPE;
  if (n % head_dim != 0 || m % s_len != 0) return DSA_ERR_SHAPE;
  if (k != kSK || n % kSCh != 0 || head_dim != 64 || dim != kWDim || n_w != kWHeads)
    return DSA_ERR_UNSUPPORTED;
  if (freqs_cis != nullptr) {
    if (rd <= 0 || rd > head_dim || (rd & 1)) return DSA_ERR_SHAPE;
    if (rope_mode != DSA_ROPE_CPU && rope_mode != DSA_ROPE_TORCH_ROCM) return DSA_ERR_UNSUPPORTED;
    if (rd != 32) return DSA_ERR_UNSUPPORTED;
  }
  // Buffer offsets are 32-bit byte counts.
  // (The w role's padding rows of the last chain read up to one chain past m * dim * 2.)
  if (m > INT32_MAX / 2 || m * n > (int64_t)UINT32_MAX / 2 || m * dim * 2 > (int64_t)UINT32_MAX - 2 * kWChainBytes)
    return DSA_ERR_UNSUPPORTED;
  if (m == 0) return DSA_OK;
  if (!qr || !wq_packed || !q || !x || !wproj_packed || !wl) return DSA_ERR_NULL;
  if (!dsa_host::aligned16(qr) || !dsa_host::aligned16(wq_packed) || !dsa_host::aligned16(q) ||
      !dsa_host::aligned16(x) || !dsa_host::aligned16(wproj_packed) || ((uintptr_t)wl & 7u) ||
      (freqs_cis != nullptr && ((uintptr_t)freqs_cis & 15u)))
    return DSA_ERR_ALIGN;
  SProjParams qp;
  qp.x = (const uint16_t*)qr;
  qp.w = (const uint16_t*)wq_packed;
  qp.q = (uint16_t*)q;
  qp.freqs = (const float*)freqs_cis;
  qp.M = (int32_t)m;
  qp.N = (int32_t)n;
  qp.D = (int32_t)head_dim;
  qp.H = (int32_t)(n / head_dim);
  qp.S = (int32_t)s_len;
  qp.tail16 = 0;
  WProjParams wp;
  wp.x = (const uint16_t*)x;
  wp.wp = (const u32x4*)wproj_packed;
  wp.wl = (uint16_t*)wl;
  wp.M = (int32_t)m;
  wp.nwaves = 0;
  if (freqs_cis == nullptr) return launch_proj2<0, 0>(qp, wp, stream);
  return rope_mode == DSA_ROPE_CPU ? launch_proj2<32, DSA_ROPE_CPU>(qp, wp, stream)
                                   : launch_proj2<32, DSA_ROPE_TORCH_ROCM>(qp, wp, stream);
}
