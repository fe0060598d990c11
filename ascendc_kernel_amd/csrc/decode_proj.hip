// Task2 decode projections: q = qr . wq_b^T and wl = x . weights_proj^T for a few
// tokens (1..16) in one launch, at the DeepSeek-V3.2 indexer shapes (q_lora_rank
// 1536, dim 7168). These are the two F.linear calls of the indexer's forward,
// reference/task2_v0_ref.py:129 (q) and :132 (weights), through Linear.forward
// :81-83; RoPE stays with the score kernel as on the F.linear route.
//
// Rounding reproduced: torch-ROCm runs both products through hipBLASLt, which
// for 1..16 tokens at these shapes picks a kernel with a local split of the
// depth loop over 4 waves (macro tiles 32x16x128 for q and 16x16x512 for wl,
// one tile per workgroup). Measured with planted inputs and random data: in
// every depth block of D (128 for q, 512 for wl) wave c owns the c-th quarter,
// [it*D + c*D/4, it*D + (c+1)*D/4), and accumulates it in 16x16x32 bf16 matrix
// products in ascending k into one fp32 chain over all blocks; the four chains
// are then summed as ((c0 + c1) + c2) + c3 and rounded once to bf16 (RNE).
// This kernel evaluates exactly those chains and that sum, with a work split
// that keeps all of a workgroup's weight bytes in flight at once (one workgroup
// per CU, up to 256 VGPRs a lane, no workgroup waits for another):
//
//  * q (25 MB of weights): a workgroup covers 64 output channels (4 row groups
//    of 16); wave w runs chain w%4 of two row groups, so it issues 24 weight
//    fragments and the 12 qr fragments both chains share before its first
//    product; the chains meet in LDS.
//  * wl (0.9 MB, 4 row groups of 16 channels): a workgroup per row group; its
//    8 waves issue the group's whole 229 KB of weight rows at once and stage
//    them, with the tokens' x rows, through LDS in 4 phases of 2048 k; waves
//    0..3 run the 4 chains from LDS.
//
// The wl workgroups come first in the grid, so they start before the q ones.
#include "dsa_common.h"

using namespace dsa;

namespace {

constexpr int kThreads = 512;                      // 8 waves, one workgroup per CU
constexpr int kSplit = 4;                          // chains per row group
constexpr int kQDepth = 128;                       // q depth block
constexpr int kQSteps = 12;                        // 1536 / 128 products per q chain
constexpr int kQK = kQSteps * kQDepth;             // 1536
constexpr int kQRows = 64;                         // q channels per workgroup
constexpr int kWDepth = 512;                       // wl depth block
constexpr int kWK = 7168;                          // wl depth
constexpr int kPhaseBlocks = 4;                    // depth blocks per LDS phase (2048 k)
constexpr int kPhases = 4;                         // 4 + 4 + 4 + 2 blocks
constexpr int kRowChunks = kPhaseBlocks * kWDepth * 2 / 16;  // 256 chunks of 16 B per row and phase
constexpr int kRowPitch = kRowChunks * 16 + 16;    // padded LDS row (4112 B)
constexpr int kTile = 16 * kRowPitch;              // 16 rows of one phase
constexpr int kPhaseLoads = 16 * kRowChunks / kThreads;  // 8 chunks per lane for a full phase
constexpr int kLdsBytes = 2 * kTile;               // W rows + x rows of one phase: 131,584 B
static_assert(kWK == (kPhases - 1) * kPhaseBlocks * kWDepth + 2 * kWDepth, "wl phases");

struct DecodeProjParams {
  const uint16_t* qr;   // [m, 1536]
  const uint16_t* wq;   // [n_q, 1536]
  const uint16_t* x;    // [m, 7168]
  const uint16_t* wp;   // [n_w, 7168]
  uint16_t* q;          // [m, n_q]
  uint16_t* wl;         // [m, n_w]
  int32_t m, n_q, n_w, wl_blocks;
};

__device__ __forceinline__ float add_rn(float a, float b) { return __fadd_rn(a, b); }

// Element t (0..255) of a 16-channel x 16-token tile whose four chains are f32x4
// lanes of red[w0 .. w0+3][64]: lane t/4, register t%4 -> token lane%16, channel
// 4*(lane/16) + t%4. Sums the chains in order and stores bf16 for tokens < m.
__device__ __forceinline__ void reduce_store(const f32x4* red, int w0, int t, int m, uint16_t* out,
                                             int n, int n0) {
  const int lane = t >> 2, r = t & 3;
  const float* f = reinterpret_cast<const float*>(red);
  const float s = add_rn(add_rn(add_rn(f[(w0 * 64 + lane) * 4 + r], f[((w0 + 1) * 64 + lane) * 4 + r]),
                                f[((w0 + 2) * 64 + lane) * 4 + r]),
                         f[((w0 + 3) * 64 + lane) * 4 + r]);
  const int col = lane & 15, row = 4 * (lane >> 4) + r;
  if (col < m) out[(int64_t)col * n + n0 + row] = f2bf(s);
}

__device__ void q_role(const DecodeProjParams& p, int blk, uint8_t* smem) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = wave & 3, rp = wave >> 2;  // chain, pair of row groups (2 rp, 2 rp + 1)
  const int r16 = lane & 15, g = lane >> 4;
  const int nb = blk * kQRows + rp * 32;
  const int tok = min(r16, p.m - 1);  // columns >= m compute on a valid row and are not stored
  const int koff = c * (kQDepth / 4) + g * 8;
  const u32x4* wa0 = reinterpret_cast<const u32x4*>(p.wq + (int64_t)(nb + r16) * kQK + koff);
  const u32x4* wa1 = reinterpret_cast<const u32x4*>(p.wq + (int64_t)(nb + 16 + r16) * kQK + koff);
  const u32x4* xb = reinterpret_cast<const u32x4*>(p.qr + (int64_t)tok * kQK + koff);
  u32x4 a0[kQSteps], a1[kQSteps], b[kQSteps];
#pragma unroll
  for (int s = 0; s < kQSteps; ++s) {
    b[s] = xb[s * (kQDepth / 8)];
    a0[s] = ld_nt(wa0 + s * (kQDepth / 8));
    a1[s] = ld_nt(wa1 + s * (kQDepth / 8));
  }
  // All 36 loads in flight before the first product (the scheduler would otherwise
  // interleave them with the chains and keep fewer outstanding).
  __builtin_amdgcn_sched_barrier(0);
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < kQSteps; ++s) {
    acc0 = mfma16x16x32(__builtin_bit_cast(bf16x8, a0[s]), __builtin_bit_cast(bf16x8, b[s]), acc0);
    acc1 = mfma16x16x32(__builtin_bit_cast(bf16x8, a1[s]), __builtin_bit_cast(bf16x8, b[s]), acc1);
  }
  // red[row group][chain][lane]: row group 2 rp + i of chain c
  f32x4* red = reinterpret_cast<f32x4*>(smem);
  red[((2 * rp) * 4 + c) * 64 + lane] = acc0;
  red[((2 * rp + 1) * 4 + c) * 64 + lane] = acc1;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int e = tid + i * kThreads;  // 4 row groups x 256 elements
    const int rgp = e >> 8;
    reduce_store(red, rgp * 4, e & 255, p.m, p.q, p.n_q, blk * kQRows + rgp * 16);
  }
}

// Phase ph covers NB depth blocks (NB * 512 k from k0 = 2048 ph): a row of it is
// NB * 64 chunks of 16 B. Chunk j (< 16 * NB * 64) is row j / (NB * 64) (channel
// n0 + row, or token row), chunk j % (NB * 64); lane tid takes j = tid + 512 i,
// i < 2 NB.
template <int NB>
__device__ __forceinline__ void load_w(u32x4 (&r)[2 * NB], const uint16_t* wp, int n0, int ph, int tid) {
  constexpr int kRow = NB * 64;
#pragma unroll
  for (int i = 0; i < 2 * NB; ++i) {
    const int j = tid + i * kThreads;
    r[i] = ld_nt(reinterpret_cast<const u32x4*>(wp + (int64_t)(n0 + j / kRow) * kWK + ph * 2048 + (j % kRow) * 8));
  }
}
template <int NB>
__device__ __forceinline__ void load_x(u32x4 (&r)[kPhaseLoads], const uint16_t* x, int m, int ph, int tid) {
  constexpr int kRow = NB * 64;
#pragma unroll
  for (int i = 0; i < 2 * NB; ++i) {
    const int j = tid + i * kThreads, row = j / kRow;
    if (row < m) r[i] = *reinterpret_cast<const u32x4*>(x + (int64_t)row * kWK + ph * 2048 + (j % kRow) * 8);
  }
}
// Write one phase to LDS (row pitch kRowPitch, chunk at 16 B * its index in the row),
// then (after the barrier) run chain c over its NB depth blocks.
template <int NB>
__device__ __forceinline__ void wl_phase(const u32x4 (&w)[2 * NB], const u32x4 (&xr)[kPhaseLoads], uint8_t* smem,
                                         int m, int tid, int wave, int lane, f32x4& acc) {
  constexpr int kRow = NB * 64;
  uint8_t* wt = smem;
  uint8_t* xt = smem + kTile;
#pragma unroll
  for (int i = 0; i < 2 * NB; ++i) {
    const int j = tid + i * kThreads, row = j / kRow;
    *reinterpret_cast<u32x4*>(wt + row * kRowPitch + (j % kRow) * 16) = w[i];
    if (row < m) *reinterpret_cast<u32x4*>(xt + row * kRowPitch + (j % kRow) * 16) = xr[i];
  }
  __syncthreads();
  if (wave < kSplit) {
    // Chain c = wave: k [blk*512 + c*128, +128) of each depth block of the phase,
    // four products of 32 in ascending k. Token rows >= m hold stale data: their
    // columns are not stored.
    // Step t (= 4 d + s) reads k = d * 512 + c * 128 + s * 32 of the phase; the
    // fragments of step t + 2 are read while step t's product runs.
    const int r16 = lane & 15, g = lane >> 4;
    const uint8_t* wa = wt + r16 * kRowPitch + (wave * (kWDepth / kSplit) + g * 8) * 2;
    const uint8_t* xa = xt + r16 * kRowPitch + (wave * (kWDepth / kSplit) + g * 8) * 2;
    constexpr int kSteps = 4 * NB;
    auto at = [](int t) { return (t >> 2) * kWDepth * 2 + (t & 3) * 64; };
    u32x4 fa[3], fb[3];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      fa[t] = *reinterpret_cast<const u32x4*>(wa + at(t));
      fb[t] = *reinterpret_cast<const u32x4*>(xa + at(t));
    }
#pragma unroll
    for (int t = 0; t < kSteps; ++t) {
      if (t + 2 < kSteps) {
        fa[(t + 2) % 3] = *reinterpret_cast<const u32x4*>(wa + at(t + 2));
        fb[(t + 2) % 3] = *reinterpret_cast<const u32x4*>(xa + at(t + 2));
      }
      __builtin_amdgcn_sched_barrier(0);  // keep the read-ahead ahead of the product
      acc = mfma16x16x32(__builtin_bit_cast(bf16x8, fa[t % 3]), __builtin_bit_cast(bf16x8, fb[t % 3]), acc);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

__device__ void wl_role(const DecodeProjParams& p, int blk, uint8_t* smem) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n0 = blk * 16;
  // The group's whole weight rows (28 chunks a lane) and the first two phases of x
  // are issued before anything waits; x of phases 2 and 3 reuses those registers.
  u32x4 w0[8], w1[8], w2[8], w3[4], xa[kPhaseLoads], xb[kPhaseLoads];
  load_x<4>(xa, p.x, p.m, 0, tid);
  load_w<4>(w0, p.wp, n0, 0, tid);
  load_x<4>(xb, p.x, p.m, 1, tid);
  load_w<4>(w1, p.wp, n0, 1, tid);
  load_w<4>(w2, p.wp, n0, 2, tid);
  load_w<2>(w3, p.wp, n0, 3, tid);
  __builtin_amdgcn_sched_barrier(0);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  wl_phase<4>(w0, xa, smem, p.m, tid, wave, lane, acc);
  load_x<4>(xa, p.x, p.m, 2, tid);
  __syncthreads();
  wl_phase<4>(w1, xb, smem, p.m, tid, wave, lane, acc);
  load_x<2>(xb, p.x, p.m, 3, tid);
  __syncthreads();
  wl_phase<4>(w2, xa, smem, p.m, tid, wave, lane, acc);
  __syncthreads();
  wl_phase<2>(w3, xb, smem, p.m, tid, wave, lane, acc);
  __syncthreads();  // the last phase's tiles are no longer read
  f32x4* red = reinterpret_cast<f32x4*>(smem);
  if (wave < kSplit) red[wave * 64 + lane] = acc;
  __syncthreads();
  if (tid < 256) reduce_store(red, 0, tid, p.m, p.wl, p.n_w, n0);
}

__global__ __launch_bounds__(kThreads) void ix_decode_proj_kernel(DecodeProjParams p) {
  __shared__ __align__(16) uint8_t smem[kLdsBytes];
  if ((int)blockIdx.x < p.wl_blocks) wl_role(p, blockIdx.x, smem);
  else q_role(p, blockIdx.x - p.wl_blocks, smem);
}

}  // namespace

extern "C" int dsa_indexer_decode_projections(const void* qr, const void* wq, const void* x, const void* wproj,
                                              void* q, void* wl, int64_t m, int64_t n_q, int64_t k_q,
                                              int64_t n_w, int64_t k_w, void* stream) {
  if (m < 0 || n_q <= 0 || k_q <= 0 || n_w <= 0 || k_w <= 0) return DSA_ERR_SHAPE;
  if (m > 16 || k_q != kQK || k_w != kWK || n_q % kQRows != 0 || n_w % 16 != 0 || n_q > (1 << 20) ||
      n_w > (1 << 16))
    return DSA_ERR_UNSUPPORTED;
  if (m == 0) return DSA_OK;
  if (!qr || !wq || !x || !wproj || !q || !wl) return DSA_ERR_NULL;
  if (!dsa_host::aligned16(qr) || !dsa_host::aligned16(wq) || !dsa_host::aligned16(x) ||
      !dsa_host::aligned16(wproj) || ((uintptr_t)q & 1u) || ((uintptr_t)wl & 1u))
    return DSA_ERR_ALIGN;
  DecodeProjParams p;
  p.qr = (const uint16_t*)qr;
  p.wq = (const uint16_t*)wq;
  p.x = (const uint16_t*)x;
  p.wp = (const uint16_t*)wproj;
  p.q = (uint16_t*)q;
  p.wl = (uint16_t*)wl;
  p.m = (int32_t)m;
  p.n_q = (int32_t)n_q;
  p.n_w = (int32_t)n_w;
  p.wl_blocks = (int32_t)(n_w / 16);
  const unsigned grid = (unsigned)(p.wl_blocks + n_q / kQRows);
  hipLaunchKernelGGL(ix_decode_proj_kernel, dim3(grid), dim3(kThreads), 0, (hipStream_t)stream, p);
  return hipGetLastError() == hipSuccess ? DSA_OK : DSA_ERR_LAUNCH;
}
