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
  const int64_t blocks = (m + kTM - 1) / kTM * (n / kTN);
  if (blocks > INT32_MAX) return DSA_ERR_SHAPE;
  const size_t smem = (size_t)kStages * kStageBytes;
  if (dsa_host::ensure_dyn_lds((const void*)ix_proj_kernel, (int)smem) != DSA_OK) return DSA_ERR_LAUNCH;
  hipLaunchKernelGGL(ix_proj_kernel, dim3((unsigned)blocks), dim3(256), smem, (hipStream_t)stream, p);
  return hipGetLastError() == hipSuccess ? DSA_OK : DSA_ERR_LAUNCH;
}
