// Sparse MLA forward: the attention of the DSA layer. It is Task1's
// sparse attention (reference/task1_v0_ref.py:5-24: gather, fp32 scores with the
// sink in the softmax denominator, bf16 output) with one latent kv row serving as
// the key (its first d_qk = 576 channels) and as the value (its first d_v = 512
// channels): out[b,m,h,:] = sum_t softmax_t(scale * q . kv_t[:576]) kv_t[:512].
//
// One workgroup per token, one wave per 16 heads (8 waves for 128 heads). Per
// wave, Q^T (576 x 16 heads, 72 VGPRs) and O^T (512 x 16, fp32, 128 registers)
// stay in registers. Slots go in blocks of 32: the 32 selected rows (1152 B each)
// are copied by buffer_load ... lds into a ring of 4 LDS buffers, each row padded
// to 73 chunks of 16 B so that one chunk read across 16 rows, and the transposed
// reads of V, hit distinct banks. Per block and wave (mfma 16x16x32, lane l:
// head l%16, key / channel group g = l/16):
//   S^T[2 x 16 keys x 16 heads] = K . Q^T                  (2 x 18 mfma)
//   online softmax over the 32 keys of a head (held by the 4 lane groups, reduced
//   with permlane16/32 swaps), sink as the initial max, log2 domain
//   O^T[512 x 16] += V^T[512 x 32] . (P_hi + P_lo)^T         (32 x 2 mfma)
// with the contraction over keys ordered so that each lane's 8 P values are the B
// operand as they stand (keys 4g..4g+3 and 16+4g..16+4g+3 for lane group g).
// The two waves of a SIMD overlap one's softmax with the other's products.
#include "dsa_common.h"

#include <float.h>

using namespace dsa;

namespace {

constexpr int kDQK = 576;                       // key / query channels
constexpr int kDV = 512;                        // value channels
constexpr int kKS = kDQK / 32;                  // 18 k-steps of the score product
constexpr int kCT = kDV / 16;                   // 32 output tiles of 16 channels
constexpr int kKB = 32;                         // slots per block
constexpr int kRowC = kDQK / 8 + 1;             // LDS row: 72 chunks + 1 pad chunk
constexpr int kBlkPos = kKB * kRowC;            // 2336 chunk positions per block
constexpr int kUnitsBlk = (kBlkPos + 63) / 64;  // 37 copy units of 64 chunks
constexpr int kBlkBytes = kUnitsBlk * 1024;     // 37888 B per buffer (copy tail included)
constexpr int kRingM = 4;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRaise = 8.0f;
constexpr uint32_t kOob = 0xfffffff0u;          // a copy offset beyond any resource: reads zeros

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4* lds_s16x4_ptr;

struct MlaParams {
  const uint16_t* q;     // [B, M, H, 576]
  const uint16_t* kv;    // [B, NKV, kv_dim] (kv_dim >= 576 channels per row)
  const void* idx;       // [B, M, TOPK] int32 or int64 (the kernel's IdxT)
  const float* sink;     // [H]
  uint16_t* out;         // [B, M, H, 512]
  int64_t M;
  float* part;           // split mode: [B*M, nsplit, H/16 waves, 32 tiles, 64 lanes, 4] fp32 O^T ...
  float* ml;             // ... and [B*M, nsplit, H, 2] (running max, log2 domain; sum); else null
  int32_t nsplit;        // slot ranges per token (1: the whole slot list, bf16 output)
  int32_t bps;           // slot blocks per split
  int32_t hg;            // split mode: head groups per token (workgroups of 16 NW heads)
  int32_t B, H, NKV, TOPK, kv_dim;
  float scale_log2;
};

struct S2 {
  f32x4 t0, t1;
};

// kSplit: the token's slot blocks are divided among p.nsplit workgroups, each
// writing its unnormalised partial state to p.part / p.ml (a separate
// instantiation, so the one-pass kernel's code is unchanged by it).
template <int NW, typename IdxT, bool kSplit>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2)))
void sa_mla_kernel(MlaParams p) {
  const IdxT* const idx = static_cast<const IdxT*>(p.idx);
  extern __shared__ __align__(16) uint8_t smem[];
  uint8_t* ring = smem;                                                   // [kRingM][kBlkBytes]
  int32_t* slot = reinterpret_cast<int32_t*>(smem + kRingM * kBlkBytes);  // [nblk * 32]
  const int nblk = (p.TOPK + kKB - 1) / kKB;
  int32_t* nblk_sh = slot + nblk * kKB;  // [NW] blocks up to each wave's last valid slot
  // Split mode: workgroup (token, sp) takes slot blocks [kb0, kb0 + nbl) of the token;
  // `slot` and the block numbers kb below count from kb0.
  // Split mode: workgroup ((token * nsplit + sp) * hg + hgi) takes the 16 NW heads of
  // head group hgi.
  const int hgi = kSplit ? (int)(blockIdx.x % p.hg) : 0;
  const int64_t tsp = kSplit ? (int64_t)(blockIdx.x / p.hg) : 0;
  // One-pass mode takes the tokens last to first: with causal slot lists the late
  // tokens have the most blocks, so the short early tokens fill the end of the grid
  // (2-3 % at configs[4]).
  const int64_t tok = kSplit ? tsp / p.nsplit : (int64_t)(gridDim.x - 1 - blockIdx.x);
  const int sp = kSplit ? (int)(tsp % p.nsplit) : 0;
  const int kb0 = kSplit ? sp * p.bps : 0;
  const int nbl = kSplit ? max(0, min(p.bps, nblk - kb0)) : nblk;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wi = tid >> 6;
  const int b = (int)(tok / p.M);
  const int n = lane & 15;  // head 16wi + n
  const int g = lane >> 4;  // lane group: k-slice 8g..8g+7, C rows 4g..4g+3
  const int head = 16 * (NW * hgi + wi) + n;

  // The token's global reads (Q^T, the sink, the slot indices) are all issued
  // before any of them is waited for. Q^T fragments (B operand): head `head`,
  // channels 32ks + 8g .. +7; every head is valid (H % 16 == 0).
  bf16x8 qf[kKS];
  {
    const uint16_t* qrow = p.q + (tok * p.H + head) * kDQK + 8 * g;
#pragma unroll
    for (int ks = 0; ks < kKS; ++ks)
      qf[ks] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(qrow + 32 * ks));
  }
  const float sink_raw = p.sink[head];
  // Slot indices -> LDS, 8 per thread in flight at a time (loads unconditional,
  // clamped to the row, so that none sits in a branch).
  int last = 0;
  auto slot_chunk = [&](const int s0) {
    int v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int s = kb0 * kKB + s0 + 64 * NW * u + tid;
      v[u] = slot_index(idx, tok * p.TOPK + min(s, p.TOPK - 1));
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int s = s0 + 64 * NW * u + tid;
      if (s < nbl * kKB) {
        const int w = (kb0 * kKB + s < p.TOPK && v[u] < p.NKV) ? v[u] : -1;
        slot[s] = w;
        if (w >= 0) last = s / kKB + 1;
      }
    }
  };
  slot_chunk(0);
  for (int s0 = 8 * 64 * NW; s0 < nbl * kKB; s0 += 8 * 64 * NW) slot_chunk(s0);
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) last = max(last, __shfl_xor(last, m, 64));
  if (lane == 0) nblk_sh[wi] = last;
  __syncthreads();
  int nb = nblk_sh[0];
  for (int w = 1; w < NW; ++w) nb = max(nb, nblk_sh[w]);

  // Copies: unit u covers chunk positions 64u .. 64u+63 of a block buffer
  // (position P = row * 73 + chunk). Wave wi moves units wi, wi + NW, ...; every
  // wave issues kUnitsW copies (surplus ones repeat the last unit: same bytes).
  constexpr int kUnitsW = (kUnitsBlk + NW - 1) / NW;
  const int wis = __builtin_amdgcn_readfirstlane(wi);
  const i32x4 rsrc = make_rsrc(p.kv + (int64_t)b * p.NKV * p.kv_dim,
                               (uint32_t)p.NKV * (uint32_t)p.kv_dim * 2u);
  const uint32_t ring_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)ring;
  const uint32_t row_bytes = (uint32_t)p.kv_dim * 2u;
  // Copy offsets of block blk for this wave's units. They are recomputed from the
  // lane id at every use: an opaque copy of the id keeps the compiler from holding
  // ten per-lane values in registers across the block loop (which spilled them and
  // put a scratch reload, with its vmcnt(0) wait on the copies in flight, into the
  // loop).
  auto rows_of = [&](int blk, uint32_t (&rv)[kUnitsW]) {
    int ln = lane;
    asm volatile("" : "+v"(ln));
#pragma unroll
    for (int i = 0; i < kUnitsW; ++i) {
      int u = wis + NW * i;
      if (u >= kUnitsBlk) u = kUnitsBlk - 1;
      const int pos = 64 * u + ln;
      const int r = pos / kRowC;
      const int c = pos - r * kRowC;
      const int w = slot[blk * kKB + min(r, kKB - 1)];
      rv[i] = (r < kKB && w >= 0 && c < kRowC - 1) ? (uint32_t)w * row_bytes + 16u * (uint32_t)c : kOob;
    }
  };
  auto issue = [&](int blk, const uint32_t (&rv)[kUnitsW]) {
    const uint32_t base = ring_lds + (uint32_t)(blk % kRingM) * (uint32_t)kBlkBytes;
#pragma unroll
    for (int i = 0; i < kUnitsW; ++i) {
      int u = wis + NW * i;
      if (u >= kUnitsBlk) u = kUnitsBlk - 1;
      lds_dma16(rsrc, rv[i], base + 1024u * (uint32_t)u);
    }
  };

  f32x4 o[kCT];
#pragma unroll
  for (int ct = 0; ct < kCT; ++ct) o[ct] = f32x4{};
  const float sink_l2 = sink_raw * kLog2e;
  const float c2 = p.scale_log2;  // > 0 (checked by the host)
  // The running max starts at the sink, floored at -FLT_MAX: with a -inf sink and
  // a fully masked first block, exp2(s * c2 - m_run) is then exp2(-inf) = 0
  // instead of exp2(-inf + inf) = NaN.
  float m_run = fmaxf(sink_l2, -FLT_MAX);
  float l_run = 0.f;

  // S^T of the block in buffer kvl: tile kt has keys 16kt + (lane%16) as A rows,
  // channels 32ks + 8g; the lane's results are keys 16kt + 4g + r of head n.
  // Key tile 0 then key tile 1, one K fragment read ahead of its product (order
  // pinned below), so the LDS latency overlaps the matrix work.
  auto qk = [&](const uint8_t* kvl) {
    S2 acc = {f32x4{}, f32x4{}};
    const u32x4* r0 = reinterpret_cast<const u32x4*>(kvl) + n * kRowC + g;
    auto frag = [&](int i) {  // i = 18 kt + ks
      return __builtin_bit_cast(bf16x8, r0[(i >= kKS ? 16 * kRowC : 0) + 4 * (i % kKS)]);
    };
    bf16x8 a_cur = frag(0);
#pragma unroll
    for (int i = 0; i < 2 * kKS; ++i) {
      bf16x8 a_nxt = a_cur;
      if (i + 1 < 2 * kKS) a_nxt = frag(i + 1);
      if (i < kKS) acc.t0 = mfma16x16x32(a_cur, qf[i], acc.t0);
      else acc.t1 = mfma16x16x32(a_cur, qf[i - kKS], acc.t1);
      a_cur = a_nxt;
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
    for (int i = 0; i < 2 * kKS - 1; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    return acc;
  };

#pragma unroll
  for (int j = 0; j < kRingM - 1; ++j) {
    if (j < nb) {
      uint32_t rv[kUnitsW];
      rows_of(j, rv);
      issue(j, rv);
    }
  }
  int vslot = slot[lane & 31];
#pragma unroll
  for (int ks = 0; ks < kKS; ++ks) asm volatile("" ::"v"(qf[ks]));
  asm volatile("" ::"v"(m_run));

  // bf16 pairs (-1, 0), (0, -1) in SGPRs for the dot2 residuals (see the gather kernel).
  uint32_t neg_lo_bits = 0x0000bf80u, neg_hi_bits = 0xbf800000u;
  asm volatile("" : "+s"(neg_lo_bits), "+s"(neg_hi_bits));
  const bf16v2 neg_lo = __builtin_bit_cast(bf16v2, neg_lo_bits);
  const bf16v2 neg_hi = __builtin_bit_cast(bf16v2, neg_hi_bits);

  static_assert(kRingM == 4, "the waits assume a ring of 4 buffers");
  uint32_t vm_cur = 0u;
  // The waves of the second half (one of the two waves on each SIMD) meet the
  // block's barrier after their QK products instead of before them. Every wave
  // still passes one barrier per block, so barrier kb still orders the copies of
  // block kb+1 before every read of it and every read of block kb-1 before the
  // copies that reuse its buffer; the two waves of a SIMD then run half a step
  // apart, one's QK (LDS-heavy) beside the other's PV (matrix-heavy).
  const bool late_sync = wis >= (NW + 1) / 2;
  auto sync_issue = [&](const int kb, uint32_t& vm_next) {
    if (kb + 1 < nb) {
      if (kb + 2 < nb) wait_vmcnt<kUnitsW>();
      else wait_vmcnt<0>();
      __syncthreads();  // block kb+1 is in LDS; block kb-1's buffer is free
      if (kb + kRingM - 1 < nb) {
        uint32_t rv[kUnitsW];
        rows_of(kb + kRingM - 1, rv);
        issue(kb + kRingM - 1, rv);
      }
      vm_next = (uint32_t)__ballot(vslot >= 0);
      vslot = slot[min(kb + 2, nb - 1) * kKB + (lane & 31)];
    }
  };
  auto step = [&](const int kb) {
    uint32_t vm_next = 0u;
    if (!late_sync) sync_issue(kb, vm_next);
    const S2 sc = qk(ring + (kb % kRingM) * kBlkBytes);
    if (late_sync) sync_issue(kb, vm_next);
    float sv[8];  // keys 4g + r (r < 4) and 16 + 4g + (r - 4)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sv[r] = sc.t0[r];
      sv[r + 4] = sc.t1[r];
    }
    if (vm_cur != 0xffffffffu) {
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int key = (r < 4) ? 4 * g + r : 16 + 4 * g + (r - 4);
        if (!((vm_cur >> key) & 1u)) sv[r] = -INFINITY;
      }
    }
    float bmax = sv[0];
#pragma unroll
    for (int r = 1; r < 8; ++r) bmax = fmaxf(bmax, sv[r]);
    bmax *= c2;
    {  // max over the 4 lane groups holding the same head
      const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(bmax), __float_as_uint(bmax), false, false);
      bmax = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
      const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(bmax), __float_as_uint(bmax), false, false);
      bmax = fmaxf(__uint_as_float(c[0]), __uint_as_float(c[1]));
    }
    const bool raise = bmax > m_run + kRaise;
    if (__ballot(raise) != 0) {
      const float m_new = raise ? bmax : m_run;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int ct = 0; ct < kCT; ++ct)
#pragma unroll
        for (int r = 0; r < 4; ++r) o[ct][r] *= alpha;
      m_run = m_new;
    }
    float pe[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) pe[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[r], c2, -m_run));
#pragma unroll
    for (int r = 0; r < 8; ++r) l_run += pe[r];
    // P = hi + lo (~16 bits) or, in split mode, hi + lo + lo2 (all 24 bits): the split
    // kernel's workgroups each take a few blocks (latency-bound), where the third
    // products cost nothing measurable; in the one-pass kernel they would cost ~23 %.
    u32x4 wh, wl, wl2;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float p0 = pe[2 * w], p1 = pe[2 * w + 1];
      const uint32_t h = pack_bf2(p0, p1);
      wh[w] = h;
      const bf16v2 hv = __builtin_bit_cast(bf16v2, h);
      const float r0 = __builtin_amdgcn_fdot2_f32_bf16(hv, neg_lo, p0, false);
      const float r1 = __builtin_amdgcn_fdot2_f32_bf16(hv, neg_hi, p1, false);
      const uint32_t l = pack_bf2(r0, r1);
      wl[w] = l;
      if constexpr (kSplit) {
        const bf16v2 lv = __builtin_bit_cast(bf16v2, l);
        wl2[w] = pack_bf2(__builtin_amdgcn_fdot2_f32_bf16(lv, neg_lo, r0, false),
                          __builtin_amdgcn_fdot2_f32_bf16(lv, neg_hi, r1, false));
      }
    }
    const bf16x8 phi = __builtin_bit_cast(bf16x8, wh);
    const bf16x8 plo = __builtin_bit_cast(bf16x8, wl);
    const bf16x8 plo2 = __builtin_bit_cast(bf16x8, wl2);
    // O^T += V^T . P^T: supplier lane s = lane%16 of group g reads 4 channels
    // 16ct + 4(s%4) .. +3 of key row 4g + s/4 (first read) and 16 + 4g + s/4
    // (second); the transposed reads hand channel 16ct + (lane%16) keys
    // 4g + 0..3 and 16 + 4g + 0..3 to each lane, matching the P operand.
    const uint16_t* kvh = reinterpret_cast<const uint16_t*>(ring + (kb % kRingM) * kBlkBytes);
    const uint16_t* row0 = kvh + (4 * g + (n >> 2)) * (kRowC * 8) + 4 * (n & 3);
    const uint16_t* row1 = row0 + 16 * (kRowC * 8);
    // One V^T fragment is read ahead: the two reads of fragment ct+1 are issued
    // before the two products of fragment ct (the order is pinned below), so the
    // LDS latency overlaps the matrix work.
    auto read_v = [&](int ct) {
      const s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(row0 + 16 * ct));
      const s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(row1 + 16 * ct));
      return __builtin_bit_cast(bf16x8, __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7));
    };
    bf16x8 a_cur = read_v(0);
#pragma unroll
    for (int ct = 0; ct < kCT; ++ct) {
      bf16x8 a_nxt = a_cur;
      if (ct + 1 < kCT) a_nxt = read_v(ct + 1);
      if constexpr (kSplit) o[ct] = mfma16x16x32(a_cur, plo2, o[ct]);
      o[ct] = mfma16x16x32(a_cur, plo, o[ct]);
      o[ct] = mfma16x16x32(a_cur, phi, o[ct]);
      a_cur = a_nxt;
    }
    constexpr int kPv = kSplit ? 3 : 2;  // products per V^T fragment
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
    for (int ct = 0; ct < kCT - 1; ++ct) {
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, kPv, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, kPv, 0);
    vm_cur = vm_next;
  };

  if (nb > 0) {
    if (nb >= 3) wait_vmcnt<2 * kUnitsW>();
    else if (nb == 2) wait_vmcnt<kUnitsW>();
    else wait_vmcnt<0>();
    __syncthreads();
    vm_cur = (uint32_t)__ballot(vslot >= 0);
    vslot = slot[min(1, nb - 1) * kKB + (lane & 31)];
    for (int kb = 0; kb < nb; ++kb) step(kb);
  }
  __syncthreads();  // the ring is reused for the output transpose

  // Z = the sum over the 4 lane groups + exp2(sink - m).
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  if constexpr (kSplit) {
    // Split mode: this range's state relative to its running max m_run (the sink is
    // applied once, by sa_mla_combine_kernel). O^T goes out in register order, per
    // (token, split, wave) 32 tiles of 64 lanes x 16 B, so that every store writes
    // 1 KB contiguously; lane (n, g) of tile ct holds channels 16ct + 4g .. +3 of
    // head 16(NW hgi + wi) + n.
    const int64_t pw = (tok * p.nsplit + sp) * (p.H >> 4) + NW * hgi + wi;
    f32x4* dstp = reinterpret_cast<f32x4*>(p.part) + pw * (kCT * 64) + lane;
#pragma unroll
    for (int ct = 0; ct < kCT; ++ct) dstp[ct * 64] = o[ct];
    if (g == 0) {
      const int64_t prow = (tok * p.nsplit + sp) * p.H + head;
      *reinterpret_cast<float2*>(p.ml + prow * 2) = make_float2(m_run, l_run);
    }
    return;
  }
  const float rz = 1.0f / (l_run + __builtin_amdgcn_exp2f(sink_l2 - m_run));
  // O^T lane data: head n, channels 16ct + 4g + r. Transpose through LDS: per wave
  // 16 head rows of 64 chunks (1 KB); chunk q of row n sits at n*64 + (q ^ n).
  uint8_t* obuf = ring + wi * (16 * 1024);
#pragma unroll
  for (int ct = 0; ct < kCT; ++ct) {
    const uint32_t lo = pack_bf2(o[ct][0] * rz, o[ct][1] * rz);
    const uint32_t hi = pack_bf2(o[ct][2] * rz, o[ct][3] * rz);
    const int q = 2 * ct + (g >> 1);
    *reinterpret_cast<uint2*>(obuf + n * 1024 + (q ^ n) * 16 + 8 * (g & 1)) = uint2{lo, hi};
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  u32x4* dst = reinterpret_cast<u32x4*>(p.out + (tok * p.H + 16 * wi) * kDV);
  for (int r = 0; r < 16; ++r)
    if (16 * wi + r < p.H)
      st_nt(dst + r * 64 + lane, *reinterpret_cast<const u32x4*>(obuf + r * 1024 + (lane ^ r) * 16));
}

#ifndef DSA_MLA_MIN_BPS
#define DSA_MLA_MIN_BPS 2  // slot blocks per split at least (2, 4, 8 measured: 2 best)
#endif
constexpr int kMaxSplit = 32;  // splits per token at most (the combine keeps them in registers)

// Split mode's second step: per (token, head) row, M = max(sink, m_i),
// Z = exp2(sink - M) + sum_i l_i exp2(m_i - M), out = bf16(sum_i O_i exp2(m_i - M) / Z).
// One thread per (token, wave, tile, lane) of the split kernel's register layout
// (head 16 wave + lane % 16, channels 16 tile + 4 (lane / 16) .. +3), so that each
// split's partial is read 1 KB per wave instruction. One wave per workgroup: a
// token's 16 K threads then spread over 256 CUs (each thread reads 16 B of every
// split, 512 B for 32 splits).
struct MlaCombineParams {
  const float* part;
  const float* ml;
  const float* sink;
  uint16_t* out;
  int64_t n;  // threads: B * M * H * 128
  int32_t H, nsplit;
};

__global__ __launch_bounds__(64) void sa_mla_combine_kernel(MlaCombineParams p) {
  const int64_t f = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (f >= p.n) return;
  const int lane = (int)(f & 63);
  const int ct = (int)((f >> 6) & (kCT - 1));
  const int nwv = p.H >> 4;  // waves per token in the split kernel
  const int64_t tw = f >> 11;  // token * nwv + wave
  const int64_t tok = tw / nwv;
  const int w = (int)(tw - tok * nwv);
  const int head = 16 * w + (lane & 15), g = lane >> 4;
  const float sink_l2 = p.sink[head] * kLog2e;
  const f32x4* part = reinterpret_cast<const f32x4*>(p.part);
  // All splits' loads are issued before any is used (the host caps nsplit at
  // kMaxSplit).
  float2 ml[kMaxSplit];
  f32x4 v[kMaxSplit];
#pragma unroll
  for (int i = 0; i < kMaxSplit; ++i) {
    if (i < p.nsplit) {
      const int64_t ts = tok * p.nsplit + i;
      ml[i] = *reinterpret_cast<const float2*>(p.ml + (ts * p.H + head) * 2);
      v[i] = part[((ts * nwv + w) * kCT + ct) * 64 + lane];
    }
  }
  float mx = sink_l2;
#pragma unroll
  for (int i = 0; i < kMaxSplit; ++i)
    if (i < p.nsplit) mx = fmaxf(mx, ml[i].x);
  float z = __builtin_amdgcn_exp2f(sink_l2 - mx);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < kMaxSplit; ++i) {
    if (i < p.nsplit) {
      const float wgt = __builtin_amdgcn_exp2f(ml[i].x - mx);
      z += ml[i].y * wgt;
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] += v[i][r] * wgt;
    }
  }
  const float rz = 1.0f / z;
  uint2 pk;
  pk.x = pack_bf2(acc[0] * rz, acc[1] * rz);
  pk.y = pack_bf2(acc[2] * rz, acc[3] * rz);
  *reinterpret_cast<uint2*>(p.out + (tok * p.H + head) * kDV + 16 * ct + 4 * g) = pk;
}

// Split plan for few tokens (fewer than CUs): each token's heads go to hg head groups
// (h / 16 / hg >= 2 waves each: one wave's copies of two blocks in flight would
// exceed the vmcnt range) and its slot blocks to nsplit ranges (at least
// DSA_MLA_MIN_BPS blocks each, at most kMaxSplit), one workgroup per (token, range,
// group) and about one workgroup per CU in all (each holds the CU's LDS). More head
// groups mean fewer waves per workgroup but fewer query bytes and partials per
// workgroup; more ranges mean more partials to combine. Graph-replayed sweeps at
// 128 heads, 2048 slots, 256 CUs put the best at 4 groups up to cu/64 tokens, 2 up to
// cu/16, else 1, with nsplit = cu / (tokens * hg) (1-2 tokens: 32 x 4; 8: 16 x 2;
// 16: 8 x 2; 32: 8 x 1; 64: 4 x 1; 128: 2 x 1; 192: one pass).
void mla_split_plan(int64_t tokens, int64_t h, int64_t topk, int cu, int* nsplit, int* bps, int* hg) {
  const int nblk = (int)((topk + kKB - 1) / kKB);
  *nsplit = 1;
  *bps = nblk;
  *hg = 1;
  if (tokens <= 0 || tokens >= cu || nblk < 2 * DSA_MLA_MIN_BPS) return;
  int g = 1;
  for (int c = 2; c <= 4; c *= 2)
    if ((h / 16) % c == 0 && h / 16 / c >= 2 && tokens * 4 * c * c <= cu) g = c;
  int64_t want = cu / (tokens * g);
  if (want > nblk / DSA_MLA_MIN_BPS) want = nblk / DSA_MLA_MIN_BPS;
  if (want > kMaxSplit) want = kMaxSplit;
  if (want < 2) return;
  const int per = (int)((nblk + want - 1) / want);
  *bps = per;
  *nsplit = (nblk + per - 1) / per;
  *hg = g;
}

int64_t mla_split_bytes(int64_t tokens, int64_t h, int nsplit) {
  return nsplit > 1 ? tokens * nsplit * h * (kDV + 2) * 4 : 0;
}

template <typename IdxT, bool kSplit>
int mla_launch(const MlaParams& p, int nw, size_t smem, hipStream_t st) {
  const dim3 grid((unsigned)((int64_t)p.B * p.M * p.nsplit * p.hg));
  switch (nw) {
#define DSA_MLA_CASE(n)                                                                           \
  case n:                                                                                         \
    if (dsa_host::ensure_dyn_lds((const void*)sa_mla_kernel<n, IdxT, kSplit>, (int)smem) !=      \
        DSA_OK)                                                                                   \
      return DSA_ERR_LAUNCH;                                                                      \
    hipLaunchKernelGGL((sa_mla_kernel<n, IdxT, kSplit>), grid, dim3(64 * n), smem, st, p);        \
    break;
    DSA_MLA_CASE(2)
    DSA_MLA_CASE(3)
    DSA_MLA_CASE(4)
    DSA_MLA_CASE(5)
    DSA_MLA_CASE(6)
    DSA_MLA_CASE(7)
    DSA_MLA_CASE(8)
#undef DSA_MLA_CASE
    default:
      return DSA_ERR_UNSUPPORTED;
  }
  return hipGetLastError() == hipSuccess ? DSA_OK : DSA_ERR_LAUNCH;
}

// Shared by dsa_sparse_mla_fwd (int32 indices) and dsa_sparse_mla_fwd_i64.
int sparse_mla_fwd(const void* q, const void* kv, const void* topk_idxs, bool idx64,
                   const float* attn_sink, void* out, int64_t b, int64_t m, int64_t h,
                   int64_t d_qk, int64_t d_v, int64_t kv_dim, int64_t n_kv, int64_t topk,
                   float softmax_scale, void* workspace, int64_t workspace_bytes, void* stream) {
  if (b < 0 || m < 0 || h <= 0 || n_kv < 1 || topk < 1 || workspace_bytes < 0) return DSA_ERR_SHAPE;
  if (d_qk != kDQK || d_v != kDV || kv_dim < kDQK) return DSA_ERR_UNSUPPORTED;
  // 4..8 waves of 16 heads (with fewer, a block takes too many copies per wave to
  // keep two blocks in flight under the 6-bit vmcnt).
  if (h % 16 != 0 || h < 64 || h > 128 || topk > 2048) return DSA_ERR_UNSUPPORTED;
  if (!(softmax_scale > 0.f) || !(softmax_scale < INFINITY)) return DSA_ERR_UNSUPPORTED;
  if (n_kv > (1 << 21) || kv_dim > (1 << 16) || (kv_dim % 8) != 0) return DSA_ERR_UNSUPPORTED;
  // The kernel addresses a batch's kv rows through one buffer resource whose size
  // and row offsets are 32-bit byte counts.
  if (n_kv * kv_dim * 2 > (int64_t)UINT32_MAX) return DSA_ERR_UNSUPPORTED;
  if (b * m > INT32_MAX) return DSA_ERR_SHAPE;
  if (b == 0 || m == 0) return DSA_OK;
  if (!q || !kv || !topk_idxs || !attn_sink || !out) return DSA_ERR_NULL;
  if (!dsa_host::aligned16(q) || !dsa_host::aligned16(kv) || !dsa_host::aligned16(out)) return DSA_ERR_ALIGN;
  MlaParams p;
  p.q = (const uint16_t*)q;
  p.kv = (const uint16_t*)kv;
  p.idx = topk_idxs;
  p.sink = attn_sink;
  p.out = (uint16_t*)out;
  p.M = m;
  p.B = (int32_t)b;
  p.H = (int32_t)h;
  p.NKV = (int32_t)n_kv;
  p.TOPK = (int32_t)topk;
  p.kv_dim = (int32_t)kv_dim;
  p.scale_log2 = softmax_scale * kLog2e;
  const int64_t nblk = (topk + kKB - 1) / kKB;
  p.part = nullptr;
  p.ml = nullptr;
  p.nsplit = 1;
  p.bps = (int32_t)nblk;
  p.hg = 1;
  if (workspace != nullptr) {
    int cu = 0;
    if (dsa_host::device_cu_count(&cu) != DSA_OK) return DSA_ERR_DEVICE;
    int nsplit, bps, hg;
    mla_split_plan(b * m, h, topk, cu, &nsplit, &bps, &hg);
    const int64_t need = mla_split_bytes(b * m, h, nsplit);
    if (need > 0 && workspace_bytes >= need) {  // else the one-pass kernel (nothing to split)
      if (!dsa_host::aligned16(workspace)) return DSA_ERR_ALIGN;
      if (b * m * nsplit > INT32_MAX) return DSA_ERR_SHAPE;
      p.part = (float*)workspace;
      p.ml = p.part + b * m * nsplit * h * kDV;
      p.nsplit = nsplit;
      p.bps = bps;
      p.hg = hg;
    }
  }
  const size_t smem = (size_t)kRingM * kBlkBytes + (size_t)nblk * kKB * 4 + 32;  // + per-wave counts
  hipStream_t st = (hipStream_t)stream;
  const int nw = (int)(h / 16) / p.hg;
  int rc;
  if (p.nsplit > 1)
    rc = idx64 ? mla_launch<int64_t, true>(p, nw, smem, st) : mla_launch<int32_t, true>(p, nw, smem, st);
  else
    rc = idx64 ? mla_launch<int64_t, false>(p, nw, smem, st) : mla_launch<int32_t, false>(p, nw, smem, st);
  if (rc != DSA_OK || p.nsplit == 1) return rc;
  MlaCombineParams c;
  c.part = p.part;
  c.ml = p.ml;
  c.sink = attn_sink;
  c.out = (uint16_t*)out;
  c.n = b * m * h * 128;
  c.H = (int32_t)h;
  c.nsplit = p.nsplit;
  hipLaunchKernelGGL(sa_mla_combine_kernel, dim3((unsigned)((c.n + 63) / 64)), dim3(64), 0, st, c);
  return hipGetLastError() == hipSuccess ? DSA_OK : DSA_ERR_LAUNCH;
}

}  // namespace

extern "C" int dsa_sparse_mla_fwd(const void* q, const void* kv, const int32_t* topk_idxs,
                                  const float* attn_sink, void* out, int64_t b, int64_t m,
                                  int64_t h, int64_t d_qk, int64_t d_v, int64_t kv_dim,
                                  int64_t n_kv, int64_t topk, float softmax_scale, void* stream) {
  return sparse_mla_fwd(q, kv, topk_idxs, false, attn_sink, out, b, m, h, d_qk, d_v, kv_dim, n_kv,
                        topk, softmax_scale, nullptr, 0, stream);
}

extern "C" int dsa_sparse_mla_fwd_i64(const void* q, const void* kv, const int64_t* topk_idxs,
                                      const float* attn_sink, void* out, int64_t b, int64_t m,
                                      int64_t h, int64_t d_qk, int64_t d_v, int64_t kv_dim,
                                      int64_t n_kv, int64_t topk, float softmax_scale,
                                      void* stream) {
  return sparse_mla_fwd(q, kv, topk_idxs, true, attn_sink, out, b, m, h, d_qk, d_v, kv_dim, n_kv,
                        topk, softmax_scale, nullptr, 0, stream);
}

extern "C" int64_t dsa_sparse_mla_workspace_bytes(int64_t b, int64_t m, int64_t h, int64_t topk) {
  if (b < 0 || m < 0 || h <= 0 || topk <= 0 || b * m > INT32_MAX) return DSA_ERR_SHAPE;
  if (b == 0 || m == 0) return 0;
  int cu = 0;
  if (dsa_host::device_cu_count(&cu) != DSA_OK) return DSA_ERR_DEVICE;
  int nsplit, bps, hg;
  mla_split_plan(b * m, h, topk, cu, &nsplit, &bps, &hg);
  return mla_split_bytes(b * m, h, nsplit);
}

extern "C" int dsa_sparse_mla_fwd_ws(const void* q, const void* kv, const int32_t* topk_idxs,
                                     const float* attn_sink, void* out, int64_t b, int64_t m,
                                     int64_t h, int64_t d_qk, int64_t d_v, int64_t kv_dim,
                                     int64_t n_kv, int64_t topk, float softmax_scale,
                                     void* workspace, int64_t workspace_bytes, void* stream) {
  return sparse_mla_fwd(q, kv, topk_idxs, false, attn_sink, out, b, m, h, d_qk, d_v, kv_dim, n_kv,
                        topk, softmax_scale, workspace, workspace_bytes, stream);
}

extern "C" int dsa_sparse_mla_fwd_i64_ws(const void* q, const void* kv, const int64_t* topk_idxs,
                                         const float* attn_sink, void* out, int64_t b, int64_t m,
                                         int64_t h, int64_t d_qk, int64_t d_v, int64_t kv_dim,
                                         int64_t n_kv, int64_t topk, float softmax_scale,
                                         void* workspace, int64_t workspace_bytes, void* stream) {
  return sparse_mla_fwd(q, kv, topk_idxs, true, attn_sink, out, b, m, h, d_qk, d_v, kv_dim, n_kv,
                        topk, softmax_scale, workspace, workspace_bytes, stream);
}
