// Task1, true-gather variant (any n_kv): each token attends to the kv rows its
// topk slots select, gathered from the batch's kv block (reference semantics
// of sparse_attn_ref, reference/task1_v0_ref.py:5-24; duplicates and masked
// slots handled exactly like the gather there).
//
// One workgroup per token, one wave per 32 heads (ceil(h/32) waves). The slots are
// processed in blocks of 32. The selected kv rows (256 B each) of a block are
// copied straight from global memory into LDS by global_load_lds_dwordx4 (no
// register staging), into a ring of kRing block buffers: kRing - 1 blocks are in
// flight while one is computed. Every wave then runs
//   S^T[32 keys x 32 heads]  = K[32 x 128] . Q^T[128 x 32]   (8 x mfma 32x32x16)
//   online softmax with the sink as the initial maximum (log2 domain)
//   O^T[128 x 32 heads]     += V^T[128 x 32] . (P_hi + P_lo)^T (16 x mfma 32x32x16)
// K fragments are 16-byte LDS reads of the swizzled rows; V^T fragments come
// from the same rows through ds_read_b64_tr_b16, which transposes 4x16-bit
// elements across each 16-lane group. The running maximum is only raised when
// a block exceeds it by more than 2^8 (then O and the sum are rescaled), which
// keeps exp2 arguments <= 8 and makes the rescale rare. P is split into a bf16
// high part and a bf16 residual so that the PV product keeps ~16 bits of P.
#include "dsa_common.h"

#include <float.h>

using namespace dsa;

namespace {

constexpr int kD = 128;
constexpr int kKB = 32;          // slots per block
constexpr int kRing = 4;         // LDS block buffers (kRing - 1 blocks in flight)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRaise = 8.0f;   // log2 headroom before the running max is raised
// bf16 pairs (-1, 0) and (0, -1) as bit patterns: dot2(h, neg_lo, p0) = p0 - h.lo,
// dot2(h, neg_hi, p1) = p1 - h.hi.
constexpr uint32_t kNegLoBits = 0x0000bf80u;
constexpr uint32_t kNegHiBits = 0xbf800000u;

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4* lds_s16x4_ptr;

struct GatherParams {
  const uint16_t* q;     // [B, M, H, 128]
  const uint16_t* kv;    // [B, NKV, 128]
  const void* idx;       // [B, M, TOPK] int32 or int64 (the kernel's IdxT)
  const float* sink;     // [H]
  uint16_t* out;         // [B, M, H, 128]
  int64_t M;
  int32_t B, H, NKV, TOPK;
  int32_t xpb;           // XCDs per batch for the block -> token map (0: identity)
  float scale_log2;      // softmax_scale * log2(e)
};

// Output channel of row i of d-tile dt (O^T rows): lane half hf = (i >> 2) & 1
// gets the contiguous channels 64*hf .. 64*hf + 63 across the four d-tiles.
__device__ __forceinline__ int out_ch(int dt, int i) {
  const int q = i >> 3, hf = (i >> 2) & 1, c = i & 3;
  return 64 * hf + 16 * dt + 4 * q + c;
}

// LDS row r (256 B = 16 chunks of 16 B): chunk c lives at r*16 + (c ^ (r & 15)).
__device__ __forceinline__ int swz(int r, int c) { return r * 16 + (c ^ (r & 15)); }

template <int NW, typename IdxT>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(NW >= 2 ? 2 : 1)))
void sa_gather_kernel(GatherParams p) {
  const IdxT* const idx = static_cast<const IdxT*>(p.idx);
  __shared__ u32x4 ring[kRing][kKB * 16];  // kRing blocks of 32 gathered rows (8 KB each)
  __shared__ int32_t nblk_w[NW];  // per wave: blocks up to its last valid slot
  extern __shared__ int32_t slot[];         // the token's slot indices (masked -> -1)
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wi = tid >> 6;
  // Blocks are dispatched to the 8 XCDs round-robin; map them so that XCD x
  // only serves batch x % B and its L2 keeps that batch's kv block.
  int64_t tok;
  if (p.xpb > 0) {
    const int xcd = blockIdx.x & 7;
    const int64_t slotno = blockIdx.x >> 3;
    tok = (int64_t)(xcd % p.B) * p.M + slotno * p.xpb + xcd / p.B;
  } else {
    tok = blockIdx.x;
  }
  const int b = (int)(tok / p.M);
  const int hbase = 32 * wi;             // this wave's heads
  const int col = lane & 31;             // head hbase + col (MFMA column)
  const int hf = lane >> 5;              // lane half: contraction slice 8*hf..8*hf+7
  const bool hvalid = hbase + col < p.H;  // the last wave may cover fewer than 32 heads
  const uint16_t* kvb = p.kv + (int64_t)b * p.NKV * kD;

  // The token's global reads (Q^T, the sink, the slot indices) are all issued
  // before any of them is waited for: one memory latency instead of one per
  // round of the slot loop.
  // Q^T fragments (B operand of the first product): head hbase+col, channels
  // 16ks + 8hf .. +7.
  // Lanes of heads >= H (the last wave when H % 32 != 0) load head 0's row: their
  // MFMA columns and softmax stay separate from the valid heads' and are never
  // stored; loading unconditionally keeps the loads out of branches (whose joins
  // would make the compiler wait for them at once).
  bf16x8 qf[8];
  {
    const uint16_t* qrow = p.q + (tok * p.H + (hvalid ? hbase + col : 0)) * kD + 8 * hf;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
      qf[ks] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(qrow + 16 * ks));
  }
  const float sink_raw = p.sink[hvalid ? hbase + col : 0];  // unconditional: no wait in a branch
  // Slot indices -> LDS, 8 per thread in flight at a time; out-of-range indices
  // count as masked. Blocks after the last one holding a valid slot are neither
  // loaded nor computed.
  const int nblk = (p.TOPK + kKB - 1) / kKB;
  int last = 0;
  auto slot_chunk = [&](const int s0) {
    int v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int s = s0 + 64 * NW * u + tid;
      v[u] = slot_index(idx, tok * p.TOPK + min(s, p.TOPK - 1));  // unconditional (see q)
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int s = s0 + 64 * NW * u + tid;
      if (s < nblk * kKB) {
        const int w = (s < p.TOPK && v[u] < p.NKV) ? v[u] : -1;
        slot[s] = w;
        if (w >= 0) last = s / kKB + 1;
      }
    }
  };
  // the first chunk outside the loop, so that nothing waits for Q^T before its loads issue
  slot_chunk(0);
  for (int s0 = 8 * 64 * NW; s0 < nblk * kKB; s0 += 8 * 64 * NW) slot_chunk(s0);
  // Blocks to compute: the maximum of `last` over the wave, then over the waves.
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) last = max(last, __shfl_xor(last, m, 64));
  if (lane == 0) nblk_w[wi] = last;
  __syncthreads();
  int nb = nblk_w[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) nb = max(nb, nblk_w[w]);

  // A block is 8 units of 4 rows (1 KB); one global_load_lds_dwordx4 moves a
  // unit: lane l writes LDS chunk 64u + l, i.e. row 4u + l/16, swizzled chunk
  // position l%16, which holds logical chunk (l%16) ^ (row & 15). Wave wi moves
  // units wi, wi + NW, ...; with NW = 3 the last wave reloads unit 0 (same bytes).
  constexpr int kUnits = (8 + NW - 1) / NW;
  const int wis = __builtin_amdgcn_readfirstlane(wi);
  const i32x4 rsrc = make_rsrc(kvb, (uint32_t)p.NKV * (uint32_t)(kD * 2));
  const uint32_t ring_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) u32x4*)&ring[0][0];
  int urow[kUnits];
  uint32_t uoff[kUnits], ulds[kUnits];
#pragma unroll
  for (int i = 0; i < kUnits; ++i) {
    int u = wis + NW * i;
    if (u >= 8) u -= 8;
    urow[i] = 4 * u + (lane >> 4);
    uoff[i] = 16u * (uint32_t)((lane & 15) ^ (urow[i] & 15));  // bytes within the row
    ulds[i] = ring_lds + 1024u * (uint32_t)u;
  }
  // Slot values (kv rows) of this lane's units of block blk.
  auto rows_of = [&](int blk, int (&rv)[kUnits]) {
#pragma unroll
    for (int i = 0; i < kUnits; ++i) rv[i] = slot[blk * kKB + urow[i]];
  };
  // Copy block blk (rows rv) into ring buffer rs. A masked row (-1) gives an
  // offset beyond the resource, which reads zeros.
  auto issue = [&](int rs, const int (&rv)[kUnits]) {
#pragma unroll
    for (int i = 0; i < kUnits; ++i)
      lds_dma16(rsrc, (uint32_t)rv[i] * (uint32_t)(kD * 2) + uoff[i], ulds[i] + 8192u * (uint32_t)rs);
  };
  f32x16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = f32x16{};
  const float sink_l2 = hvalid ? sink_raw * kLog2e : 0.f;
  const float c2 = p.scale_log2;  // > 0 (checked by the host)
  // Running max (log2 units) incl. the sink, floored at -FLT_MAX so that a -inf
  // sink with a fully masked first block gives exp2(-inf) = 0, not NaN.
  float m_run = fmaxf(sink_l2, -FLT_MAX);
  float l_run = 0.f;       // this lane's partial sum of exp2(s - m_run)

  // S^T = K . Q^T for the block in LDS buffer kvl: A = K rows (key = lane%32,
  // channels 16ks + 8hf ..). Lane holds keys 8(r/4) + 4hf + (r%4) of head col.
  auto qk = [&](const u32x4* kvl) {
    f32x16 acc = {};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      const bf16x8 a = __builtin_bit_cast(bf16x8, kvl[swz(lane & 31, 2 * ks + hf)]);
      acc = mfma32x32x16(a, qf[ks], acc);
    }
    return acc;
  };

  int rv[kUnits];
#pragma unroll
  for (int j = 0; j < kRing - 1; ++j) {
    if (j < nb) {
      rows_of(j, rv);
      issue(j, rv);
    }
  }
  // The LDS reads that feed the next iteration are issued one iteration early,
  // so their latency hides behind the wait and the compute: the rows of the
  // block to copy next and this lane's slot of the block to compute next.
  if (nb > 0) rows_of(min(kRing - 1, nb - 1), rv);
  int vslot = slot[lane & 31];
  // The compiler-tracked loads (q, sink) are consumed here, so its own waitcnt
  // (a vmcnt(0), which also covers the copies just issued) stays out of the loop.
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) asm volatile("" ::"v"(qf[ks]));
  asm volatile("" ::"v"(m_run));

  // Two-stage pipeline: iteration kb computes S of block kb+1 on the matrix
  // cores while the VALU runs the softmax of block kb, then O += P(kb) V(kb).
  // Block kb+1 must be in LDS at the start of iteration kb, block kb is read
  // until its end; the copy issued in iteration kb (block kb+3) goes to the
  // buffer of block kb-1, released by the barrier. So 2 copies are in flight.
  static_assert(kRing == 4, "the waits assume a ring of 4 buffers");
  // One iteration for block kb, which sits in ring buffer j = kb % kRing (the
  // loop is unrolled by kRing so that j, and with it every LDS offset below,
  // is a compile-time constant).
  uint32_t vm_cur = 0u;
  f32x16 s_cur = {};
  // The two dot2 operands live in SGPRs: as a literal, the compiler encodes the
  // pair (-1, 0) as the inline constant -1.0, which v_dot2c_f32_bf16 reads as the
  // fp32 bit pattern, i.e. the pair (0, -1).
  uint32_t neg_lo_bits = kNegLoBits, neg_hi_bits = kNegHiBits;
  asm volatile("" : "+s"(neg_lo_bits), "+s"(neg_hi_bits));
  const bf16v2 neg_lo = __builtin_bit_cast(bf16v2, neg_lo_bits);
  const bf16v2 neg_hi = __builtin_bit_cast(bf16v2, neg_hi_bits);
  auto step = [&](const int kb, const int j) {
    uint32_t vm_next = 0u;
    if (kb + 1 < nb) {
      // Block kb+1 has landed once at most one younger block is outstanding.
      if (kb + 2 < nb) wait_vmcnt<kUnits>();
      else wait_vmcnt<0>();
      __syncthreads();  // block kb+1 is in LDS for every wave; block kb-1 is consumed
      if (kb + kRing - 1 < nb) issue((j + kRing - 1) % kRing, rv);
      vm_next = (uint32_t)__ballot(vslot >= 0);
      rows_of(min(kb + kRing, nb - 1), rv);
      vslot = slot[min(kb + 2, nb - 1) * kKB + (lane & 31)];
    }
    // Masked slots of block kb -> -inf (uniform branch; full blocks skip it).
    if (vm_cur != 0xffffffffu) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = 8 * (r >> 2) + 4 * hf + (r & 3);
        if (!((vm_cur >> key) & 1u)) s_cur[r] = -INFINITY;
      }
    }
    // max(s) * c2 == max(s * c2) for c2 > 0; the other lane half holds the
    // other 16 keys of the same head.
    float bmax = s_cur[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) bmax = fmaxf(bmax, s_cur[r]);
    bmax *= c2;
    {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(bmax), __float_as_uint(bmax),
                                                       false, false);
      bmax = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    }
    // Raise the running max only when this block exceeds it by > kRaise.
    const bool raise = bmax > m_run + kRaise;
    if (__ballot(raise) != 0) {
      const float m_new = raise ? bmax : m_run;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
      m_run = m_new;
    }

    // S of the next block (after the last block this reads a stale buffer and
    // the result is unused), independent of the softmax below.
    // The wave runs at raised priority from here to the PV products: on a SIMD
    // shared with another workgroup's wave, the softmax (VALU) of one wave then
    // tends to issue while the other's products occupy the matrix cores (~4 %).
    __builtin_amdgcn_s_setprio(1);
    const f32x16 s_next = qk(ring[(j + 1) % kRing]);

    float pe[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) pe[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[r], c2, -m_run));
#pragma unroll
    for (int r = 0; r < 16; ++r) l_run += pe[r];
    // B operands of the second product, hi + lo bf16: K-step st uses the
    // lane's registers 8st..8st+7 (keys 16st + 8(j/4) + 4hf + j%4).
    bf16x8 phi[2], plo[2];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      u32x4 wh, wl;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float p0 = pe[8 * st + 2 * w], p1 = pe[8 * st + 2 * w + 1];
        const uint32_t h = pack_bf2(p0, p1);
        wh[w] = h;
        // residuals p - bf16(p), exact in fp32: one v_dot2c each
        const bf16v2 hv = __builtin_bit_cast(bf16v2, h);
        wl[w] = pack_bf2(__builtin_amdgcn_fdot2_f32_bf16(hv, neg_lo, p0, false),
                         __builtin_amdgcn_fdot2_f32_bf16(hv, neg_hi, p1, false));
      }
      phi[st] = __builtin_bit_cast(bf16x8, wh);
      plo[st] = __builtin_bit_cast(bf16x8, wl);
    }
    // O^T += V^T . P^T. A operand rows: channel out_ch(dt, lane%32); the two
    // transposed reads give keys 16st + 4hf + (0..3) and 16st + 8 + 4hf + (0..3).
    // Supplier lane u of a 16-lane group reads 4 channels of one key row:
    // key = base + (u >> 2), channels out_ch(dt, 16*g16 + 4*(u & 3)) .. +3.
    __builtin_amdgcn_s_setprio(0);
    const int u = lane & 15, g16 = (lane >> 4) & 1;
    const uint16_t* kvh = reinterpret_cast<const uint16_t*>(ring[j]);
#pragma unroll
    for (int st = 0; st < 2; ++st) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const int ch = out_ch(dt, 16 * g16 + 4 * (u & 3));
        const int r0 = 16 * st + 4 * hf + (u >> 2);
        const int r1 = r0 + 8;
        const s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s16x4_ptr)(kvh + swz(r0, ch >> 3) * 8 + (ch & 7)));
        const s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s16x4_ptr)(kvh + swz(r1, ch >> 3) * 8 + (ch & 7)));
        const s16x8 v01 = __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
        const bf16x8 a = __builtin_bit_cast(bf16x8, v01);
        o[dt] = mfma32x32x16(a, plo[st], o[dt]);
        o[dt] = mfma32x32x16(a, phi[st], o[dt]);
      }
    }
    s_cur = s_next;
    vm_cur = vm_next;
  };

  if (nb > 0) {
    if (nb >= 3) wait_vmcnt<2 * kUnits>();
    else if (nb == 2) wait_vmcnt<kUnits>();
    else wait_vmcnt<0>();
    __syncthreads();
    vm_cur = (uint32_t)__ballot(vslot >= 0);
    vslot = slot[min(1, nb - 1) * kKB + (lane & 31)];
    s_cur = qk(ring[0]);
    for (int kb0 = 0; kb0 < nb; kb0 += kRing) {
#pragma unroll
      for (int j = 0; j < kRing; ++j) {
        if (kb0 + j >= nb) break;
        step(kb0 + j, j);
      }
    }
  }
  __syncthreads();  // every wave is done with the ring; it is reused below

  // Normalise: Z = sum over both lane halves + exp2(sink - m_run).
  l_run += __shfl_xor(l_run, 32, 64);
  const float rz = 1.0f / (l_run + __builtin_amdgcn_exp2f(sink_l2 - m_run));
  // O^T lane data: head col, channels out_ch(dt, 8(r/4) + 4hf + r%4) =
  // 64hf + 16dt + 4(r/4) + r%4 -> the lane owns channels 64hf .. 64hf+63.
  // Transpose through LDS (ring buffer wi; 32 heads x 16 chunks = 8 KB) for
  // coalesced stores.
  u32x4* obuf = ring[wi];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
    for (int hc = 0; hc < 2; ++hc) {
      // channels 64hf + 16dt + 8hc .. +7 = registers r = 8hc .. 8hc+7
      u32x4 w;
#pragma unroll
      for (int k = 0; k < 4; ++k)
        w[k] = pack_bf2(o[dt][8 * hc + 2 * k] * rz, o[dt][8 * hc + 2 * k + 1] * rz);
      const int chunk = 8 * hf + 2 * dt + hc;
      obuf[swz(col, chunk)] = w;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  u32x4* dst = reinterpret_cast<u32x4*>(p.out + (tok * p.H + hbase) * kD);
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int r = 4 * k + (lane >> 4), c = lane & 15;
    if (hbase + r < p.H) st_nt(dst + r * 16 + c, obuf[swz(r, c)]);
  }
}

}  // namespace

int dsa_sparse_attn_gather_launch(const void* q, const void* kv, const void* idx, bool idx64,
                                  const float* sink, void* out, int64_t b, int64_t m, int64_t h,
                                  int64_t n_kv, int64_t topk, float scale, hipStream_t stream) {
  if (h % 16 != 0 || h > 128) return DSA_ERR_UNSUPPORTED;
  if (topk > 2048) return DSA_ERR_UNSUPPORTED;
  if (!(scale > 0.f) || !(scale < INFINITY)) return DSA_ERR_UNSUPPORTED;  // the kernel's max uses scale > 0
  if (n_kv > (INT64_C(1) << 23)) return DSA_ERR_UNSUPPORTED;  // byte offsets of kv rows fit 32 bits
  const int64_t tokens = b * m;
  if (tokens > INT32_MAX) return DSA_ERR_SHAPE;
  GatherParams p;
  p.q = (const uint16_t*)q;
  p.kv = (const uint16_t*)kv;
  p.idx = idx;
  p.sink = sink;
  p.out = (uint16_t*)out;
  p.M = m;
  p.B = (int32_t)b;
  p.H = (int32_t)h;
  p.NKV = (int32_t)n_kv;
  p.TOPK = (int32_t)topk;
  p.scale_log2 = scale * kLog2e;
  p.xpb = (b <= 8 && 8 % b == 0 && m % (8 / b) == 0) ? (int32_t)(8 / b) : 0;
  const dim3 grid((unsigned)tokens);
  // Dynamic LDS: the slot list, padded to whole blocks.
  const size_t smem = (size_t)((topk + kKB - 1) / kKB) * kKB * sizeof(int32_t);
  const int nw = (int)((h + 31) / 32);
  if (nw < 1 || nw > 4) return DSA_ERR_UNSUPPORTED;
  if (idx64) {
    switch (nw) {
      case 1: hipLaunchKernelGGL((sa_gather_kernel<1, int64_t>), grid, dim3(64), smem, stream, p); break;
      case 2: hipLaunchKernelGGL((sa_gather_kernel<2, int64_t>), grid, dim3(128), smem, stream, p); break;
      case 3: hipLaunchKernelGGL((sa_gather_kernel<3, int64_t>), grid, dim3(192), smem, stream, p); break;
      default: hipLaunchKernelGGL((sa_gather_kernel<4, int64_t>), grid, dim3(256), smem, stream, p); break;
    }
  } else {
    switch (nw) {
      case 1: hipLaunchKernelGGL((sa_gather_kernel<1, int32_t>), grid, dim3(64), smem, stream, p); break;
      case 2: hipLaunchKernelGGL((sa_gather_kernel<2, int32_t>), grid, dim3(128), smem, stream, p); break;
      case 3: hipLaunchKernelGGL((sa_gather_kernel<3, int32_t>), grid, dim3(192), smem, stream, p); break;
      default: hipLaunchKernelGGL((sa_gather_kernel<4, int32_t>), grid, dim3(256), smem, stream, p); break;
    }
  }
  return hipGetLastError() == hipSuccess ? DSA_OK : DSA_ERR_LAUNCH;
}
