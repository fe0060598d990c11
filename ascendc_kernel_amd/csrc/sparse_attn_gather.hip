// Task1, true-gather variant (any n_kv): each token attends to the kv rows its
// topk slots select, gathered from the batch's kv block (reference semantics
// of sparse_attn_ref, reference/task1_v0_ref.py:5-24; duplicates and masked
// slots handled exactly like the gather there).
//
// One workgroup per token, one wave per 32 heads (ceil(h/32) waves). The slots are
// processed in blocks of 32: the workgroup gathers the 32 selected kv rows
// (256 B each) into LDS -- double-buffered, the next block's rows are loaded
// while the current one is computed -- and every wave runs
//   S^T[32 keys x 32 heads]  = K[32 x 128] . Q^T[128 x 32]   (8 x mfma 32x32x16)
//   online softmax with the sink as the initial maximum (log2 domain)
//   O^T[128 x 32 heads]     += V^T[128 x 32] . (P_hi + P_lo)^T (16 x mfma 32x32x16)
// K fragments are 16-byte LDS reads of the swizzled rows; V^T fragments come
// from the same rows through ds_read_b64_tr_b16, which transposes 4x16-bit
// elements across each 16-lane group. The running maximum is only raised when
// a block exceeds it by more than 2^8 (then O and the sum are rescaled), which
// keeps exp2 arguments <= 8 and makes the rescale rare.
#include "dsa_common.h"

using namespace dsa;

namespace {

constexpr int kD = 128;
constexpr int kKB = 32;          // slots per block
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRaise = 8.0f;   // log2 headroom before the running max is raised

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4* lds_s16x4_ptr;

struct GatherParams {
  const uint16_t* q;     // [B, M, H, 128]
  const uint16_t* kv;    // [B, NKV, 128]
  const int32_t* idx;    // [B, M, TOPK]
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

template <int NW>
__global__ __launch_bounds__(64 * NW) void sa_gather_kernel(GatherParams p) {
  __shared__ u32x4 kvbuf[2][kKB * 16];   // two blocks of 32 gathered rows
  __shared__ int32_t slot[2048];          // the token's slot indices (masked -> -1)
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

  // Slot indices -> LDS; out-of-range indices count as masked.
  const int nblk = (p.TOPK + kKB - 1) / kKB;
  for (int s = tid; s < nblk * kKB; s += 64 * NW) {
    int v = -1;
    if (s < p.TOPK) {
      v = p.idx[tok * p.TOPK + s];
      if (v >= p.NKV) v = -1;
    }
    slot[s] = v;
  }

  // Q^T fragments (B operand of the first product): head hbase+col, channels
  // 16ks + 8hf .. +7.
  bf16x8 qf[8];
  {
    const uint16_t* qrow = p.q + (tok * p.H + (hvalid ? hbase + col : 0)) * kD + 8 * hf;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
      qf[ks] = hvalid ? __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(qrow + 16 * ks))
                      : __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
  }
  __syncthreads();

  // Gather loads of one block: chunk e (0..511) = row e/16, chunk e%16;
  // thread tid covers e = tid + 64*NW*j.
  constexpr int kPer = (512 + 64 * NW - 1) / (64 * NW);
  u32x4 stage[kPer];
  auto load_block = [&](int kb) {
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = tid + 64 * NW * j, r = (e >> 4) & 31, c = e & 15;
      int row = slot[kb * kKB + r];
      if (row < 0) row = 0;
      if (e < 512) stage[j] = *reinterpret_cast<const u32x4*>(kvb + (int64_t)row * kD + 8 * c);
    }
  };
  auto store_block = [&](int buf) {
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = tid + 64 * NW * j, r = (e >> 4) & 31, c = e & 15;
      if (e < 512) kvbuf[buf][swz(r, c)] = stage[j];
    }
  };

  f32x16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = f32x16{};
  const float sink_l2 = hvalid ? p.sink[hbase + col] * kLog2e : 0.f;
  float m_run = sink_l2;   // running max (log2 units) incl. the sink
  float l_run = 0.f;       // this lane's partial sum of exp2(s - m_run)

  load_block(0);
  store_block(0);
  __syncthreads();

  for (int kb = 0; kb < nblk; ++kb) {
    const int buf = kb & 1;
    if (kb + 1 < nblk) load_block(kb + 1);
    const u32x4* kvl = kvbuf[buf];

    // Slot validity of this block as a bit mask (uniform).
    const int myslot = slot[kb * kKB + (lane & 31)];
    const uint32_t vmask = (uint32_t)__ballot(myslot >= 0);

    if (vmask != 0u) {
      // S^T = K . Q^T : A = K rows (key = lane%32, channels 16ks + 8hf ..).
      f32x16 s = {};
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const bf16x8 a = __builtin_bit_cast(bf16x8, kvl[swz(lane & 31, 2 * ks + hf)]);
        s = mfma32x32x16(a, qf[ks], s);
      }
      // Lane holds keys 8(r/4) + 4hf + (r%4) of head col.
      float sv[16];
      float bmax = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = 8 * (r >> 2) + 4 * hf + (r & 3);
        const bool ok = (vmask >> key) & 1u;
        sv[r] = ok ? s[r] * p.scale_log2 : -INFINITY;
        bmax = fmaxf(bmax, sv[r]);
      }
      bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
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
      float pe[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        pe[r] = __builtin_amdgcn_exp2f(sv[r] - m_run);  // exp2(-inf) = 0 for masked slots
        l_run += pe[r];
      }
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
          wl[w] = pack_bf2(p0 - bf_lo(h), p1 - bf_hi(h));
        }
        phi[st] = __builtin_bit_cast(bf16x8, wh);
        plo[st] = __builtin_bit_cast(bf16x8, wl);
      }
      // O^T += V^T . P^T. A operand rows: channel out_ch(dt, lane%32); the two
      // transposed reads give keys 16st + 4hf + (0..3) and 16st + 8 + 4hf + (0..3).
      // Supplier lane u of a 16-lane group reads 4 channels of one key row:
      // key = base + (u >> 2), channels out_ch(dt, 16*g16 + 4*(u & 3)) .. +3.
      const int u = lane & 15, g16 = (lane >> 4) & 1;
      const uint16_t* kvh = reinterpret_cast<const uint16_t*>(kvl);
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
    }

    if (kb + 1 < nblk) store_block(buf ^ 1);
    __syncthreads();
  }

  // Normalise: Z = sum over both lane halves + exp2(sink - m_run).
  l_run += __shfl_xor(l_run, 32, 64);
  const float rz = 1.0f / (l_run + __builtin_amdgcn_exp2f(sink_l2 - m_run));
  // O^T lane data: head col, channels out_ch(dt, 8(r/4) + 4hf + r%4) =
  // 64hf + 16dt + 4(r/4) + r%4 -> the lane owns channels 64hf .. 64hf+63.
  // Transpose through LDS (the gather buffer is free now) for coalesced stores.
  __shared__ u32x4 obuf[NW][32 * 16];  // 32 heads x 16 chunks = 8 KB per wave
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
      obuf[wi][swz(col, chunk)] = w;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  u32x4* dst = reinterpret_cast<u32x4*>(p.out + (tok * p.H + hbase) * kD);
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int r = 4 * k + (lane >> 4), c = lane & 15;
    if (hbase + r < p.H) st_nt(dst + r * 16 + c, obuf[wi][swz(r, c)]);
  }
}

}  // namespace

int dsa_sparse_attn_gather_launch(const void* q, const void* kv, const int32_t* idx, const float* sink,
                                  void* out, int64_t b, int64_t m, int64_t h, int64_t n_kv,
                                  int64_t topk, float scale, hipStream_t stream) {
  if (h % 16 != 0 || h > 128) return DSA_ERR_UNSUPPORTED;
  if (topk > 2048) return DSA_ERR_UNSUPPORTED;
  if (n_kv > (int64_t)INT32_MAX) return DSA_ERR_SHAPE;
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
  switch ((h + 31) / 32) {
    case 1: hipLaunchKernelGGL(sa_gather_kernel<1>, grid, dim3(64), 0, stream, p); break;
    case 2: hipLaunchKernelGGL(sa_gather_kernel<2>, grid, dim3(128), 0, stream, p); break;
    case 3: hipLaunchKernelGGL(sa_gather_kernel<3>, grid, dim3(192), 0, stream, p); break;
    case 4: hipLaunchKernelGGL(sa_gather_kernel<4>, grid, dim3(256), 0, stream, p); break;
    default: return DSA_ERR_UNSUPPORTED;
  }
  return hipGetLastError() == hipSuccess ? DSA_OK : DSA_ERR_LAUNCH;
}
