// Task1: sparse attention with attention sink on gfx950 (MI355X).
//
// Semantics follow sparse_attn_ref (reference/task1_v0_ref.py:5-24): for every
// (batch b, token m, head h) the scores s_t = scale * q . kv[idx_t] over the
// token's topk slots (slots with idx < 0 are masked), M = max(max_t s_t, sink_h),
// weights e_t / (sum_t e_t + exp(sink_h - M)) with e_t = exp(s_t - M), and
// out = sum_t weight_t * kv[idx_t], rounded to bf16.
//
// Multiplicity kernel (n_kv <= 32). A token's topk slots only select rows of
// the batch's small kv block, so sum_t f(idx_t) = sum_j c_j f(j) with c_j the
// number of slots holding j (the identity the Ascend kernel also uses,
// src/sparse_attn_kernel_mm.asc:155-292). Each wave streams 16-row tiles
// (16 heads of one token) straight from HBM into MFMA operands:
//   S^T[32 x 16]  = KV[32 x 128] . Q^T[128 x 16]        (8 x mfma 16x16x32)
//   P             = c_j * exp(S - M) / Z, fp32, split into three bf16 terms
//                   P_hi + P_lo + P_lo2 (together all 24 bits of P)
//   O^T[128 x 16] = KV^T[128 x 32] . (P_lo2 + P_lo + P_hi)^T  (24 x mfma 16x16x32)
// The kv block of the current batch lives in registers in both operand
// layouts, so S and P never leave the CU. The contraction indices of both
// products are permuted (pi over kv rows, delta over channels) so that the
// softmax output is already in the B-operand layout of the second product and
// every lane loads and stores 16 contiguous bytes of a row.
#include "dsa_common.h"

#include <atomic>
#include <mutex>

using namespace dsa;

namespace {

constexpr int kD = 128;

// Streaming knobs (compile-time): cache policy of the q loads / out stores and
// the number of resident waves the grid is sized for.
#ifndef DSA_SA_NT_LOAD
#define DSA_SA_NT_LOAD 1
#endif
#ifndef DSA_SA_NT_STORE
#define DSA_SA_NT_STORE 1
#endif
#ifndef DSA_SA_TILES_PER_WAVE
#define DSA_SA_TILES_PER_WAVE 2
#endif

struct MultParams {
  const uint16_t* q;
  const uint16_t* kv;
  const void* idx;           // [B, M, TOPK] int32 or int64 (the kernel's IdxT)
  const float* sink;
  uint16_t* out;
  int64_t M;                 // tokens per batch
  int64_t tiles_per_batch;   // M * H / 16
  int64_t blocks_per_batch;  // ceil(tiles_per_batch / (4 * tiles per wave))
  int32_t H;
  int32_t NKV;
  int32_t TOPK;
  float scale;
};

// Contraction permutation of the second product: logical k (lane group g owns
// k = 8g..8g+7) -> kv row. Lane group g holds the softmax of kv rows
// 4g..4g+3 (first S tile) and 16+4g..16+4g+3 (second S tile).
__device__ __forceinline__ int pi_kv(int k) {
  const int g = k >> 3, j = k & 7;
  return (j < 4) ? (4 * g + j) : (16 + 4 * g + (j - 4));
}
// Output-channel permutation of the second product: logical row i of M-tile mt
// -> channel. Chosen so lane group g of store p holds channels 32p+8g..32p+8g+7.
__device__ __forceinline__ int delta_ch(int mt, int i) {
  return 32 * (mt >> 1) + 8 * (i >> 2) + 4 * (mt & 1) + (i & 3);
}

// Orders this wave's LDS accesses across lanes (LDS executes a wave's
// instructions in order; this keeps the compiler from reordering them).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ bf16x8 load_row16(const uint16_t* p) {
#if DSA_SA_NT_LOAD
  return __builtin_bit_cast(bf16x8, ld_nt(reinterpret_cast<const u32x4*>(p)));
#else
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(p));
#endif
}

// One workgroup = 4 waves = 4 * TPW consecutive 16-row tiles of one batch.
// Load order matters because vector-memory completions are counted in issue
// order: the batch's kv block and the small per-tile values (sink, slot
// indices) are requested first, then all q tiles of the wave; the workgroup
// waits only for the first group, stages the kv block in LDS (as a swizzled
// row copy and as the pre-permuted operand of the second product) and then
// computes tile by tile while the q loads are still arriving.
// Four resident workgroups per CU (<= 128 VGPRs, 32 KB LDS each): with two tiles
// per wave that keeps 128 KB of q loads in flight per CU, which measured faster
// than three workgroups of four tiles per wave.
template <int TPW, bool BIGK, typename IdxT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 4))) void sa_mult_kernel(MultParams p) {
  const IdxT* const idx = static_cast<const IdxT*>(p.idx);
  __shared__ u32x4 kraw[32 * 16];  // kv row r chunk c (8 channels) at r*16 + (c ^ (r & 15))
  __shared__ u32x4 img_pv[8][64];  // fragment mt: kv[pi(8g+j)][delta(mt, n)], j = 0..7
  __shared__ u32x4 obuf[4][256];   // per-wave output tile, 16 rows x 16 chunks, chunk ^ row
  const int lane = threadIdx.x & 63;
  const int wi = threadIdx.x >> 6;
  const int n = lane & 15;  // row of the tile (head h0 + n) = MFMA column
  const int g = lane >> 4;  // lane group: contraction slice 8g..8g+7
  const int b = (int)(blockIdx.x / p.blocks_per_batch);
  const int64_t lt0 = ((blockIdx.x % p.blocks_per_batch) * 4 + wi) * TPW;  // first tile in batch b
  const int tpt = p.H >> 4;  // 16-row tiles per token
  const int64_t ntb = p.tiles_per_batch;
  const bool live = lt0 < ntb;
  const int nlive = live ? (int)((ntb - lt0) < TPW ? (ntb - lt0) : TPW) : 0;  // tiles of this wave

  // Token and head block of each tile, from one division per wave. Dead tiles
  // repeat the wave's last live tile so that every load below is unconditional
  // (vector-memory waits are then exact counts of the loads issued later).
  int64_t tok[TPW];
  int h0[TPW];
  {
    const int64_t first = live ? lt0 : ntb - 1;
    int64_t tk = (int64_t)b * p.M + first / tpt;
    int hh = (int)(first % tpt);
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      if (i > 0 && i < nlive) {
        if (++hh == tpt) {
          hh = 0;
          ++tk;
        }
      }
      tok[i] = tk;
      h0[i] = hh * 16;
    }
  }

  // 0. kv block of batch b: 32 rows x 16 chunks, two 16-byte chunks per thread.
  const uint16_t* kvb = p.kv + (int64_t)b * p.NKV * kD;
  u32x4 kr[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int e = threadIdx.x + 256 * j, r = e >> 4, c = e & 15;
    const int rr = r < p.NKV ? r : p.NKV - 1;
    kr[j] = *reinterpret_cast<const u32x4*>(kvb + (int64_t)rr * kD + 8 * c);
  }
  __builtin_amdgcn_sched_barrier(0);  // keep the issue order: kv, small values, q
  // 1. sink of this lane's head per tile; slot indices of the wave's tokens
  //    (token j of the wave is tok[0] + j; at most TPW of them).
  float skv[TPW];
  int idxv[TPW];
  const int64_t tok_last = tok[TPW - 1];
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    skv[i] = p.sink[h0[i] + n];
    const int64_t tj = tok[0] + i < tok_last ? tok[0] + i : tok_last;
    idxv[i] = slot_index(idx, tj * p.TOPK + (lane < p.TOPK ? lane : p.TOPK - 1));
  }
  __builtin_amdgcn_sched_barrier(0);
  // 2. q loads of all this wave's tiles.
  bf16x8 qv[TPW][4];
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const uint16_t* a = p.q + (tok[i] * p.H + h0[i] + n) * kD + 8 * g;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qv[i][ks] = load_row16(a + 32 * ks);
  }
  // 3. stage kv in LDS (rows >= n_kv zero), then build the operand image of
  //    the second product from it.
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int e = threadIdx.x + 256 * j, r = e >> 4, c = e & 15;
    kraw[r * 16 + (c ^ (r & 15))] = (r < p.NKV) ? kr[j] : u32x4{0u, 0u, 0u, 0u};
  }
  __syncthreads();
  {
    const uint16_t* kh = reinterpret_cast<const uint16_t*>(kraw);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int e = threadIdx.x + 256 * j, f = e >> 6, ln = e & 63, nn = ln & 15, gg = ln >> 4;
      const int ch = delta_ch(f, nn), cc = ch >> 3, ce = ch & 7;
      u32x4 w;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int r0 = pi_kv(8 * gg + 2 * jj), r1 = pi_kv(8 * gg + 2 * jj + 1);
        const uint32_t v0 = kh[(r0 * 16 + (cc ^ (r0 & 15))) * 8 + ce];
        const uint32_t v1 = kh[(r1 * 16 + (cc ^ (r1 & 15))) * 8 + ce];
        w[jj] = v0 | (v1 << 16);
      }
      img_pv[f][ln] = w;
    }
  }
  __syncthreads();
  if (!live) return;

  float cnt[8];   // multiplicities of kv rows 16mt + 4g + r (index mt*4 + r)
  bool used[8];   // cnt > 0
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    if (i >= nlive) break;
    if (i == 0 || tok[i] != tok[i - 1]) {
      // Histogram of the token's slots over kv rows 0..31 with wave ballots;
      // each lane keeps the eight counts of the rows it owns in the S^T layout.
      int c[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) c[k] = 0;
      const int jt = (int)(tok[i] - tok[0]);
      for (int c0 = 0; c0 < (BIGK ? p.TOPK : 1); c0 += 64) {
        int v = -1;
        if (c0 == 0) {
#pragma unroll
          for (int q = 0; q < TPW; ++q)
            if (q == jt && lane < p.TOPK) v = idxv[q];
        } else if (c0 + lane < p.TOPK) {  // only for topk > 64
          v = slot_index(idx, tok[i] * p.TOPK + c0 + lane);
        }
        if (v >= p.NKV) v = -1;  // out-of-range slots are ignored (masked)
#pragma unroll
        for (int k = 0; k < 32; ++k) {
          const int ck = __popcll(__ballot(v == k));
          if (g == ((k >> 2) & 3)) c[(k >> 4) * 4 + (k & 3)] += ck;
        }
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        cnt[k] = (float)c[k];
        used[k] = c[k] > 0;
      }
    }

    // S^T tiles: kv rows 0..15 and 16..31 against the 16 rows of this tile.
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      // A operand: chunk 4ks+g of kv row 16mt+n (row & 15 == n)
      s0 = mfma16x16x32(__builtin_bit_cast(bf16x8, kraw[n * 16 + ((4 * ks + g) ^ n)]), qv[i][ks], s0);
      s1 = mfma16x16x32(__builtin_bit_cast(bf16x8, kraw[(16 + n) * 16 + ((4 * ks + g) ^ n)]), qv[i][ks], s1);
    }
    float sv[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sv[r] = s0[r] * p.scale;
      sv[4 + r] = s1[r] * p.scale;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (used[k]) mx = fmaxf(mx, sv[k]);
    mx = fmaxf(mx, shfl_xor_f(mx, 16));
    mx = fmaxf(mx, shfl_xor_f(mx, 32));
    const float sk = skv[i];
    const int64_t tk = tok[i];
    const float mrow = fmaxf(mx, sk);
    float e[8];
    float z = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      e[k] = used[k] ? __expf(sv[k] - mrow) * cnt[k] : 0.f;
      z += e[k];
    }
    z += shfl_xor_f(z, 16);
    z += shfl_xor_f(z, 32);
    z += __expf(sk - mrow);
    const float rz = __builtin_amdgcn_rcpf(z);
    // P = hi + lo + lo2: hi = bf16(p), lo = bf16(p - hi), lo2 = bf16(p - hi - lo)
    // (both differences exact in fp32). With two terms P kept ~16 bits and 0.19 %
    // of the configs[1] outputs differed from the reference's fp32 path by one
    // bf16 ulp; with three, 0.011 %. The third products are free here: the
    // kernel is bound by HBM, its matrix cores ~10 % busy.
    u32x4 whi, wlo, wlo2;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float p0 = e[2 * w] * rz, p1 = e[2 * w + 1] * rz;
      const uint32_t h = pack_bf2(p0, p1);
      whi[w] = h;
      const float r0 = p0 - bf_lo(h), r1 = p1 - bf_hi(h);
      const uint32_t l = pack_bf2(r0, r1);
      wlo[w] = l;
      wlo2[w] = pack_bf2(r0 - bf_lo(l), r1 - bf_hi(l));
    }
    const bf16x8 phi = __builtin_bit_cast(bf16x8, whi);
    const bf16x8 plo = __builtin_bit_cast(bf16x8, wlo);
    const bf16x8 plo2 = __builtin_bit_cast(bf16x8, wlo2);

    // O^T = KV^T . P^T, smallest part first, into one accumulator.
    f32x4 o[8];
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) {
      const bf16x8 a = __builtin_bit_cast(bf16x8, img_pv[mt][lane]);
      o[mt] = mfma16x16x32(a, plo2, f32x4{0.f, 0.f, 0.f, 0.f});
      o[mt] = mfma16x16x32(a, plo, o[mt]);
      o[mt] = mfma16x16x32(a, phi, o[mt]);
    }
    // Transpose the tile through LDS so every store instruction writes four
    // whole 256-byte rows (1 KB contiguous) instead of 16 rows x 64 bytes.
    u32x4* ob = obuf[wi];
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      u32x4 w;
      w[0] = pack_bf2(o[2 * pp][0], o[2 * pp][1]);
      w[1] = pack_bf2(o[2 * pp][2], o[2 * pp][3]);
      w[2] = pack_bf2(o[2 * pp + 1][0], o[2 * pp + 1][1]);
      w[3] = pack_bf2(o[2 * pp + 1][2], o[2 * pp + 1][3]);
      ob[n * 16 + ((4 * pp + g) ^ n)] = w;  // chunk 4pp+g of row n
    }
    wave_lds_sync();
    u32x4* dst = reinterpret_cast<u32x4*>(p.out + (tk * p.H + h0[i]) * kD);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int r = 4 * k + (lane >> 4), c = lane & 15;
      const u32x4 w = ob[r * 16 + (c ^ r)];
#if DSA_SA_NT_STORE
      st_nt(dst + r * 16 + c, w);
#else
      dst[r * 16 + c] = w;
#endif
    }
    wave_lds_sync();
  }
}

}  // namespace

namespace dsa_host {
// The CU count of each device, queried once. Relaxed atomics: threads that race
// on the first call of a device store the same value.
int device_cu_count(int* out) {
  static std::atomic<int> cached[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return DSA_ERR_DEVICE;
  int cu = cached[dev].load(std::memory_order_relaxed);
  if (cu <= 0) {
    if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cu <= 0)
      return DSA_ERR_DEVICE;
    cached[dev].store(cu, std::memory_order_relaxed);
  }
  *out = cu;
  return DSA_OK;
}

// hipFuncSetAttribute(MaxDynamicSharedMemorySize) once per (kernel, device) and
// size: the limit only ever grows, and a launch asking for no more than what was
// set skips the runtime call (it costs microseconds per launch otherwise).
int ensure_dyn_lds(const void* fn, int bytes) {
  struct Entry {
    const void* fn;
    int dev;
    int bytes;
  };
  static std::mutex mu;
  static Entry tab[256];
  static int n = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return DSA_ERR_DEVICE;
  std::lock_guard<std::mutex> lock(mu);
  Entry* e = nullptr;
  for (int i = 0; i < n; ++i)
    if (tab[i].fn == fn && tab[i].dev == dev) e = &tab[i];
  if (e != nullptr && e->bytes >= bytes) return DSA_OK;
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess)
    return DSA_ERR_LAUNCH;
  if (e != nullptr) e->bytes = bytes;
  else if (n < 256) tab[n++] = Entry{fn, dev, bytes};
  return DSA_OK;
}
}  // namespace dsa_host

extern "C" int dsa_abi_version(void) { return DSA_ABI_VERSION; }

extern "C" const char* dsa_strerror(int code) {
  switch (code) {
    case DSA_OK: return "ok";
    case DSA_ERR_NULL: return "null pointer argument";
    case DSA_ERR_SHAPE: return "invalid or inconsistent sizes";
    case DSA_ERR_UNSUPPORTED: return "configuration not supported by this build";
    case DSA_ERR_LAUNCH: return "kernel launch failed";
    case DSA_ERR_DEVICE: return "device query failed";
    case DSA_ERR_ALIGN: return "pointer not 16-byte aligned";
    case DSA_ERR_SCRATCH: return "request exceeds the library's static scratch buffer";
    default: return "unknown error";
  }
}

int dsa_sparse_attn_gather_launch(const void* q, const void* kv, const void* idx, bool idx64,
                                  const float* sink, void* out, int64_t b, int64_t m, int64_t h,
                                  int64_t n_kv, int64_t topk, float scale, hipStream_t stream);

namespace {

// Shared by dsa_sparse_attn_fwd (int32 indices) and dsa_sparse_attn_fwd_i64.
int sparse_attn_fwd(const void* q, const void* kv, const void* topk_idxs, bool idx64,
                    const float* attn_sink, void* out, int64_t b, int64_t m, int64_t h, int64_t d,
                    int64_t n_kv, int64_t topk, float softmax_scale, int32_t variant, void* stream) {
  if (b < 0 || m < 0 || h <= 0 || d <= 0 || n_kv < 1 || topk < 1) return DSA_ERR_SHAPE;
  if (d != kD || (h % 16) != 0) return DSA_ERR_UNSUPPORTED;
  if (variant == DSA_SA_AUTO) variant = (n_kv <= 32) ? DSA_SA_MULTIPLICITY : DSA_SA_GATHER;
  if (variant != DSA_SA_MULTIPLICITY && variant != DSA_SA_GATHER) return DSA_ERR_UNSUPPORTED;
  if (variant == DSA_SA_MULTIPLICITY && n_kv > 32) return DSA_ERR_UNSUPPORTED;
  if (h > (1 << 20) || n_kv > (1 << 30) || topk > (1 << 30) || m > (INT64_C(1) << 40) ||
      b > (1 << 20))
    return DSA_ERR_SHAPE;
  if (b == 0 || m == 0) return DSA_OK;
  if (!q || !kv || !topk_idxs || !attn_sink || !out) return DSA_ERR_NULL;
  if (!dsa_host::aligned16(q) || !dsa_host::aligned16(kv) || !dsa_host::aligned16(out))
    return DSA_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  if (variant == DSA_SA_GATHER)
    return dsa_sparse_attn_gather_launch(q, kv, topk_idxs, idx64, attn_sink, out, b, m, h, n_kv,
                                         topk, softmax_scale, s);

  MultParams p;
  p.q = (const uint16_t*)q;
  p.kv = (const uint16_t*)kv;
  p.idx = topk_idxs;
  p.sink = attn_sink;
  p.out = (uint16_t*)out;
  p.M = m;
  p.H = (int32_t)h;
  p.NKV = (int32_t)n_kv;
  p.TOPK = (int32_t)topk;
  p.scale = softmax_scale;
  p.tiles_per_batch = m * (h / 16);
  constexpr int tiles_per_block = 4 * DSA_SA_TILES_PER_WAVE;
  p.blocks_per_batch = (p.tiles_per_batch + tiles_per_block - 1) / tiles_per_block;
  const int64_t blocks = b * p.blocks_per_batch;
  if (blocks > INT32_MAX) return DSA_ERR_SHAPE;
  const dim3 grid((unsigned)blocks);
  if (idx64) {
    if (topk <= 64)
      hipLaunchKernelGGL((sa_mult_kernel<DSA_SA_TILES_PER_WAVE, false, int64_t>), grid, dim3(256), 0, s, p);
    else
      hipLaunchKernelGGL((sa_mult_kernel<DSA_SA_TILES_PER_WAVE, true, int64_t>), grid, dim3(256), 0, s, p);
  } else {
    if (topk <= 64)
      hipLaunchKernelGGL((sa_mult_kernel<DSA_SA_TILES_PER_WAVE, false, int32_t>), grid, dim3(256), 0, s, p);
    else
      hipLaunchKernelGGL((sa_mult_kernel<DSA_SA_TILES_PER_WAVE, true, int32_t>), grid, dim3(256), 0, s, p);
  }
  return hipGetLastError() == hipSuccess ? DSA_OK : DSA_ERR_LAUNCH;
}

}  // namespace

extern "C" int dsa_sparse_attn_fwd(const void* q, const void* kv, const int32_t* topk_idxs,
                                   const float* attn_sink, void* out, int64_t b, int64_t m,
                                   int64_t h, int64_t d, int64_t n_kv, int64_t topk,
                                   float softmax_scale, int32_t variant, void* stream) {
  return sparse_attn_fwd(q, kv, topk_idxs, false, attn_sink, out, b, m, h, d, n_kv, topk,
                         softmax_scale, variant, stream);
}

extern "C" int dsa_sparse_attn_fwd_i64(const void* q, const void* kv, const int64_t* topk_idxs,
                                       const float* attn_sink, void* out, int64_t b, int64_t m,
                                       int64_t h, int64_t d, int64_t n_kv, int64_t topk,
                                       float softmax_scale, int32_t variant, void* stream) {
  return sparse_attn_fwd(q, kv, topk_idxs, true, attn_sink, out, b, m, h, d, n_kv, topk,
                         softmax_scale, variant, stream);
}
