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
//   P             = c_j * exp(S - M) / Z, fp32, split hi + lo bf16
//   O^T[128 x 16] = KV^T[128 x 32] . (P_hi + P_lo)^T    (16 x mfma 16x16x32)
// The kv block of the current batch lives in registers in both operand
// layouts, so S and P never leave the CU. The contraction indices of both
// products are permuted (pi over kv rows, delta over channels) so that the
// softmax output is already in the B-operand layout of the second product and
// every lane loads and stores 16 contiguous bytes of a row.
#include "dsa_common.h"

using namespace dsa;

namespace {

constexpr int kD = 128;

struct MultParams {
  const uint16_t* q;
  const uint16_t* kv;
  const int32_t* idx;
  const float* sink;
  uint16_t* out;
  int64_t M;  // tokens per batch
  int32_t H;
  int32_t NKV;
  int32_t TOPK;
  float scale;
  int64_t total_tiles;
  int64_t tiles_per_wave;
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

__device__ __forceinline__ bf16x8 load_row16(const uint16_t* p) {
  return __builtin_bit_cast(bf16x8, ld_nt(reinterpret_cast<const u32x4*>(p)));
}

__global__ __launch_bounds__(256) void sa_mult_kernel(MultParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t t0 = wave * p.tiles_per_wave;
  const int64_t t1 = t0 + p.tiles_per_wave < p.total_tiles ? t0 + p.tiles_per_wave : p.total_tiles;
  if (t0 >= t1) return;

  const int n = lane & 15;  // row of the tile (head h0 + n) = MFMA column
  const int g = lane >> 4;  // lane group: contraction slice 8g..8g+7
  const int tpt = p.H >> 4; // 16-row tiles per token

  bf16x8 kqk[2][4];  // A operand of S^T: kv[16mt + n][32ks + 8g + j]
  bf16x8 kpv[8];     // A operand of O^T: kv[pi(8g + j)][delta(mt, n)]
  float cnt[8];      // multiplicities of kv rows 16mt + 4g + r (index mt*4 + r)
  int cur_b = -1;
  int64_t cur_tok = -1;

  auto qaddr = [&](int64_t tile) -> const uint16_t* {
    const int64_t tok = tile / tpt;
    const int64_t row = tok * p.H + (tile - tok * tpt) * 16 + n;
    return p.q + row * kD + 8 * g;
  };

  bf16x8 qv[4];
  {
    const uint16_t* a = qaddr(t0);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qv[ks] = load_row16(a + 32 * ks);
  }

  for (int64_t tile = t0; tile < t1; ++tile) {
    const int64_t tok = tile / tpt;
    const int h0 = (int)(tile - tok * tpt) * 16;
    const int b = (int)(tok / p.M);

    if (b != cur_b) {
      const uint16_t* kvb = p.kv + (int64_t)b * p.NKV * kD;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const int r = 16 * mt + n;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          if (r < p.NKV) {
            kqk[mt][ks] = __builtin_bit_cast(
                bf16x8, *reinterpret_cast<const u32x4*>(kvb + (int64_t)r * kD + 32 * ks + 8 * g));
          } else {
            kqk[mt][ks] = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
          }
        }
      }
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) {
        const int ch = delta_ch(mt, n);
        uint16_t v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int r = pi_kv(8 * g + j);
          v[j] = (r < p.NKV) ? kvb[(int64_t)r * kD + ch] : (uint16_t)0;
        }
        u32x4 w;
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = (uint32_t)v[2 * j] | ((uint32_t)v[2 * j + 1] << 16);
        kpv[mt] = __builtin_bit_cast(bf16x8, w);
      }
      cur_b = b;
    }

    if (tok != cur_tok) {
      // Histogram of the token's slots over kv rows 0..31 with wave ballots;
      // each lane keeps the eight counts of the rows it owns in the S^T layout.
      int c[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) c[i] = 0;
      const int32_t* ip = p.idx + tok * p.TOPK;
      for (int c0 = 0; c0 < p.TOPK; c0 += 64) {
        int v = -1;
        if (c0 + lane < p.TOPK) v = ip[c0 + lane];
        if (v >= p.NKV) v = -1;  // out-of-range slots are ignored (masked)
#pragma unroll
        for (int k = 0; k < 32; ++k) {
          const int ck = __popcll(__ballot(v == k));
          if (g == ((k >> 2) & 3)) c[(k >> 4) * 4 + (k & 3)] += ck;
        }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) cnt[i] = (float)c[i];
      cur_tok = tok;
    }

    // Prefetch the next tile's q while this one is computed.
    bf16x8 qn[4];
    const bool has_next = tile + 1 < t1;
    if (has_next) {
      const uint16_t* a = qaddr(tile + 1);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) qn[ks] = load_row16(a + 32 * ks);
    }

    // S^T tiles: kv rows 0..15 and 16..31 against the 16 rows of this tile.
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      s0 = mfma16x16x32(kqk[0][ks], qv[ks], s0);
      s1 = mfma16x16x32(kqk[1][ks], qv[ks], s1);
    }
    float sv[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sv[r] = s0[r] * p.scale;
      sv[4 + r] = s1[r] * p.scale;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (cnt[i] > 0.f) mx = fmaxf(mx, sv[i]);
    mx = fmaxf(mx, shfl_xor_f(mx, 16));
    mx = fmaxf(mx, shfl_xor_f(mx, 32));
    const float sk = p.sink[h0 + n];
    const float mrow = fmaxf(mx, sk);
    float e[8];
    float z = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      e[i] = (cnt[i] > 0.f) ? __expf(sv[i] - mrow) * cnt[i] : 0.f;
      z += e[i];
    }
    z += shfl_xor_f(z, 16);
    z += shfl_xor_f(z, 32);
    z += __expf(sk - mrow);
    const float rz = 1.0f / z;
    u32x4 whi, wlo;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float p0 = e[2 * w] * rz, p1 = e[2 * w + 1] * rz;
      const uint32_t h = pack_bf2(p0, p1);
      whi[w] = h;
      wlo[w] = pack_bf2(p0 - bf_lo(h), p1 - bf_hi(h));
    }
    const bf16x8 phi = __builtin_bit_cast(bf16x8, whi);
    const bf16x8 plo = __builtin_bit_cast(bf16x8, wlo);

    // O^T = KV^T . P^T, low part first then high part into the same accumulator.
    f32x4 o[8];
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) {
      o[mt] = mfma16x16x32(kpv[mt], plo, f32x4{0.f, 0.f, 0.f, 0.f});
      o[mt] = mfma16x16x32(kpv[mt], phi, o[mt]);
    }
    {
      const int64_t row = tok * p.H + h0 + n;
      uint16_t* dst = p.out + row * kD + 8 * g;
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) {
        u32x4 w;
        w[0] = pack_bf2(o[2 * pp][0], o[2 * pp][1]);
        w[1] = pack_bf2(o[2 * pp][2], o[2 * pp][3]);
        w[2] = pack_bf2(o[2 * pp + 1][0], o[2 * pp + 1][1]);
        w[3] = pack_bf2(o[2 * pp + 1][2], o[2 * pp + 1][3]);
        st_nt(reinterpret_cast<u32x4*>(dst + 32 * pp), w);
      }
    }

    if (has_next) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) qv[ks] = qn[ks];
    }
  }
}

}  // namespace

namespace dsa_host {
int device_cu_count(int* out) {
  static int cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return DSA_ERR_DEVICE;
  if (cached[dev] <= 0) {
    int cu = 0;
    if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cu <= 0)
      return DSA_ERR_DEVICE;
    cached[dev] = cu;
  }
  *out = cached[dev];
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
    default: return "unknown error";
  }
}

int dsa_sparse_attn_gather_launch(const void* q, const void* kv, const int32_t* idx, const float* sink,
                                  void* out, int64_t b, int64_t m, int64_t h, int64_t n_kv,
                                  int64_t topk, float scale, hipStream_t stream);

extern "C" int dsa_sparse_attn_fwd(const void* q, const void* kv, const int32_t* topk_idxs,
                                   const float* attn_sink, void* out, int64_t b, int64_t m,
                                   int64_t h, int64_t d, int64_t n_kv, int64_t topk,
                                   float softmax_scale, int32_t variant, void* stream) {
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
    return dsa_sparse_attn_gather_launch(q, kv, topk_idxs, attn_sink, out, b, m, h, n_kv, topk,
                                         softmax_scale, s);

  int cu = 0;
  int rc = dsa_host::device_cu_count(&cu);
  if (rc != DSA_OK) return rc;
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
  p.total_tiles = b * m * (h / 16);
  const int64_t waves = (int64_t)cu * 16;
  p.tiles_per_wave = (p.total_tiles + waves - 1) / waves;
  const int64_t used_waves = (p.total_tiles + p.tiles_per_wave - 1) / p.tiles_per_wave;
  const int64_t blocks = (used_waves + 3) / 4;
  hipLaunchKernelGGL(sa_mult_kernel, dim3((unsigned)blocks), dim3(256), 0, s, p);
  return hipGetLastError() == hipSuccess ? DSA_OK : DSA_ERR_LAUNCH;
}
