// Per-row part of the absorbed-MLA decode preparation, shared by mla_prepare_kernel
// (mla.hip) and the one-launch prepare + q_lat absorption of the batch family (gemm.hip):
// RoPE(q_pe) of the 16 heads into columns 512..575 of the query rows, and the token's new
// cache row (kv-norm of the 512-wide latent, RoPE(k_pe)) at its position.
#pragma once
#include "common.h"

struct MlaRowArgs {
  const bf16_t* qkva;  // [rows, qs]: q (16 x 192: 128 nope + 64 pe) | latent (512) | k_pe (64)
  int64_t qs;
  const int32_t* pos;
  const int64_t* base;
  const int32_t* cap;
  const bf16_t* kvw;   // kv-norm weight [512]
  float eps;
  const bf16_t* cosT;  // [max_pos, 64]
  const bf16_t* sinT;
  int max_pos;
  bf16_t* cache;       // compressed cache rows of 576 (512 latent + 64 rotated k_pe)
  bf16_t* qout;        // [rows, 16, 576]
  int32_t* status;
};

// Row b on 256 threads t = 0..255 (t < 64: one whole wave, for the latent's norm).  A position
// outside [0, cap) would land in another row's cache slots: the row is skipped and the status
// word flagged.  Two dependent load round trips: the position with every operand that does not
// depend on it, then the cos / sin entries at that position (thread t's two (head, pair) items
// and, for t < 32, k_pe's pair t share the same four).  RoPE on de-interleaved pairs:
// out[i] = e cos[i] - o sin[i], out[32 + i] = o cos[32 + i] + e sin[32 + i] with (e, o) =
// (x[2i], x[2i + 1]), fp32 math, one bf16 round.
__device__ __forceinline__ void mla_prepare_row(const MlaRowArgs& m, int b, int t) {
  constexpr int kHeadsR = 16, kRowR = 576, kLatR = 512;
  const int pb = m.pos[b], cb = m.cap[b];
  const int64_t bb = m.base[b];
  const bf16_t* q = m.qkva + b * m.qs;
  const int tt = t & 31;
  // (head, pair) items t and t + 256: heads t >> 5 and 8 + (t >> 5), pair tt
  uint32_t xq[2];
#pragma unroll
  for (int k = 0; k < 2; ++k)
    xq[k] = *reinterpret_cast<const uint32_t*>(q + ((t + 256 * k) >> 5) * 192 + 128 + 2 * tt);
  uint4 lat = make_uint4(0u, 0u, 0u, 0u), g4 = lat;
  uint32_t kpe = 0u;
  if (t < 64) {
    lat = ldg16(q + 3072 + t * 8);
    g4 = ldg16(m.kvw + t * 8);
    kpe = *reinterpret_cast<const uint32_t*>(q + 3584 + 2 * tt);
  }
  const int p = pb < 0 ? 0 : (pb >= m.max_pos ? m.max_pos - 1 : pb);
  const bf16_t* cs = m.cosT + (int64_t)p * 64;
  const bf16_t* sn = m.sinT + (int64_t)p * 64;
  const float c0 = bf2f(cs[tt]), c1 = bf2f(cs[32 + tt]), s0 = bf2f(sn[tt]), s1 = bf2f(sn[32 + tt]);
  // RoPE(q_pe) of the 16 heads
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int h = (t + 256 * k) >> 5;
    const float e = __uint_as_float(xq[k] << 16), o = __uint_as_float(xq[k] & 0xffff0000u);
    bf16_t* out = m.qout + ((int64_t)b * kHeadsR + h) * kRowR + kLatR;
    out[tt] = f2bf(e * c0 - o * s0);
    out[32 + tt] = f2bf(o * c1 + e * s1);
  }
  if (t < 64) {
    const int lane = t;
    float f[8], g[8];
    unpack8(lat, f);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(f[i], f[i], ss);
    ss = wave_sum(ss);
    const float rs = rsqrtf(ss / static_cast<float>(kLatR) + m.eps);
    unpack8(g4, g);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = g[i] * rbf(f[i] * rs);
    if (pb < 0 || pb >= cb) {
      if (lane == 0 && m.status) atomicOr(m.status, DSV2_DEVERR_CACHE_FULL);
      return;
    }
    bf16_t* crow = m.cache + (bb + pb) * kRowR;
    *reinterpret_cast<uint4*>(crow + lane * 8) = pack8(f);
    if (lane < 32) {
      const float e = __uint_as_float(kpe << 16), o = __uint_as_float(kpe & 0xffff0000u);
      crow[kLatR + lane] = f2bf(e * c0 - o * s0);
      crow[kLatR + 32 + lane] = f2bf(o * c1 + e * s1);
    }
  }
}
