// Per-row part of the absorbed-MLA decode preparation, shared by mla_prepare_kernel
// (mla.hip) and the one-launch prepare + q_lat absorption of the batch family (gemm.hip):
// RoPE(q_pe) of the 16 heads into columns 512..575 of the query rows, and the token's new
// cache row (kv-norm of the 512-wide latent, RoPE(k_pe)) at its position.
#pragma once
#include "common.h"

// RoPE on de-interleaved pairs: out[t] = e*cos[t] - o*sin[t], out[32+t] = o*cos[32+t] + e*sin[32+t]
// (e, o = x[2t], x[2t+1]); lanes 0..31 each produce one pair.  fp32 math, one bf16 round.
__device__ __forceinline__ void rope_pair(const bf16_t* x, const bf16_t* cs, const bf16_t* sn, bf16_t* out, int t) {
  const float e = bf2f(x[2 * t]), o = bf2f(x[2 * t + 1]);
  out[t] = f2bf(e * bf2f(cs[t]) - o * bf2f(sn[t]));
  out[32 + t] = f2bf(o * bf2f(cs[32 + t]) + e * bf2f(sn[32 + t]));
}

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
// word flagged.
__device__ __forceinline__ void mla_prepare_row(const MlaRowArgs& m, int b, int t) {
  constexpr int kHeadsR = 16, kRowR = 576, kLatR = 512;
  int p = m.pos[b];
  p = p < 0 ? 0 : (p >= m.max_pos ? m.max_pos - 1 : p);
  const bf16_t* q = m.qkva + b * m.qs;
  const bf16_t* cs = m.cosT + (int64_t)p * 64;
  const bf16_t* sn = m.sinT + (int64_t)p * 64;
  // RoPE(q_pe) of the 16 heads: 512 (head, pair) items over 256 threads
  for (int it = t; it < kHeadsR * 32; it += 256) {
    const int h = it >> 5, tt = it & 31;
    rope_pair(q + h * 192 + 128, cs, sn, m.qout + ((int64_t)b * kHeadsR + h) * kRowR + kLatR, tt);
  }
  if (t < 64) {
    const int lane = t;
    float f[8], g[8];
    unpack8(ldg16(q + 3072 + lane * 8), f);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(f[i], f[i], ss);
    ss = wave_sum(ss);
    const float rs = rsqrtf(ss / static_cast<float>(kLatR) + m.eps);
    unpack8(ldg16(m.kvw + lane * 8), g);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = g[i] * rbf(f[i] * rs);
    if (m.pos[b] < 0 || m.pos[b] >= m.cap[b]) {
      if (lane == 0 && m.status) atomicOr(m.status, DSV2_DEVERR_CACHE_FULL);
      return;
    }
    bf16_t* crow = m.cache + (m.base[b] + m.pos[b]) * kRowR;
    *reinterpret_cast<uint4*>(crow + lane * 8) = pack8(f);
    if (lane < 32) rope_pair(q + 3584, cs, sn, crow + kLatR, lane);
  }
}
