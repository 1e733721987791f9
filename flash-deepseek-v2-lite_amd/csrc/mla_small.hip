// Fused absorbed-MLA decode for a few rows (the small family): one 1024-thread
// workgroup per (row, head) does the whole head:
//   1. q_lat_h = W_UK_h^T q_nope_h        (16 lanes per output)
//   2. new cache row (kv-norm + RoPE(k_pe)) into LDS; the h == 0 workgroup stores it
//   3. RoPE(q_pe_h); per-wave online softmax over kBatch-token batches of the cached rows
//      (a lane's 16-byte latent load serves both q.k and p.v, plus one rope element), the
//      new token from LDS
//   4. log-sum-exp merge of the 16 waves -> o_lat_h (fp32)
//   5. attn[row, h*128 + i] = W_UV_h o_lat_h
// Every load that depends on nothing -- W_UK, q, the new row's inputs and each wave's first
// batch of cached rows -- is requested at entry, so the kernel pays one memory round trip
// before the attention instead of three; W_UV is requested when the attention loop ends and
// arrives while the waves are merged.  Replaces prepare + split decode + combine (three
// launches) when the batch is small.
#include "common.h"

namespace {
constexpr int kRow = 576, kLat = 512, kWaves = 16, kBatch = 4;
}

__global__ __launch_bounds__(1024) void mla_fused_kernel(const bf16_t* __restrict__ qkva, int64_t qs,
                                                         const int32_t* __restrict__ pos,
                                                         const int64_t* __restrict__ base,
                                                         const int32_t* __restrict__ cap,
                                                         const bf16_t* __restrict__ kvw, float eps,
                                                         const bf16_t* __restrict__ cosT,
                                                         const bf16_t* __restrict__ sinT, int max_pos,
                                                         const bf16_t* __restrict__ w_ukt,
                                                         const bf16_t* __restrict__ w_uv, bf16_t* __restrict__ cache,
                                                         float scale_log2, bf16_t* __restrict__ out, int64_t os,
                                                         int32_t* __restrict__ status) {
  __shared__ float qv[kRow];    // q_lat (bf16-rounded) | rotated q_pe
  __shared__ float nrow[kRow];  // the new token's cache row
  __shared__ float wm[kWaves], wl[kWaves];
  __shared__ float wo[kWaves][kLat];
  __shared__ float olat[kLat];
  const int b = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const bf16_t* q = qkva + b * qs;
  // the new token goes to slot pos; the row owns slots [0, cap): a position at or past cap
  // attends the cap cached rows, is not stored, and sets DSV2_DEVERR_CACHE_FULL
  const int pr = pos[b], cp = cap[b];
  const bool fits = pr >= 0 && pr < cp;
  const int p = pr < 0 ? 0 : (pr > cp ? cp : pr);  // cached rows read: [0, p)
  const int pc = p >= max_pos ? max_pos - 1 : p;
  const bf16_t* cs = cosT + (int64_t)pc * 64;
  const bf16_t* sn = sinT + (int64_t)pc * 64;
  const bf16_t* crow0 = cache + base[b] * kRow;

  // ---- entry loads -------------------------------------------------------------------
  // absorption: thread (gi = tid / 16, k = tid % 16) owns rows u*64 + gi of W_UKT_h, K slice k
  const int gi = tid >> 4, k = tid & 15;
  const uint4 qn4 = ldg16(q + h * 192 + k * 8);
  uint4 wr[8];
  {
    const bf16_t* wk = w_ukt + ((int64_t)h * kLat + gi) * 128 + k * 8;
#pragma unroll
    for (int u = 0; u < 8; ++u) wr[u] = ldg16(wk + (int64_t)u * 64 * 128);
  }
  // this wave's first batch of cached rows (rows clamped into [0, p-1]; rows past p are
  // masked out of the softmax): lane l holds latent elements 8l..8l+7 and rope element l
  uint4 va[kBatch];
  bf16_t vr[kBatch];
  const int t_first = wv * kBatch;
#pragma unroll
  for (int u = 0; u < kBatch; ++u) {
    const int t = max(min(t_first + u, p - 1), 0);
    va[u] = ldg16(crow0 + (int64_t)t * kRow + lane * 8);
    vr[u] = crow0[(int64_t)t * kRow + kLat + lane];
  }
  // new row (wave 0) / q_pe (wave 1) inputs
  uint4 kv4 = {0u, 0u, 0u, 0u}, kw4 = {0u, 0u, 0u, 0u};
  float re = 0.f, ro = 0.f, c0 = 0.f, c1 = 0.f, s0 = 0.f, s1 = 0.f;
  if (wv <= 1) {
    if (wv == 0) {
      kv4 = ldg16(q + 3072 + lane * 8);
      kw4 = ldg16(kvw + lane * 8);
    }
    if (lane < 32) {
      const bf16_t* rp = wv == 0 ? q + 3584 : q + h * 192 + 128;
      re = bf2f(rp[2 * lane]);
      ro = bf2f(rp[2 * lane + 1]);
      c0 = bf2f(cs[lane]);
      c1 = bf2f(cs[32 + lane]);
      s0 = bf2f(sn[lane]);
      s1 = bf2f(sn[32 + lane]);
    }
  }

  // ---- 1. absorption ----------------------------------------------------------------
  {
    float qn[8];
    unpack8(qn4, qn);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      float sdot = dot8(wr[u], qn);
      sdot += __shfl_xor(sdot, 8, 64);
      sdot += __shfl_xor(sdot, 4, 64);
      sdot += __shfl_xor(sdot, 2, 64);
      sdot += __shfl_xor(sdot, 1, 64);
      if (k == 0) qv[u * 64 + gi] = rbf(sdot);
    }
  }
  // ---- 2./3a. new row (wave 0) and RoPE(q_pe) (wave 1) --------------------------------
  if (wv == 0) {
    float f[8], g[8];
    unpack8(kv4, f);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(f[i], f[i], ss);
    ss = wave_sum(ss);
    const float rs = rsqrtf(ss / static_cast<float>(kLat) + eps);
    unpack8(kw4, g);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      f[i] = rbf(g[i] * rbf(f[i] * rs));
      nrow[lane * 8 + i] = f[i];
    }
    bf16_t* crow = cache + (base[b] + p) * kRow;
    const bool store = h == 0 && fits;
    if (h == 0 && !fits && lane == 0 && status) atomicOr(status, DSV2_DEVERR_CACHE_FULL);
    if (store) *reinterpret_cast<uint4*>(crow + lane * 8) = pack8(f);
    if (lane < 32) {
      const float v0 = rbf(re * c0 - ro * s0);
      const float v1 = rbf(ro * c1 + re * s1);
      nrow[kLat + lane] = v0;
      nrow[kLat + 32 + lane] = v1;
      if (store) {
        crow[kLat + lane] = f2bf(v0);
        crow[kLat + 32 + lane] = f2bf(v1);
      }
    }
  } else if (wv == 1 && lane < 32) {
    qv[kLat + lane] = rbf(re * c0 - ro * s0);
    qv[kLat + 32 + lane] = rbf(ro * c1 + re * s1);
  }
  __syncthreads();

  // ---- 3b. attention: wave wv takes token batches [wv*kBatch + n*kWaves*kBatch, +kBatch) --
  float qa[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) qa[i] = qv[lane * 8 + i];
  const float qb = qv[kLat + lane];
  float m = -INFINITY, l = 0.f, o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = 0.f;
  for (int t0 = t_first; t0 < p; t0 += kWaves * kBatch) {
    float sc[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) sc[u] = __builtin_fmaf(bf2f(vr[u]), qb, dot8(va[u], qa));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
#pragma unroll
      for (int u = 0; u < kBatch; ++u) sc[u] += __shfl_xor(sc[u], off, 64);
    float mx = m;
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      sc[u] = (t0 + u < p) ? sc[u] * scale_log2 : -INFINITY;
      mx = fmaxf(mx, sc[u]);
    }
    const float alpha = exp2f(m - mx);
    m = mx;
    l *= alpha;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] *= alpha;
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const float pu = exp2f(sc[u] - m);
      l += pu;
      float v[8];
      unpack8(va[u], v);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = __builtin_fmaf(pu, v[i], o[i]);
    }
    const int tn = t0 + kWaves * kBatch;
    if (tn < p) {
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int t = min(tn + u, p - 1);
        va[u] = ldg16(crow0 + (int64_t)t * kRow + lane * 8);
        vr[u] = crow0[(int64_t)t * kRow + kLat + lane];
      }
    }
  }
  // W_UV rows of step 5 (wave wv: rows wv*8 .. wv*8+7 of head h), in flight during the merge
  uint4 wuv[8];
  {
    const bf16_t* wp = w_uv + ((int64_t)h * 128 + wv * 8) * kLat + lane * 8;
#pragma unroll
    for (int r = 0; r < 8; ++r) wuv[r] = ldg16(wp + (int64_t)r * kLat);
  }
  if (wv == 0) {  // the new token (position p) from LDS
    float sp = qb * nrow[kLat + lane];
#pragma unroll
    for (int i = 0; i < 8; ++i) sp = __builtin_fmaf(qa[i], nrow[lane * 8 + i], sp);
    sp = wave_sum(sp) * scale_log2;
    const float mx = fmaxf(m, sp);
    const float alpha = exp2f(m - mx), pu = exp2f(sp - mx);
    m = mx;
    l = l * alpha + pu;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = o[i] * alpha + pu * nrow[lane * 8 + i];
  }
  if (lane == 0) {
    wm[wv] = m;
    wl[wv] = l;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) wo[wv][lane * 8 + i] = o[i];
  __syncthreads();

  // ---- 4. merge the waves -------------------------------------------------------------
  if (tid < kLat) {
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, wm[w]);
    float L = 0.f, acc = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float sc = exp2f(wm[w] - M);  // 0 for waves that saw no token
      L = __builtin_fmaf(wl[w], sc, L);
      acc = __builtin_fmaf(wo[w][tid], sc, acc);
    }
    olat[tid] = acc / L;
  }
  __syncthreads();

  // ---- 5. W_UV: wave wv computes rows wv*8 .. wv*8+7 of head h ------------------------
  float xo[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) xo[i] = olat[lane * 8 + i];
  float rr[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) rr[r] = dot8(wuv[r], xo);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
#pragma unroll
    for (int r = 0; r < 8; ++r) rr[r] += __shfl_xor(rr[r], off, 64);
  if (lane == 0) *reinterpret_cast<uint4*>(out + b * os + h * 128 + wv * 8) = pack8(rr);
}

extern "C" int dsv2_mla_fused(const void* qkva, int64_t qkva_stride, int rows, const int32_t* pos,
                              const int64_t* base, const int32_t* cap, const void* kv_norm_w, float eps,
                              const void* rope_cos, const void* rope_sin, int max_pos, const void* w_ukt,
                              const void* w_uv, void* cache, float softmax_scale, void* out, int64_t out_stride,
                              int32_t* status, void* stream) {
  DSV2_REQUIRE(qkva && pos && base && cap && kv_norm_w && rope_cos && rope_sin && w_ukt && w_uv && cache && out,
               DSV2_E_NULL,
               "mla_fused: null pointer");
  DSV2_REQUIRE(rows >= 0 && rows <= 65535 && max_pos > 0 && qkva_stride >= 3648, DSV2_E_SHAPE,
               "mla_fused: bad shape");
  DSV2_REQUIRE(dsv2_aligned16(qkva) && qkva_stride % 8 == 0 && dsv2_aligned16(kv_norm_w) && dsv2_aligned16(cache) &&
                   dsv2_aligned16(w_ukt) && dsv2_aligned16(w_uv) && dsv2_aligned16(out) && out_stride % 8 == 0,
               DSV2_E_ALIGN, "mla_fused: alignment");
  if (rows == 0) return DSV2_OK;
  hipLaunchKernelGGL(mla_fused_kernel, dim3(rows, 16), dim3(1024), 0, (hipStream_t)stream, (const bf16_t*)qkva,
                     qkva_stride, pos, base, cap, (const bf16_t*)kv_norm_w, eps, (const bf16_t*)rope_cos,
                     (const bf16_t*)rope_sin, max_pos, (const bf16_t*)w_ukt, (const bf16_t*)w_uv, (bf16_t*)cache,
                     softmax_scale * 1.4426950408889634f, (bf16_t*)out, out_stride, status);
  return dsv2_launch_status("mla_fused");
}
