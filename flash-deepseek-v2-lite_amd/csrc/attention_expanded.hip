// q_len = 1 decode attention over an EXPANDED per-head K/V cache ([B, H, L, Dq] keys,
// [B, H, L, Dv] values, bf16): the reference's batched_attention_decode_q1_triton surface.
// The decode step itself never uses it (it reads the compressed 576-wide latent cache);
// it is here so a caller that keeps the reference's expanded cache layout can still call
// that function.
//
// One 256-thread workgroup per (row, head).  Tokens go in 64-token chunks:
//   scores  -- 8 tokens per pass, one 32-lane half-wave per token (8 elements per lane,
//              Dq <= 256), half-wave reductions, scaled logits into LDS;
//   softmax -- wave 0 takes the chunk's 64 logits (one per lane): chunk max, running max,
//              rescale factor, p = exp2(logit - max) into LDS, running sum;
//   P.V     -- thread (token group tg = tid / 16, dim group dg = tid % 16) accumulates
//              tokens tg, tg + 16, ... of the chunk over dims 8*dg .. 8*dg + 7 (Dv <= 128
//              per pass of 16 groups; Dv <= 256 takes two dim groups per thread).
// The 16 token groups are summed through LDS at the end; fp32 throughout, one bf16 round.
#include "common.h"

namespace {
constexpr int kChunk = 64;
}

__global__ __launch_bounds__(256) void attention_expanded_kernel(
    const bf16_t* __restrict__ q, int64_t qsb, int64_t qsh, const bf16_t* __restrict__ k, int64_t ksb, int64_t ksh,
    int64_t kss, const bf16_t* __restrict__ v, int64_t vsb, int64_t vsh, int64_t vss, bf16_t* __restrict__ out,
    int64_t osb, int64_t osh, int qd, int vd, int L, const int64_t* __restrict__ cache_position, float scale_log2,
    int32_t* __restrict__ status) {
  __shared__ float s_log[kChunk];
  __shared__ float s_p[kChunk];
  __shared__ float s_alpha;
  __shared__ float s_acc[16][257];
  const int b = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  int64_t pos = cache_position[0];
  if (pos < 0 || pos >= L) {  // positions past the cache: attend the rows that exist, and flag
    if (tid == 0 && h == 0 && b == 0 && status) atomicOr(status, DSV2_DEVERR_CACHE_FULL);
    pos = pos < 0 ? 0 : L - 1;
  }
  const int len = static_cast<int>(pos) + 1;
  const bf16_t* qr = q + b * qsb + h * qsh;
  const bf16_t* kr = k + b * ksb + h * ksh;
  const bf16_t* vr = v + b * vsb + h * vsh;

  // scores: half-wave hw = tid / 32 (0..7) scores token c0 + 8j + hw; lane l32 holds dims 8*l32..
  const int hw = tid >> 5, l32 = tid & 31;
  const bool qon = l32 * 8 < qd;
  float qf[8];
  unpack8(qon ? ldg16(qr + l32 * 8) : make_uint4(0u, 0u, 0u, 0u), qf);
  // P.V: token group tg, dim groups dg and dg + 16
  const int tg = tid >> 4, dg = tid & 15;
  const bool von0 = dg * 8 < vd, von1 = (dg + 16) * 8 < vd;
  float acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;  // meaningful in wave 0

  for (int c0 = 0; c0 < len; c0 += kChunk) {
#pragma unroll
    for (int j = 0; j < kChunk / 8; ++j) {
      const int slot = j * 8 + hw;
      const int t = c0 + slot;
      const int tc = t < len ? t : len - 1;
      float d = qon ? dot8(ldg16(kr + tc * kss + l32 * 8), qf) : 0.f;
#pragma unroll
      for (int off = 16; off > 0; off >>= 1) d += __shfl_xor(d, off, 32);
      if (l32 == 0) s_log[slot] = t < len ? d * scale_log2 : -INFINITY;
    }
    __syncthreads();
    if (wv == 0) {
      const float s = s_log[lane];
      const float m_new = fmaxf(m_run, wave_max(s));
      const float alpha = exp2f(m_run - m_new);
      const float p = exp2f(s - m_new);
      l_run = l_run * alpha + wave_sum(p);
      m_run = m_new;
      s_p[lane] = p;
      if (lane == 0) s_alpha = alpha;
    }
    __syncthreads();
    const float alpha = s_alpha;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] *= alpha;
    for (int tt = tg; tt < kChunk; tt += 16) {
      const int t = c0 + tt;
      if (t >= len) break;
      const float p = s_p[tt];
      if (von0) {
        float f[8];
        unpack8(ldg16(vr + t * vss + dg * 8), f);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = __builtin_fmaf(p, f[i], acc[i]);
      }
      if (von1) {
        float f[8];
        unpack8(ldg16(vr + t * vss + (dg + 16) * 8), f);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[8 + i] = __builtin_fmaf(p, f[i], acc[8 + i]);
      }
    }
    __syncthreads();  // s_log / s_p are rewritten by the next chunk
  }
  __shared__ float s_l;
  if (tid == 0) s_l = l_run;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    s_acc[tg][dg * 8 + i] = acc[i];             // dims of dim group dg
    s_acc[tg][(dg + 16) * 8 + i] = acc[8 + i];  // and of dim group dg + 16
  }
  __syncthreads();
  const float inv = 1.f / s_l;
  for (int d = tid; d < vd; d += 256) {
    float o = 0.f;
#pragma unroll
    for (int g = 0; g < 16; ++g) o += s_acc[g][d];
    out[b * osb + h * osh + d] = f2bf(o * inv);
  }
}

extern "C" int dsv2_attention_decode_expanded(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k,
                                              int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_s,
                                              const void* v, int64_t v_stride_b, int64_t v_stride_h,
                                              int64_t v_stride_s, void* out, int64_t out_stride_b,
                                              int64_t out_stride_h, int batch, int heads, int q_dim, int v_dim,
                                              int seq_len, const int64_t* cache_position, float softmax_scale,
                                              int32_t* status, void* stream) {
  DSV2_REQUIRE(q && k && v && out && cache_position, DSV2_E_NULL, "attention_decode_expanded: null pointer");
  DSV2_REQUIRE(batch >= 0 && batch <= 65535 && heads > 0 && heads <= 65535 && q_dim > 0 && q_dim <= 256 &&
                   q_dim % 8 == 0 && v_dim > 0 && v_dim <= 256 && v_dim % 8 == 0 && seq_len > 0,
               DSV2_E_SHAPE, "attention_decode_expanded: bad shape (q_dim, v_dim <= 256 and %% 8, seq_len > 0)");
  DSV2_REQUIRE(dsv2_aligned16(q) && dsv2_aligned16(k) && dsv2_aligned16(v) && q_stride_b % 8 == 0 &&
                   q_stride_h % 8 == 0 && k_stride_b % 8 == 0 && k_stride_h % 8 == 0 && k_stride_s % 8 == 0 &&
                   v_stride_b % 8 == 0 && v_stride_h % 8 == 0 && v_stride_s % 8 == 0,
               DSV2_E_ALIGN, "attention_decode_expanded: rows must be 16-byte aligned (strides %% 8 elements)");
  if (batch == 0) return DSV2_OK;
  hipLaunchKernelGGL(attention_expanded_kernel, dim3(batch, heads), dim3(256), 0, (hipStream_t)stream,
                     (const bf16_t*)q, q_stride_b, q_stride_h, (const bf16_t*)k, k_stride_b, k_stride_h, k_stride_s,
                     (const bf16_t*)v, v_stride_b, v_stride_h, v_stride_s, (bf16_t*)out, out_stride_b, out_stride_h,
                     q_dim, v_dim, seq_len, cache_position, softmax_scale * 1.4426950408889634f, status);
  return dsv2_launch_status("attention_decode_expanded");
}
