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

// ---------------------------------------------------------------------------------------
// Spread absorbed-MLA attention for a few rows, after mla_prepare (absorbed, rotated q and
// the new cache row already written): per row 64 workgroups of 512 threads, one per (head
// h, quarter qq of W_UV_h's 128 output rows).  Each attends all of the row's cached tokens
// and applies its 32 W_UV rows (requested at entry); no communication between workgroups.
// A token is spread over 16 lanes (lane li holds latent chunks li, li+16, li+32, li+48 of 8
// elements and rope elements 4li .. 4li+3), so a wave scores 4 tokens per instruction:
// q.k by v_dot2_f32_bf16 on the packed bf16 pairs, a 16-lane DPP sum, an online softmax per
// 16-lane row, p.v by v_dot2_f32_bf16 over the row's two tokens with p rounded to bf16 (the
// reference also rounds its softmax weights to bf16 before p.v).  Each wave takes 8 consecutive tokens per batch (2 per row),
// two batches in flight.  The 32 row states of the workgroup merge in LDS.
namespace {
constexpr int kAttWaves = 8, kAttTB = 2;  // tokens per 16-lane row per batch (p.v pairs them)
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot2bf(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}
// sum over the 16 lanes of a row, left in all of them
__device__ __forceinline__ float row16_sum(float v) {
  v += DSV2_DPP(v, 0xB1);   // quad_perm [1,0,3,2]
  v += DSV2_DPP(v, 0x4E);   // quad_perm [2,3,0,1]
  v += DSV2_DPP(v, 0x141);  // row_half_mirror
  v += DSV2_DPP(v, 0x140);  // row_mirror
  return v;
}
struct AttTok {
  uint4 c[4];  // latent chunks li + 16j
  uint2 r;     // rope elements 4li .. 4li+3
};
}  // namespace

__global__ __launch_bounds__(512) void mla_attend_kernel(const bf16_t* __restrict__ q,
                                                         const bf16_t* __restrict__ cache,
                                                         const int64_t* __restrict__ base,
                                                         const int32_t* __restrict__ pos,
                                                         const int32_t* __restrict__ cap,
                                                         const bf16_t* __restrict__ w_uv, float scale_log2,
                                                         bf16_t* __restrict__ out, int64_t os) {
  constexpr int kRows = kAttWaves * 4;  // 16-lane rows per workgroup
  __shared__ float wo[kRows][kLat];
  __shared__ float wm[kRows], wl[kRows];
  __shared__ float olat[kLat];
  const int b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int li = lane & 15, rg = lane >> 4;
  const int h = blockIdx.x >> 2, qq = blockIdx.x & 3;
  // tokens attended: the cached rows [0, n) including the new one (n = pos + 1 at most cap)
  const int pr = pos[b], cp = cap[b];
  const int n = max(1, pr < 0 ? 1 : min(pr + 1, cp));
  const bf16_t* crow0 = cache + base[b] * kRow;

  // ---- entry loads: q_h, the W_UV rows, two token batches ---------------------------------
  const bf16_t* qh = q + ((int64_t)b * 16 + h) * kRow;
  uint4 qc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) qc[j] = ldg16(qh + (li + 16 * j) * 8);
  const uint2 qr = *reinterpret_cast<const uint2*>(qh + kLat + 4 * li);
  uint4 wuv[4];
  {
    const bf16_t* wp = w_uv + ((int64_t)h * 128 + qq * 32 + wv * 4) * kLat + lane * 8;
#pragma unroll
    for (int r = 0; r < 4; ++r) wuv[r] = ldg16(wp + (int64_t)r * kLat);
  }
  constexpr int kStep = kAttWaves * 4 * kAttTB;  // tokens per workgroup per batch
  AttTok ta[kAttTB], tb[kAttTB];
  // token of slot u of this lane's row in the batch starting at T: T + wv*8 + 4u + rg
#define DSV2_ATT_LOAD(S, T)                                                                            \
  do {                                                                                                 \
    _Pragma("unroll") for (int u = 0; u < kAttTB; ++u) {                                               \
      const bf16_t* rp = crow0 + (int64_t)min((T) + wv * 4 * kAttTB + 4 * u + rg, n - 1) * kRow;       \
      _Pragma("unroll") for (int j = 0; j < 4; ++j) S[u].c[j] = ldg16(rp + (li + 16 * j) * 8);         \
      S[u].r = *reinterpret_cast<const uint2*>(rp + kLat + 4 * li);                                    \
    }                                                                                                  \
    asm volatile("" ::: "memory"); /* keeps the loads here, ahead of the batch consumed next */        \
  } while (0)
  const int tw = wv * 4 * kAttTB;
  DSV2_ATT_LOAD(ta, 0);
  DSV2_ATT_LOAD(tb, kStep);

  // ---- attention over [0, n): online softmax per 16-lane row -------------------------------
  float m = -INFINITY, l = 0.f, o[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) o[i] = 0.f;
#define DSV2_ATT_CONSUME(S, T)                                                                         \
  do {                                                                                                 \
    float sc[kAttTB];                                                                                  \
    float mx = m;                                                                                      \
    _Pragma("unroll") for (int u = 0; u < kAttTB; ++u) {                                               \
      float a0 = dot2bf(S[u].r.x, qr.x, 0.f), a1 = dot2bf(S[u].r.y, qr.y, 0.f);                        \
      _Pragma("unroll") for (int j = 0; j < 4; j += 2) {                                               \
        a0 = dot2bf(S[u].c[j].x, qc[j].x, a0);                                                         \
        a1 = dot2bf(S[u].c[j].y, qc[j].y, a1);                                                         \
        a0 = dot2bf(S[u].c[j].z, qc[j].z, a0);                                                         \
        a1 = dot2bf(S[u].c[j].w, qc[j].w, a1);                                                         \
        a0 = dot2bf(S[u].c[j + 1].x, qc[j + 1].x, a0);                                                 \
        a1 = dot2bf(S[u].c[j + 1].y, qc[j + 1].y, a1);                                                 \
        a0 = dot2bf(S[u].c[j + 1].z, qc[j + 1].z, a0);                                                 \
        a1 = dot2bf(S[u].c[j + 1].w, qc[j + 1].w, a1);                                                 \
      }                                                                                                \
      const float sv = row16_sum(a0 + a1);                                                             \
      sc[u] = ((T) + tw + 4 * u + rg < n) ? sv * scale_log2 : -INFINITY;                               \
      mx = fmaxf(mx, sc[u]);                                                                           \
    }                                                                                                  \
    const bool live = mx != -INFINITY; /* a row past n has seen no token yet */                       \
    const float alpha = live ? exp2f(m - mx) : 1.f;                                                    \
    m = mx;                                                                                            \
    l *= alpha;                                                                                        \
    _Pragma("unroll") for (int i = 0; i < 32; ++i) o[i] *= alpha;                                      \
    /* p.v over the row's two tokens by v_dot2_f32_bf16: p rounded to bf16 (and l summed over */     \
    /* the rounded values), each value pair gathered by v_perm_b32 */                                  \
    const uint32_t pp = live ? pack2(exp2f(sc[0] - m), exp2f(sc[1] - m)) : 0u;                         \
    l += __uint_as_float(pp << 16) + __uint_as_float(pp & 0xffff0000u);                                \
    _Pragma("unroll") for (int j = 0; j < 4; ++j) {                                                    \
      const uint32_t a4[4] = {S[0].c[j].x, S[0].c[j].y, S[0].c[j].z, S[0].c[j].w};                     \
      const uint32_t b4[4] = {S[1].c[j].x, S[1].c[j].y, S[1].c[j].z, S[1].c[j].w};                     \
      _Pragma("unroll") for (int w = 0; w < 4; ++w) {                                                  \
        o[8 * j + 2 * w] = dot2bf(__builtin_amdgcn_perm(b4[w], a4[w], 0x05040100u), pp, o[8 * j + 2 * w]); \
        o[8 * j + 2 * w + 1] =                                                                         \
            dot2bf(__builtin_amdgcn_perm(b4[w], a4[w], 0x07060302u), pp, o[8 * j + 2 * w + 1]);        \
      }                                                                                                \
    }                                                                                                  \
  } while (0)
  for (int t0 = 0; t0 < n; t0 += 2 * kStep) {
    DSV2_ATT_CONSUME(ta, t0);
    DSV2_ATT_LOAD(ta, t0 + 2 * kStep);
    if (t0 + kStep < n) DSV2_ATT_CONSUME(tb, t0 + kStep);
    DSV2_ATT_LOAD(tb, t0 + 3 * kStep);
  }
#undef DSV2_ATT_CONSUME
#undef DSV2_ATT_LOAD
  const int row = wv * 4 + rg;
  if (li == 0) {
    wm[row] = m;
    wl[row] = l;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) wo[row][(li + 16 * j) * 8 + i] = o[8 * j + i];
  __syncthreads();
  // merge the rows (a row that saw no token carries m = -inf: weight 0; row 0 of wave 0
  // always sees token 0, so M is finite)
  {
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kRows; ++w) M = fmaxf(M, wm[w]);
    float L = 0.f, acc = 0.f;
#pragma unroll
    for (int w = 0; w < kRows; ++w) {
      const float sw = exp2f(wm[w] - M);
      L = __builtin_fmaf(wl[w], sw, L);
      acc = __builtin_fmaf(wo[w][tid], sw, acc);
    }
    olat[tid] = acc / L;
  }
  __syncthreads();

  // ---- W_UV rows qq*32 + wv*4 .. +3 of head h ---------------------------------------------
  float xo[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) xo[i] = olat[lane * 8 + i];
  float yr[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) yr[r] = wave_sum_dpp(dot8(wuv[r], xo));
  if (lane == 0) {
    uint2 w;
    w.x = pack2(yr[0], yr[1]);
    w.y = pack2(yr[2], yr[3]);
    *reinterpret_cast<uint2*>(out + (int64_t)b * os + h * 128 + qq * 32 + wv * 4) = w;
  }
}

void mla_prepare_absorb_launch(const void* qkva, int64_t qkva_stride, int rows, const int32_t* pos,
                               const int64_t* base, const int32_t* cap, const void* kv_norm_w, float eps,
                               const void* rope_cos, const void* rope_sin, int max_pos, const void* w_ukt,
                               const void* w_uv, void* cache, void* q_out, int32_t* status, hipStream_t stream);

static void mla_attend_launch(const void* q, const void* cache, const int64_t* base, const int32_t* pos,
                              const int32_t* cap, int rows, const void* w_uv, float softmax_scale, void* out,
                              int64_t out_stride, hipStream_t stream) {
  hipLaunchKernelGGL(mla_attend_kernel, dim3(64, rows), dim3(512), 0, stream, (const bf16_t*)q, (const bf16_t*)cache,
                     base, pos, cap, (const bf16_t*)w_uv, softmax_scale * 1.4426950408889634f, (bf16_t*)out,
                     out_stride);
}

extern "C" int dsv2_mla_attend(const void* q, const void* cache, const int64_t* base, const int32_t* pos,
                               const int32_t* cap, int rows, const void* w_uv, float softmax_scale, void* out,
                               int64_t out_stride, void* stream) {
  DSV2_REQUIRE(q && cache && base && pos && cap && w_uv && out, DSV2_E_NULL, "mla_attend: null pointer");
  DSV2_REQUIRE(rows >= 0 && rows <= 65535 && out_stride >= 2048, DSV2_E_SHAPE, "mla_attend: bad shape");
  DSV2_REQUIRE(dsv2_aligned16(q) && dsv2_aligned16(cache) && dsv2_aligned16(w_uv) && dsv2_aligned16(out) &&
                   out_stride % 8 == 0,
               DSV2_E_ALIGN, "mla_attend: alignment");
  if (rows == 0) return DSV2_OK;
  mla_attend_launch(q, cache, base, pos, cap, rows, w_uv, softmax_scale, out, out_stride, (hipStream_t)stream);
  return dsv2_launch_status("mla_attend");
}

extern "C" int dsv2_mla_spread(const void* qkva, int64_t qkva_stride, int rows, const int32_t* pos,
                               const int64_t* base, const int32_t* cap, const void* kv_norm_w, float eps,
                               const void* rope_cos, const void* rope_sin, int max_pos, const void* w_ukt,
                               const void* w_uv, void* cache, void* q_buf, float softmax_scale, void* out,
                               int64_t out_stride, int32_t* status, void* stream) {
  DSV2_REQUIRE(qkva && pos && base && cap && kv_norm_w && rope_cos && rope_sin && w_ukt && w_uv && cache && q_buf &&
                   out,
               DSV2_E_NULL, "mla_spread: null pointer");
  DSV2_REQUIRE(rows >= 0 && rows <= 65535 && max_pos > 0 && qkva_stride >= 3648 && out_stride >= 2048, DSV2_E_SHAPE,
               "mla_spread: bad shape");
  DSV2_REQUIRE(dsv2_aligned16(qkva) && qkva_stride % 8 == 0 && dsv2_aligned16(kv_norm_w) && dsv2_aligned16(cache) &&
                   dsv2_aligned16(w_ukt) && dsv2_aligned16(w_uv) && dsv2_aligned16(q_buf) && dsv2_aligned16(out) &&
                   out_stride % 8 == 0,
               DSV2_E_ALIGN, "mla_spread: alignment");
  if (rows == 0) return DSV2_OK;
  mla_prepare_absorb_launch(qkva, qkva_stride, rows, pos, base, cap, kv_norm_w, eps, rope_cos, rope_sin, max_pos,
                            w_ukt, w_uv, cache, q_buf, status, (hipStream_t)stream);
  mla_attend_launch(q_buf, cache, base, pos, cap, rows, w_uv, softmax_scale, out, out_stride, (hipStream_t)stream);
  return dsv2_launch_status("mla_spread");
}
