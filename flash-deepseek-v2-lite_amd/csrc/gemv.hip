// Few-row bf16 GEMV for the small family (bsz 1..8 per launch): weights streamed
// once with 16-byte loads, fp32 accumulation, fused RMSNorm prologue, SwiGLU /
// residual / fp32-logit epilogues.  One wave owns RPW output rows at a time (RPW gate +
// RPW up rows for SwiGLU); lanes split K in 8-element chunks.
#include <mutex>

#include "common.h"

// K <= 2048: one batch of chunks per row (lane l owns chunks l, l+64, l+128, l+192).
// Grid-stride over groups of RPW rows so at most ~4 workgroups per CU live long enough
// to keep HBM busy; the next group's weights are requested before the current group is
// reduced.  x' (normalised when nw != null) is built once per workgroup in LDS.  Every
// load is unconditional (indices clamped, masked where used) and issued in the order it is
// consumed -- x and the norm weights, then the weight rows, then the residuals -- since
// loads complete in issue order: no wait for an early operand waits for the weight stream.
template <int NB, int RPW, bool SWIGLU>
__global__ __launch_bounds__(256) void gemv_k2048_kernel(const bf16_t* __restrict__ x, int64_t xs, int B, int K,
                                                         const bf16_t* __restrict__ W, int N,
                                                         const bf16_t* __restrict__ nw, float eps,
                                                         const bf16_t* __restrict__ res, int64_t rs,
                                                         void* __restrict__ y, int64_t ys, bool out_f32,
                                                         float* __restrict__ amax) {
  constexpr int U = 4;
  __shared__ float xl[NB][2048];
  __shared__ float red[NB][4];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, tid = threadIdx.x;
  const int nch = K >> 3;
  const int ngroups = N / RPW;
  const int tw = gridDim.x * 4;
  int g = blockIdx.x * 4 + wv;

  // thread t owns chunk t of every row (clamped; threads past nch are masked below)
  const bool own = tid < nch;
  const int tc = own ? tid : nch - 1;
  // (no branch around a load -- the wait counts after a conditional load become
  // conservative: a missing norm / residual operand reads x instead and is ignored)
  uint4 xv4[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) xv4[b] = ldg16(x + (b < B ? b : 0) * xs + tc * 8);
  const uint4 g4 = ldg16((nw ? nw : x) + tc * 8);

  uint4 wg[U][RPW], wu[U][RPW];
  bf16_t rvb[RPW][NB];
  auto load = [&](int grp) {  // the group's residuals (or a harmless read of x), then its weights
    {
      const bf16_t* rp = res ? res + grp * RPW : x;
#pragma unroll
      for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int b = 0; b < NB; ++b) rvb[r][b] = rp[res ? (b < B ? b : 0) * rs + r : 0];
    }
    const bf16_t* wr = W + (int64_t)grp * RPW * K;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = min(lane + 64 * u, nch - 1);
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        wg[u][r] = ldg16_nt(wr + (int64_t)r * K + c * 8);
        if (SWIGLU) wu[u][r] = ldg16_nt(wr + (int64_t)(N + r) * K + c * 8);
      }
    }
  };
  load(min(g, ngroups - 1));  // unconditional: a wave without a group reloads the last one
  pin(g4.x);
#pragma unroll
  for (int b = 0; b < NB; ++b) pin(xv4[b].x);

  // x' -> LDS (fp32), one pass over x per row
  {
    float g8[8];
    if (nw) unpack8(g4, g8);
    float xv[NB][8];
    float ss[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      unpack8(xv4[b], xv[b]);
      ss[b] = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) ss[b] = __builtin_fmaf(xv[b][i], xv[b][i], ss[b]);
      if (!own) ss[b] = 0.f;
    }
    if (nw) {
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const float t = wave_sum(ss[b]);
        if (lane == 0) red[b][wv] = t;
      }
      __syncthreads();
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const float rn = rsqrtf((red[b][0] + red[b][1] + red[b][2] + red[b][3]) / static_cast<float>(K) + eps);
#pragma unroll
        for (int i = 0; i < 8; ++i) xv[b][i] = rbf(g8[i] * rbf(xv[b][i] * rn));
      }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b)
      if (b < B && own) {
#pragma unroll
        for (int i = 0; i < 8; ++i) xl[b][tid * 8 + i] = xv[b][i];
      }
    __syncthreads();
  }

  // amax != null (fp32 logits): per wave and row, the first index of the largest output
  // (rows are visited in increasing order, so a strict > keeps the lowest index)
  float best[NB];
  int bidx[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    best[b] = -INFINITY;
    bidx[b] = 0x7fffffff;
  }
  while (g < ngroups) {
    const int n0 = g * RPW;
    float acc[RPW][NB], accu[RPW][NB];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int b = 0; b < NB; ++b) acc[r][b] = accu[r][b] = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = lane + 64 * u;
      if (c >= nch) break;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (b < B) {
          const float* xp = &xl[b][c * 8];
#pragma unroll
          for (int r = 0; r < RPW; ++r) {
            acc[r][b] += dot8(wg[u][r], xp);
            if (SWIGLU) accu[r][b] += dot8(wu[u][r], xp);
          }
        }
      }
    }
    float rv[RPW][NB];
    if (res) {
#pragma unroll
      for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int b = 0; b < NB; ++b) rv[r][b] = bf2f(rvb[r][b]);
    }
    g += tw;
    load(min(g, ngroups - 1));  // next group's weights in flight during the reduction
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
#pragma unroll
      for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          acc[r][b] = xor_sum(acc[r][b], off);
          if (SWIGLU) accu[r][b] = xor_sum(accu[r][b], off);
        }
    if (lane == 0) {
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (b >= B) break;
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
          const int n = n0 + r;
          float v = SWIGLU ? swiglu_bf(acc[r][b], accu[r][b]) : rbf(acc[r][b]);
          if (res) v = rbf(rv[r][b] + v);
          if (out_f32)
            reinterpret_cast<float*>(y)[b * ys + n] = v;
          else
            reinterpret_cast<bf16_t*>(y)[b * ys + n] = f2bf(v);
          if (v > best[b]) {
            best[b] = v;
            bidx[b] = n;
          }
        }
      }
    }
  }
  if (amax && lane == 0) {
    const int nw = gridDim.x * 4, gw = blockIdx.x * 4 + wv;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      if (b >= B) break;
      amax[2 * (b * nw + gw)] = best[b];
      reinterpret_cast<int*>(amax)[2 * (b * nw + gw) + 1] = bidx[b];
    }
  }
}

// One row (bsz = 1), K = 2048: one-shot launch, one wave per RPW output rows (plus the RPW
// matching up rows for SwiGLU), so the grid is N / (4 RPW) workgroups.  Each wave loads x
// itself from L2/L1 while its weight rows are in flight -- no LDS staging, no barrier.
// (Used without a norm prologue: with one, the per-wave RMSNorm measured slower on MI355X
// than the workgroup-shared norm of gemv_k2048_kernel.)
template <int RPW, bool SW, bool NORM>
__global__ __launch_bounds__(256) void gemv_b1_kernel(const bf16_t* __restrict__ x, const bf16_t* __restrict__ W, int N,
                                                      const bf16_t* __restrict__ nw, float eps,
                                                      const bf16_t* __restrict__ res, void* __restrict__ y,
                                                      bool out_f32) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int n0 = (blockIdx.x * 4 + wv) * RPW;
  if (n0 >= N) return;
  // x (and the norm weights) are requested before the weight rows: loads complete in issue
  // order, so the wait for x does not wait for the weight stream behind it.  Every load is
  // unconditional and converted only where it is used.
  uint4 xr[4], gr[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) xr[j] = ldg16(x + (lane + 64 * j) * 8);
  if (NORM) {
#pragma unroll
    for (int j = 0; j < 4; ++j) gr[j] = ldg16(nw + (lane + 64 * j) * 8);
  }
  // residual (or, without one, a harmless read of x), also ahead of the weights
  bf16_t rvb[RPW];
  {
    const bf16_t* rp = res ? res + n0 : x;
#pragma unroll
    for (int r = 0; r < RPW; ++r) rvb[r] = rp[res ? r : 0];
  }
  uint4 wg[RPW][4], wu[RPW][4];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      wg[r][j] = ldg16_nt(W + (int64_t)(n0 + r) * 2048 + (lane + 64 * j) * 8);
      if (SW) wu[r][j] = ldg16_nt(W + (int64_t)(N + n0 + r) * 2048 + (lane + 64 * j) * 8);
    }
#pragma unroll
  for (int r = 0; r < RPW; ++r) pin(rvb[r]);
  if (NORM) pin(gr[0].x);
  float xf[32];
#pragma unroll
  for (int j = 0; j < 4; ++j) unpack8(xr[j], xf + 8 * j);
  if (NORM) {
    float g8[32];
#pragma unroll
    for (int j = 0; j < 4; ++j) unpack8(gr[j], g8 + 8 * j);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) ss = __builtin_fmaf(xf[i], xf[i], ss);
    ss = wave_sum(ss);
    const float rs = rsqrtf(ss / 2048.f + eps);
#pragma unroll
    for (int i = 0; i < 32; ++i) xf[i] = rbf(g8[i] * rbf(xf[i] * rs));
  }
  float ag[RPW], au[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    ag[r] = au[r] = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      ag[r] += dot8(wg[r][j], xf + 8 * j);
      if (SW) au[r] += dot8(wu[r][j], xf + 8 * j);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      ag[r] = xor_sum(ag[r], off);
      if (SW) au[r] = xor_sum(au[r], off);
    }
  // every lane forms the outputs (the residual is consumed in this block, so its load stays
  // where it was issued, in flight with the weights); lane 0 stores them
  float v[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const float t = SW ? swiglu_bf(ag[r], au[r]) : rbf(ag[r]);
    v[r] = res ? rbf(bf2f(rvb[r]) + t) : t;
  }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      if (out_f32)
        reinterpret_cast<float*>(y)[n0 + r] = v[r];
      else
        reinterpret_cast<bf16_t*>(y)[n0 + r] = f2bf(v[r]);
    }
  }
}

static void launch_b1(const bf16_t* x, const bf16_t* W, int N, const bf16_t* nw, float eps, const bf16_t* res, void* y,
                      bool sw, bool f32, hipStream_t st) {
  const dim3 grid((N + 3) / 4);
  if (sw) {
    if (nw)
      hipLaunchKernelGGL((gemv_b1_kernel<1, true, true>), grid, dim3(256), 0, st, x, W, N, nw, eps, res, y, f32);
    else
      hipLaunchKernelGGL((gemv_b1_kernel<1, true, false>), grid, dim3(256), 0, st, x, W, N, nw, eps, res, y, f32);
  } else {
    if (nw)
      hipLaunchKernelGGL((gemv_b1_kernel<1, false, true>), grid, dim3(256), 0, st, x, W, N, nw, eps, res, y, f32);
    else
      hipLaunchKernelGGL((gemv_b1_kernel<1, false, false>), grid, dim3(256), 0, st, x, W, N, nw, eps, res, y, f32);
  }
}

// K > 2048 (the dense down projection, K = 10944): one workgroup per 4*RPW rows,
// U chunks per row in flight, x read from L2 per chunk; no normalisation.
template <int NB, int RPW, int U>
__global__ __launch_bounds__(256) void gemv_klong_kernel(const bf16_t* __restrict__ x, int64_t xs, int B, int K,
                                                         const bf16_t* __restrict__ W, int N,
                                                         const bf16_t* __restrict__ res, int64_t rs,
                                                         void* __restrict__ y, int64_t ys, bool out_f32) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int nch = K >> 3;
  const int n0 = (blockIdx.x * 4 + wv) * RPW;
  if (n0 >= N) return;
  const bf16_t* wr = W + (int64_t)n0 * K;
  bf16_t rvb[RPW][NB];
  {
    const bf16_t* rp = res ? res + n0 : x;  // no branch around a load
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int b = 0; b < NB; ++b) rvb[r][b] = rp[res ? (b < B ? b : 0) * rs + r : 0];
  }
  float acc[RPW][NB];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[r][b] = 0.f;
  for (int c0 = lane; c0 < nch; c0 += 64 * U) {
    // the chunk batch's x and weights all requested before any is used (clamped chunks,
    // masked below)
    uint4 wg[U][RPW], xb[U][NB];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = min(c0 + 64 * u, nch - 1);
#pragma unroll
      for (int b = 0; b < NB; ++b) xb[u][b] = ldg16(x + (b < B ? b : 0) * xs + c * 8);
#pragma unroll
      for (int r = 0; r < RPW; ++r) wg[u][r] = ldg16_nt(wr + (int64_t)r * K + c * 8);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + 64 * u;
      if (c >= nch) break;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (b < B) {
          float xf[8];
          unpack8(xb[u][b], xf);
#pragma unroll
          for (int r = 0; r < RPW; ++r) acc[r][b] += dot8(wg[u][r], xf);
        }
      }
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int b = 0; b < NB; ++b) acc[r][b] = xor_sum(acc[r][b], off);
  if (lane == 0) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      if (b >= B) break;
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        const int n = n0 + r;
        float v = rbf(acc[r][b]);
        if (res) v = rbf(bf2f(rvb[r][b]) + v);
        if (out_f32)
          reinterpret_cast<float*>(y)[b * ys + n] = v;
        else
          reinterpret_cast<bf16_t*>(y)[b * ys + n] = f2bf(v);
      }
    }
  }
}

static int k2048_grid(int N, int RPW) {
  const int groups = N / RPW;
  const int grid = (groups + 3) / 4;
  return grid > 1024 ? 1024 : grid;  // grid-stride beyond 4 workgroups per CU
}

template <int NB, int RPW, bool SW>
static void launch_k2048(const bf16_t* x, int64_t xs, int B, int K, const bf16_t* W, int N, const bf16_t* nw,
                         float eps, const bf16_t* res, int64_t rs, void* y, int64_t ys, bool f32, hipStream_t st,
                         float* amax = nullptr) {
  hipLaunchKernelGGL((gemv_k2048_kernel<NB, RPW, SW>), dim3(k2048_grid(N, RPW)), dim3(256), 0, st, x, xs, B, K, W, N,
                     nw, eps, res, rs, y, ys, f32, amax);
}

template <int NB>
static void launch_gemv_nb(const bf16_t* x, int64_t xs, int B, int K, const bf16_t* W, int N, const bf16_t* nw,
                           float eps, const bf16_t* res, int64_t rs, void* y, int64_t ys, bool sw, bool f32,
                           hipStream_t st) {
  if (K > 2048) {
    hipLaunchKernelGGL((gemv_klong_kernel<NB, 1, 8>), dim3((N + 3) / 4), dim3(256), 0, st, x, xs, B, K, W, N, res, rs,
                       y, ys, f32);
    return;
  }
  // rows per wave: SwiGLU 1 for the 2-4K-row projections (>= 2 workgroups per CU), 2 above;
  // plain 2 whenever N is even (qkv_a with its norm prologue: 5.8 us against 6.2 us with 1)
  if (sw) {
    if (N > 4096)
      launch_k2048<NB, 2, true>(x, xs, B, K, W, N, nw, eps, res, rs, y, ys, f32, st);
    else
      launch_k2048<NB, 1, true>(x, xs, B, K, W, N, nw, eps, res, rs, y, ys, f32, st);
  } else {
    if (N % 2 == 0)
      launch_k2048<NB, 2, false>(x, xs, B, K, W, N, nw, eps, res, rs, y, ys, f32, st);
    else
      launch_k2048<NB, 1, false>(x, xs, B, K, W, N, nw, eps, res, rs, y, ys, f32, st);
  }
}

extern "C" int dsv2_gemv_bf16(const void* x, int64_t x_stride, int rows, int K, const void* W, int N,
                              const void* norm_w, float eps, const void* residual, int64_t res_stride, void* y,
                              int64_t y_stride, int flags, void* stream) {
  DSV2_REQUIRE(x && W && y, DSV2_E_NULL, "gemv: null pointer");
  DSV2_REQUIRE(rows >= 0 && K > 0 && K % 8 == 0 && N > 0 && N % 8 == 0, DSV2_E_SHAPE,
               "gemv: bad shape rows=%d K=%d N=%d", rows, K, N);
  DSV2_REQUIRE((flags & ~(DSV2_LINEAR_SWIGLU | DSV2_LINEAR_OUT_F32)) == 0, DSV2_E_FLAGS, "gemv: unknown flags %d",
               flags);
  DSV2_REQUIRE(!((flags & DSV2_LINEAR_SWIGLU) && residual), DSV2_E_FLAGS, "gemv: SwiGLU with residual unsupported");
  DSV2_REQUIRE(dsv2_aligned16(x) && dsv2_aligned16(W) && x_stride % 8 == 0 && (!norm_w || dsv2_aligned16(norm_w)),
               DSV2_E_ALIGN, "gemv: x/W/norm_w must be 16-byte aligned");
  const bool sw = flags & DSV2_LINEAR_SWIGLU, f32 = flags & DSV2_LINEAR_OUT_F32;
  DSV2_REQUIRE(K <= 2048 || (!norm_w && !sw), DSV2_E_FLAGS, "gemv: K > 2048 supports neither norm nor SwiGLU");
  hipStream_t st = (hipStream_t)stream;
  const bf16_t* xb = (const bf16_t*)x;
  if (rows == 1 && K == 2048 && !norm_w) {
    launch_b1(xb, (const bf16_t*)W, N, (const bf16_t*)norm_w, eps, (const bf16_t*)residual, y, sw, f32, st);
    return dsv2_launch_status("gemv");
  }
  for (int r0 = 0; r0 < rows; r0 += 8) {
    const int B = rows - r0 < 8 ? rows - r0 : 8;
    const bf16_t* xr = xb + r0 * x_stride;
    const bf16_t* rr = residual ? (const bf16_t*)residual + r0 * res_stride : nullptr;
    void* yr = f32 ? (void*)((float*)y + r0 * y_stride) : (void*)((bf16_t*)y + r0 * y_stride);
    const bf16_t* wb = (const bf16_t*)W;
    const bf16_t* nb = (const bf16_t*)norm_w;
    if (B == 1)
      launch_gemv_nb<1>(xr, x_stride, B, K, wb, N, nb, eps, rr, res_stride, yr, y_stride, sw, f32, st);
    else if (B == 2)
      launch_gemv_nb<2>(xr, x_stride, B, K, wb, N, nb, eps, rr, res_stride, yr, y_stride, sw, f32, st);
    else if (B <= 4)
      launch_gemv_nb<4>(xr, x_stride, B, K, wb, N, nb, eps, rr, res_stride, yr, y_stride, sw, f32, st);
    else
      launch_gemv_nb<8>(xr, x_stride, B, K, wb, N, nb, eps, rr, res_stride, yr, y_stride, sw, f32, st);
    int rc = dsv2_launch_status("gemv");
    if (rc) return rc;
  }
  return DSV2_OK;
}

// ---------------------------------------------------------------------------
// lm_head + greedy argmax: the GEMV records each wave's (max, first index) while it
// writes the fp32 logits, then one workgroup per row reduces the per-wave partials
// (a few KB instead of the whole vocabulary row).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void argmax_partials_kernel(const float* __restrict__ amax, int nw,
                                                              int64_t* __restrict__ next_ids, int32_t* __restrict__ pos) {
  __shared__ float sv[4];
  __shared__ int si[4];
  const int b = blockIdx.x, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  // nw <= 4096: every thread requests its (up to) 16 partials before comparing any
  float2 pv[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int i = threadIdx.x + 256 * k;
    pv[k] = i < nw ? reinterpret_cast<const float2*>(amax)[b * nw + i] : make_float2(-INFINITY, 0.f);
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const float v = pv[k].x;
    const int ix = __float_as_int(pv[k].y);
    if (threadIdx.x + 256 * k < nw && (v > best || (v == best && ix < bi))) {
      best = v;
      bi = ix;
    }
  }
  wave_argmax(best, bi);
  if (lane == 0) {
    sv[w] = best;
    si[w] = bi;
  }
  __syncthreads();
  if (w == 0) {
    best = lane < 4 ? sv[lane] : -INFINITY;
    bi = lane < 4 ? si[lane] : 0x7fffffff;
    wave_argmax(best, bi);
    if (lane == 0) {
      next_ids[b] = bi == 0x7fffffff ? 0 : bi;
      if (pos) pos[b] += 1;
    }
  }
}

extern "C" int64_t dsv2_lm_head_argmax_workspace_size(int rows) {
  return rows < 0 ? -1 : (int64_t)rows * 1024 * 4 * 8;
}

static int lm_head_argmax_launch(const void* x, int64_t x_stride, int rows, const void* W, int vocab,
                                 const void* norm_w, float eps, float* logits, float* amax, int64_t* next_ids,
                                 int32_t* pos, hipStream_t st) {
  const bf16_t* xb = (const bf16_t*)x;
  constexpr int RPW = 2;
  if (rows == 1)
    launch_k2048<1, RPW, false>(xb, x_stride, rows, 2048, (const bf16_t*)W, vocab, (const bf16_t*)norm_w, eps,
                                nullptr, 0, logits, vocab, true, st, amax);
  else if (rows == 2)
    launch_k2048<2, RPW, false>(xb, x_stride, rows, 2048, (const bf16_t*)W, vocab, (const bf16_t*)norm_w, eps,
                                nullptr, 0, logits, vocab, true, st, amax);
  else if (rows <= 4)
    launch_k2048<4, RPW, false>(xb, x_stride, rows, 2048, (const bf16_t*)W, vocab, (const bf16_t*)norm_w, eps,
                                nullptr, 0, logits, vocab, true, st, amax);
  else
    launch_k2048<8, RPW, false>(xb, x_stride, rows, 2048, (const bf16_t*)W, vocab, (const bf16_t*)norm_w, eps,
                                nullptr, 0, logits, vocab, true, st, amax);
  int rc = dsv2_launch_status("lm_head_argmax");
  if (rc) return rc;
  // every wave of the GEMV writes its (max, index) partial of every row, so the partials
  // need no clearing between calls
  hipLaunchKernelGGL(argmax_partials_kernel, dim3(rows), dim3(256), 0, st, amax, k2048_grid(vocab, RPW) * 4, next_ids,
                     pos);
  return dsv2_launch_status("lm_head_argmax");
}

#define DSV2_LM_HEAD_ARGS_OK(fn)                                                                                     \
  DSV2_REQUIRE(x && W && norm_w && logits && next_ids, DSV2_E_NULL, fn ": null pointer");                           \
  DSV2_REQUIRE(rows >= 1 && rows <= 8 && vocab > 0 && vocab % 2 == 0, DSV2_E_SHAPE,                                  \
               fn ": 1 <= rows <= 8 and an even vocabulary required (rows %d, vocab %d)", rows, vocab);              \
  DSV2_REQUIRE(dsv2_aligned16(x) && dsv2_aligned16(W) && dsv2_aligned16(norm_w) && x_stride % 8 == 0, DSV2_E_ALIGN, \
               fn ": alignment")

extern "C" int dsv2_lm_head_argmax_bf16(const void* x, int64_t x_stride, int rows, const void* W, int vocab,
                                        const void* norm_w, float eps, float* logits, void* partials,
                                        int64_t partials_bytes, int64_t* next_ids, int32_t* pos, void* stream) {
  DSV2_LM_HEAD_ARGS_OK("lm_head_argmax");
  DSV2_REQUIRE(partials, DSV2_E_NULL, "lm_head_argmax: null pointer");
  DSV2_REQUIRE(partials_bytes >= dsv2_lm_head_argmax_workspace_size(rows), DSV2_E_SHAPE,
               "lm_head_argmax: partials buffer too small");
  return lm_head_argmax_launch(x, x_stride, rows, W, vocab, norm_w, eps, logits, (float*)partials, next_ids, pos,
                               (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// The same, for callers that cannot allocate (code under graph capture, serving loops
// that forbid hipMalloc): the argmax partials live in `scratch`, a file-scope device array
// of the library -- one copy per GPU, held until the process ends, sized for the largest
// call (8 rows x 4096 waves x (max, index) = 256 KiB).  Host code never passes the array's
// name to a kernel (on the host it is only a stand-in): each device's address comes from
// hipGetSymbolAddress, taken once per device on the first call made with that device
// current, and kept in g_scratch_dev.
// ---------------------------------------------------------------------------
namespace {
constexpr int kScratchRows = 8;
constexpr int64_t kScratchBytes = (int64_t)kScratchRows * 4096 * 8;
constexpr int kMaxDevices = 64;
void* g_scratch_dev[kMaxDevices] = {};
std::mutex g_scratch_mu;
}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

static int scratch_on_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  DSV2_REQUIRE(e == hipSuccess, (int)e, "lm_head_argmax_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
  DSV2_REQUIRE(dev >= 0 && dev < kMaxDevices, DSV2_E_SHAPE, "lm_head_argmax_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    DSV2_REQUIRE(e == hipSuccess && p, e == hipSuccess ? DSV2_E_NULL : (int)e,
                 "lm_head_argmax_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                 hipGetErrorString(e));
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return DSV2_OK;
}

extern "C" int dsv2_lm_head_argmax_bf16_noalloc(const void* x, int64_t x_stride, int rows, const void* W, int vocab,
                                                const void* norm_w, float eps, float* logits, int64_t* next_ids,
                                                int32_t* pos, void* stream) {
  DSV2_LM_HEAD_ARGS_OK("lm_head_argmax_noalloc");
  DSV2_REQUIRE(dsv2_lm_head_argmax_workspace_size(rows) <= kScratchBytes, DSV2_E_SHAPE,
               "lm_head_argmax_noalloc: %d rows need more than the %lld-byte device scratch", rows,
               (long long)kScratchBytes);
  void* dev_scratch = nullptr;
  const int rc = scratch_on_current_device(&dev_scratch);
  if (rc) return rc;
  return lm_head_argmax_launch(x, x_stride, rows, W, vocab, norm_w, eps, logits, (float*)dev_scratch, next_ids, pos,
                               (hipStream_t)stream);
}
