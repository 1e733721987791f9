// Few-row bf16 GEMV for the small family (bsz 1..8 per launch): weights streamed
// once with 16-byte loads, fp32 accumulation, fused RMSNorm prologue, SwiGLU /
// residual / fp32-logit epilogues.  One wave owns RPW output rows at a time (RPW gate +
// RPW up rows for SwiGLU); lanes split K in 8-element chunks.
#include "common.h"

// K <= 2048: one batch of chunks per row (lane l owns chunks l, l+64, l+128, l+192).
// Grid-stride over groups of RPW rows so at most ~4 workgroups per CU live long enough
// to keep HBM busy; the next group's weights are requested before the current group is
// reduced.  x' (normalised when nw != null) is built once per workgroup in LDS while the
// first group's weights are in flight; residuals are fetched before the dot products.
template <int NB, int RPW, bool SWIGLU>
__global__ __launch_bounds__(256) void gemv_k2048_kernel(const bf16_t* __restrict__ x, int64_t xs, int B, int K,
                                                         const bf16_t* __restrict__ W, int N,
                                                         const bf16_t* __restrict__ nw, float eps,
                                                         const bf16_t* __restrict__ res, int64_t rs,
                                                         void* __restrict__ y, int64_t ys, bool out_f32) {
  constexpr int U = 4;
  __shared__ float xl[NB][2048];
  __shared__ float red[NB][4];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, tid = threadIdx.x;
  const int nch = K >> 3;
  const int ngroups = N / RPW;
  const int tw = gridDim.x * 4;
  int g = blockIdx.x * 4 + wv;

  uint4 wg[U][RPW], wu[U][RPW];
  auto load = [&](int grp) {
    const bf16_t* wr = W + (int64_t)grp * RPW * K;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = lane + 64 * u;
      if (c < nch) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
          wg[u][r] = ldg16(wr + (int64_t)r * K + c * 8);
          if (SWIGLU) wu[u][r] = ldg16(wr + (int64_t)(N + r) * K + c * 8);
        }
      }
    }
  };
  if (g < ngroups) load(g);

  // x' -> LDS (fp32), one pass over x per row; thread t owns chunk t of every row
  {
    const bool own = tid < nch;
    float g8[8];
    if (nw && own) unpack8(ldg16(nw + tid * 8), g8);
    float xv[NB][8];
    float ss[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      ss[b] = 0.f;
      if (b < B && own) {
        unpack8(ldg16(x + b * xs + tid * 8), xv[b]);
#pragma unroll
        for (int i = 0; i < 8; ++i) ss[b] = __builtin_fmaf(xv[b][i], xv[b][i], ss[b]);
      }
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
        if (b < B && own) {
#pragma unroll
          for (int i = 0; i < 8; ++i) xv[b][i] = rbf(g8[i] * rbf(xv[b][i] * rn));
        }
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

  while (g < ngroups) {
    const int n0 = g * RPW;
    float rv[RPW][NB];
    if (res && lane == 0) {
#pragma unroll
      for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int b = 0; b < NB; ++b) rv[r][b] = b < B ? bf2f(res[b * rs + n0 + r]) : 0.f;
    }
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
    g += tw;
    if (g < ngroups) load(g);  // next group's weights in flight during the reduction
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
#pragma unroll
      for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          acc[r][b] += __shfl_xor(acc[r][b], off, 64);
          if (SWIGLU) accu[r][b] += __shfl_xor(accu[r][b], off, 64);
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
        }
      }
    }
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
  float rv[RPW][NB];
  if (res && lane == 0) {
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int b = 0; b < NB; ++b) rv[r][b] = b < B ? bf2f(res[b * rs + n0 + r]) : 0.f;
  }
  float acc[RPW][NB];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[r][b] = 0.f;
  for (int c0 = lane; c0 < nch; c0 += 64 * U) {
    uint4 wg[U][RPW];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + 64 * u;
      if (c < nch) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) wg[u][r] = ldg16(wr + (int64_t)r * K + c * 8);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + 64 * u;
      if (c >= nch) break;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (b < B) {
          float xf[8];
          unpack8(ldg16(x + b * xs + c * 8), xf);
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
      for (int b = 0; b < NB; ++b) acc[r][b] += __shfl_xor(acc[r][b], off, 64);
  if (lane == 0) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      if (b >= B) break;
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        const int n = n0 + r;
        float v = rbf(acc[r][b]);
        if (res) v = rbf(rv[r][b] + v);
        if (out_f32)
          reinterpret_cast<float*>(y)[b * ys + n] = v;
        else
          reinterpret_cast<bf16_t*>(y)[b * ys + n] = f2bf(v);
      }
    }
  }
}

template <int NB, int RPW, bool SW>
static void launch_k2048(const bf16_t* x, int64_t xs, int B, int K, const bf16_t* W, int N, const bf16_t* nw,
                         float eps, const bf16_t* res, int64_t rs, void* y, int64_t ys, bool f32, hipStream_t st) {
  const int groups = N / RPW;
  int grid = (groups + 3) / 4;
  if (grid > 1024) grid = 1024;  // grid-stride beyond 4 workgroups per CU
  hipLaunchKernelGGL((gemv_k2048_kernel<NB, RPW, SW>), dim3(grid), dim3(256), 0, st, x, xs, B, K, W, N, nw, eps, res,
                     rs, y, ys, f32);
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
  // rows per wave: 1 for the 2-4K-row projections (>= 2 workgroups per CU), 2 above
  if (sw) {
    if (N > 4096)
      launch_k2048<NB, 2, true>(x, xs, B, K, W, N, nw, eps, res, rs, y, ys, f32, st);
    else
      launch_k2048<NB, 1, true>(x, xs, B, K, W, N, nw, eps, res, rs, y, ys, f32, st);
  } else {
    if (N > 4096)
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
