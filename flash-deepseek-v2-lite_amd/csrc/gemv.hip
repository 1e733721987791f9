// Few-row bf16 GEMV for the small family (bsz 1..8 per launch): weights streamed
// once with 16-byte loads, fp32 accumulation, fused RMSNorm prologue, SwiGLU /
// residual / fp32-logit epilogues.  One wave owns RPW output rows (RPW gate + RPW up
// rows for SwiGLU); lanes split K in 8-element chunks, 4 chunks in flight per row.
#include "common.h"

template <int NB, int RPW, bool SWIGLU>
__global__ __launch_bounds__(256) void gemv_kernel(const bf16_t* __restrict__ x, int64_t xs, int B, int K,
                                                   const bf16_t* __restrict__ W, int N,
                                                   const bf16_t* __restrict__ nw, float eps,
                                                   const bf16_t* __restrict__ res, int64_t rs, void* __restrict__ y,
                                                   int64_t ys, bool out_f32) {
  __shared__ float rsh[NB];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int nch = K >> 3;
  if (nw) {
    for (int b = wv; b < B; b += 4) {
      float ss = 0.f;
      for (int c = lane; c < nch; c += 64) {
        float f[8];
        unpack8(ldg16(x + b * xs + c * 8), f);
#pragma unroll
        for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(f[i], f[i], ss);
      }
      ss = wave_sum(ss);
      if (lane == 0) rsh[b] = rsqrtf(ss / static_cast<float>(K) + eps);
    }
    __syncthreads();
  }
  const int n0 = (blockIdx.x * 4 + wv) * RPW;
  if (n0 >= N) return;

  float acc[RPW][NB];
  float accu[RPW][NB];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[r][b] = accu[r][b] = 0.f;

  const bf16_t* wr = W + (int64_t)n0 * K;
  const bf16_t* wu = W + (int64_t)(N + n0) * K;
  constexpr int U = 4;
  for (int c0 = lane; c0 < nch; c0 += 64 * U) {
    uint4 wg[U][RPW];
    uint4 wup[U][RPW];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + 64 * u;
      if (c < nch) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
          wg[u][r] = ldg16(wr + (int64_t)r * K + c * 8);
          if (SWIGLU) wup[u][r] = ldg16(wu + (int64_t)r * K + c * 8);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + 64 * u;
      if (c >= nch) break;
      float g[8];
      if (nw) unpack8(ldg16(nw + c * 8), g);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (b < B) {
          float xf[8];
          unpack8(ldg16(x + b * xs + c * 8), xf);
          if (nw) {
            const float r_b = rsh[b];
#pragma unroll
            for (int i = 0; i < 8; ++i) xf[i] = rbf(g[i] * rbf(xf[i] * r_b));
          }
#pragma unroll
          for (int r = 0; r < RPW; ++r) {
            acc[r][b] += dot8(wg[u][r], xf);
            if (SWIGLU) accu[r][b] += dot8(wup[u][r], xf);
          }
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      acc[r][b] = wave_sum(acc[r][b]);
      if (SWIGLU) accu[r][b] = wave_sum(accu[r][b]);
    }
  if (lane == 0) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      if (b >= B) break;
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        const int n = n0 + r;
        float v = SWIGLU ? swiglu_bf(acc[r][b], accu[r][b]) : rbf(acc[r][b]);
        if (res) v = rbf(bf2f(res[b * rs + n]) + v);
        if (out_f32)
          reinterpret_cast<float*>(y)[b * ys + n] = v;
        else
          reinterpret_cast<bf16_t*>(y)[b * ys + n] = f2bf(v);
      }
    }
  }
}

template <int NB, int RPW, bool SW>
static void launch_gemv(const bf16_t* x, int64_t xs, int B, int K, const bf16_t* W, int N, const bf16_t* nw,
                        float eps, const bf16_t* res, int64_t rs, void* y, int64_t ys, bool f32, hipStream_t st) {
  const int grid = (N + 4 * RPW - 1) / (4 * RPW);
  hipLaunchKernelGGL((gemv_kernel<NB, RPW, SW>), dim3(grid), dim3(256), 0, st, x, xs, B, K, W, N, nw, eps, res, rs,
                     y, ys, f32);
}

template <int NB, bool SW>
static void launch_gemv_rpw(const bf16_t* x, int64_t xs, int B, int K, const bf16_t* W, int N, const bf16_t* nw,
                            float eps, const bf16_t* res, int64_t rs, void* y, int64_t ys, bool f32, hipStream_t st) {
  // one row per wave keeps >= 2 workgroups per CU on the 2-4K-row projections;
  // larger outputs take two rows per wave for more bytes in flight per wave
  if (N <= 4096)
    launch_gemv<NB, 1, SW>(x, xs, B, K, W, N, nw, eps, res, rs, y, ys, f32, st);
  else
    launch_gemv<NB, 2, SW>(x, xs, B, K, W, N, nw, eps, res, rs, y, ys, f32, st);
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
  hipStream_t st = (hipStream_t)stream;
  const bf16_t* xb = (const bf16_t*)x;
  for (int r0 = 0; r0 < rows; r0 += 8) {
    const int B = rows - r0 < 8 ? rows - r0 : 8;
    const bf16_t* xr = xb + r0 * x_stride;
    const bf16_t* rr = residual ? (const bf16_t*)residual + r0 * res_stride : nullptr;
    void* yr = f32 ? (void*)((float*)y + r0 * y_stride) : (void*)((bf16_t*)y + r0 * y_stride);
#define DSV2_GEMV_NB(NBV)                                                                                        \
  (sw ? launch_gemv_rpw<NBV, true>(xr, x_stride, B, K, (const bf16_t*)W, N, (const bf16_t*)norm_w, eps, rr,     \
                                   res_stride, yr, y_stride, f32, st)                                            \
      : launch_gemv_rpw<NBV, false>(xr, x_stride, B, K, (const bf16_t*)W, N, (const bf16_t*)norm_w, eps, rr,    \
                                    res_stride, yr, y_stride, f32, st))
    if (B == 1)
      DSV2_GEMV_NB(1);
    else if (B == 2)
      DSV2_GEMV_NB(2);
    else if (B <= 4)
      DSV2_GEMV_NB(4);
    else
      DSV2_GEMV_NB(8);
#undef DSV2_GEMV_NB
    int rc = dsv2_launch_status("gemv");
    if (rc) return rc;
  }
  return DSV2_OK;
}
