// MoE for DeepSeek-V2-Lite (64 routed experts, top-6, inter 1408, 2 shared experts):
// router (+ fused post-attention RMSNorm), small-family route-local GEMV kernels,
// batch-family deterministic bucketing and the final weighted combine.
#include "common.h"

namespace {
constexpr int kH = 2048;
constexpr int kE = 64;
constexpr int kTopK = 6;
// gate_up rows per wave (gate + up each); 2 measured faster than 1 on MI355X
constexpr int kGateRPW = 2;
}  // namespace

// Softmax over the 64 router logits of one row (lane e holds logit e) and its top-6,
// published as ids / weights: the probabilities v = exp(x - max) / sum are ranked directly
// -- rank = number of lanes with a larger v, or an equal v at a lower index -- which is the
// order six rounds of argmax with ties to the lower index would produce, in one pass.
__device__ __forceinline__ void topk6_publish(float x, int64_t b, float scaling, int32_t* __restrict__ ids32,
                                              int64_t* __restrict__ ids64, float* __restrict__ wts) {
  const int lane = threadIdx.x & 63;
  const float mx = wave_max(x);
  const float ex = expf(x - mx);
  const float sm = wave_sum(ex);
  const float v = ex / sm;
  int rank = 0;
#pragma unroll 16
  for (int j = 0; j < kE; ++j) {
    const float vj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j));
    rank += (vj > v || (vj == v && j < lane)) ? 1 : 0;
  }
  if (rank < kTopK) {
    if (ids32) ids32[b * kTopK + rank] = lane;
    if (ids64) ids64[b * kTopK + rank] = lane;
    wts[b * kTopK + rank] = v * scaling;
  }
}

// ---------------------------------------------------------------------------
// router: one workgroup per token.  xn = RMSNorm(h); logits = fp32(xn).fp32(W_r)
// (bf16 x bf16 products are exact in fp32); softmax; top-6 with ties to the lower index.
// (A 16-token MFMA tile variant that reads W_r once per tile measured slower on MI355X at
// 64 and 256 rows -- 18.3 vs 11.0 us -- so every row count takes this kernel.)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void router_kernel(const bf16_t* __restrict__ h, int64_t hs,
                                                      const bf16_t* __restrict__ nw, float eps,
                                                      const bf16_t* __restrict__ wr, float scaling,
                                                      bf16_t* __restrict__ xn_out, const float* __restrict__ logits_in,
                                                      int32_t* __restrict__ ids32, int64_t* __restrict__ ids64,
                                                      float* __restrict__ wts) {
  // 16 waves x 4 experts; every router-weight load is issued before the norm
  __shared__ float xs[kH];
  __shared__ float lg[kE];
  __shared__ float red[16];
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  // wave wv takes experts 4 ew .. 4 ew + 3 with ew rotated by the row: the rows' workgroups
  // then sweep the router weights from different places instead of all requesting the same
  // lines at once (256 rows on MI355X: 11.3 -> 9.8 us, C3 step -0.2%; the logits are the
  // same. The same rotation of router_logits_kernel's workgroups made the bsz=64 step 0.5%
  // slower)
  const int ew = (wv + b) & 15;
  if (!logits_in) {
    uint4 wa[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int j = 0; j < 4; ++j) wa[r][j] = ldg16_nt(wr + (int64_t)(ew * 4 + r) * kH + (lane + 64 * j) * 8);
    // norm: 2 elements per thread
    const uint32_t x2 = reinterpret_cast<const uint32_t*>(h + b * hs)[tid];
    float f0 = __uint_as_float(x2 << 16), f1 = __uint_as_float(x2 & 0xffff0000u);
    const float ss = block_sum<16>(f0 * f0 + f1 * f1, red);
    const float rs = rsqrtf(ss / static_cast<float>(kH) + eps);
    const uint32_t g2 = reinterpret_cast<const uint32_t*>(nw)[tid];
    f0 = rbf(__uint_as_float(g2 << 16) * rbf(f0 * rs));
    f1 = rbf(__uint_as_float(g2 & 0xffff0000u) * rbf(f1 * rs));
    xs[2 * tid] = f0;
    xs[2 * tid + 1] = f1;
    if (xn_out) reinterpret_cast<uint32_t*>(xn_out + (int64_t)b * kH)[tid] = pack2(f0, f1);
    __syncthreads();
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float xl[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) xl[i] = xs[(lane + 64 * j) * 8 + i];
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] += dot8(wa[r][j], xl);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = xor_sum(acc[r], off);
    if (lane < 4) lg[ew * 4 + lane] = lane == 0 ? acc[0] : (lane == 1 ? acc[1] : (lane == 2 ? acc[2] : acc[3]));
    __syncthreads();
  } else {
    if (tid < kE) lg[tid] = logits_in[(int64_t)b * kE + tid];
    __syncthreads();
  }
  if (wv == 0) topk6_publish(lg[lane], b, scaling, ids32, ids64, wts);
}

extern "C" int dsv2_router_topk6(const void* h, int64_t h_stride, const void* norm_w, float eps, const void* w_router,
                                 float scaling, int rows, void* xn_out, int32_t* ids32, int64_t* ids64, float* weights,
                                 void* stream) {
  DSV2_REQUIRE(h && norm_w && w_router && weights && (ids32 || ids64), DSV2_E_NULL, "router: null pointer");
  DSV2_REQUIRE(rows >= 0 && rows <= 0x7fffffff / kTopK, DSV2_E_SHAPE, "router: bad rows");
  DSV2_REQUIRE(dsv2_aligned16(h) && h_stride % 8 == 0 && dsv2_aligned16(norm_w) && dsv2_aligned16(w_router) &&
                   (!xn_out || dsv2_aligned16(xn_out)),
               DSV2_E_ALIGN, "router: alignment");
  if (rows == 0) return DSV2_OK;
  hipLaunchKernelGGL(router_kernel, dim3(rows), dim3(1024), 0, (hipStream_t)stream, (const bf16_t*)h, h_stride,
                     (const bf16_t*)norm_w, eps, (const bf16_t*)w_router, scaling, (bf16_t*)xn_out, nullptr, ids32,
                     ids64, weights);
  return dsv2_launch_status("router");
}

extern "C" int dsv2_router_topk6_from_logits(const float* logits, int rows, float scaling, int32_t* ids32,
                                             int64_t* ids64, float* weights, void* stream) {
  DSV2_REQUIRE(logits && weights && (ids32 || ids64), DSV2_E_NULL, "router_from_logits: null pointer");
  DSV2_REQUIRE(rows >= 0, DSV2_E_SHAPE, "router_from_logits: bad rows");
  if (rows == 0) return DSV2_OK;
  hipLaunchKernelGGL(router_kernel, dim3(rows), dim3(1024), 0, (hipStream_t)stream, nullptr, 0, nullptr, 0.f, nullptr,
                     scaling, nullptr, logits, ids32, ids64, weights);
  return dsv2_launch_status("router_from_logits");
}

// ---------------------------------------------------------------------------
// router logits over 16 workgroups per token (one expert per wave, its 4 KB row requested
// before the norm); the softmax + top-6 runs in the consumers (route_gateup_kernel).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void router_logits_kernel(const bf16_t* __restrict__ h, int64_t hs,
                                                            const bf16_t* __restrict__ nw, float eps,
                                                            const bf16_t* __restrict__ wr,
                                                            bf16_t* __restrict__ xn_out, float* __restrict__ logits) {
  __shared__ float xs[kH];
  __shared__ float red[4];
  const int b = blockIdx.x >> 4, part = blockIdx.x & 15;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int e = part * 4 + wv;
  uint4 wa[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) wa[j] = ldg16_nt(wr + (int64_t)e * kH + (lane + 64 * j) * 8);
  float f[8], g[8];
  unpack8(ldg16(h + b * hs + tid * 8), f);
  unpack8(ldg16(nw + tid * 8), g);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(f[i], f[i], ss);
  ss = block_sum<4>(ss, red);
  const float rs = rsqrtf(ss / static_cast<float>(kH) + eps);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    f[i] = rbf(g[i] * rbf(f[i] * rs));
    xs[tid * 8 + i] = f[i];
  }
  if (part == 0 && xn_out) *reinterpret_cast<uint4*>(xn_out + (int64_t)b * kH + tid * 8) = pack8(f);
  __syncthreads();
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) acc += dot8(wa[j], &xs[(lane + 64 * j) * 8]);
  acc = wave_sum(acc);
  if (lane == 0) logits[(int64_t)b * kE + e] = acc;
}

extern "C" int dsv2_router_logits(const void* h, int64_t h_stride, const void* norm_w, float eps,
                                  const void* w_router, int rows, void* xn_out, float* logits, void* stream) {
  DSV2_REQUIRE(h && norm_w && w_router && logits, DSV2_E_NULL, "router_logits: null pointer");
  DSV2_REQUIRE(rows >= 0 && rows <= 0x7fffffff / kE, DSV2_E_SHAPE, "router_logits: bad rows");
  DSV2_REQUIRE(dsv2_aligned16(h) && h_stride % 8 == 0 && dsv2_aligned16(norm_w) && dsv2_aligned16(w_router) &&
                   (!xn_out || dsv2_aligned16(xn_out)),
               DSV2_E_ALIGN, "router_logits: alignment");
  if (rows == 0) return DSV2_OK;
  hipLaunchKernelGGL(router_logits_kernel, dim3(rows * 16), dim3(256), 0, (hipStream_t)stream, (const bf16_t*)h,
                     h_stride, (const bf16_t*)norm_w, eps, (const bf16_t*)w_router, (bf16_t*)xn_out, logits);
  return dsv2_launch_status("router_logits");
}

// ---------------------------------------------------------------------------
// small family: route-local gate_up + SwiGLU.  One workgroup per (route, block of 4*RPW
// output rows); route r: row b = r / nr, slot s = r % nr (s < 6: routed expert, s = 6, 7:
// the shared-expert halves), output row (b * hbuf_routes + s) of hbuf.  Each wave owns RPW
// gate rows and the RPW matching up rows, all requested at once; the row's x is staged in
// LDS once per workgroup.  Only the gate_up body lives in this kernel, so its register
// budget lets every workgroup of a bsz=1 launch be resident at once on MI355X.
// ---------------------------------------------------------------------------
struct RouteGateupArgs {
  int gu_blocks, nr, hbuf_routes, inter;
  const bf16_t* xn;
  int32_t* ids;          // [rows, 6]: read (logits == null) or written (logits != null)
  const float* logits;   // non-null: the row's fp32 router logits, ranked here
  float scaling;
  float* wts;            // written with ids when logits != null
  const bf16_t* wgu;
  const bf16_t* shgu;
  bf16_t* hbuf;
  // fp8 weights (route_gateup_fp8_kernel): e4m3 rows and one fp32 scale per row
  const uint8_t* wgu8;
  const float* sgu;     // [64, 2*inter]
  const uint8_t* shgu8;
  const float* sshgu;   // [2*2*inter]
};



// Expert of routed slot s < 6 from the row's 64 fp32 router logits (lane j holds logit j):
// the lane whose rank -- the number of lanes with a larger logit, or an equal one at a lower
// index -- is s (softmax is monotonic, so rank order is the router's top-6 order, ties to
// the lower index).  Fast path: count only the strictly larger logits; when exactly one lane
// has count s there is no tie at rank s and that lane is the answer.  Otherwise (ties) the
// exact count decides.
__device__ __forceinline__ int routed_expert(float x, int s) {
  const int lane = threadIdx.x & 63;
  int gt = 0;
#pragma unroll 16
  for (int j = 0; j < kE; ++j) gt += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), j)) > x ? 1 : 0;
  const unsigned long long m = __ballot(gt == s);
  if (__popcll(m) == 1) return __ffsll(m) - 1;
  int rank = 0;
  for (int j = 0; j < kE; ++j) {
    const float xj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), j));
    rank += (xj > x || (xj == x && j < lane)) ? 1 : 0;
  }
  return max(__ffsll(__ballot(rank == s)) - 1, 0);  // no lane holds rank s only when logits are NaN
}

// Expert of routed slot s of row b (every wave of the route's workgroups): from the row's ids,
// or ranked from its fp32 router logits (wave 0 of the route's first workgroup then publishes
// the row's ids and softmax weights: `publish`).  Slots s >= 6 (shared halves) return 0.
__device__ __forceinline__ int route_expert(const RouteGateupArgs& a, int b, int s, bool publish, int lane) {
  int e = 0;
  if (s < kTopK && a.logits) {
    const float x = a.logits[(int64_t)b * kE + lane];
    e = routed_expert(x, s);
    if (publish) {
      int rank = 0;
      for (int j = 0; j < kE; ++j) {
        const float xj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), j));
        rank += (xj > x || (xj == x && j < lane)) ? 1 : 0;
      }
      const float mx = wave_max(x);
      const float ex = expf(x - mx);
      const float sm = wave_sum(ex);
      if (rank < kTopK) {
        a.ids[b * kTopK + rank] = lane;
        a.wts[b * kTopK + rank] = ex / sm * a.scaling;
      }
    }
  } else if (s < kTopK) {
    e = min(max(a.ids[b * kTopK + s], 0), kE - 1);
  }
  return e;
}

// Slot of a row's route r (grid order): with the shared halves (nr = 8) they come first, so
// their workgroups -- which need no routing -- are dispatched first and stream their weights
// while the routed ones still wait for the router logits (a launch's workgroups are dispatched
// over ~1.7 us at bsz=1).
__device__ __forceinline__ int route_slot(int r, int nr) { return nr > kTopK ? (r + kTopK) % nr : r; }

// 6 waves per SIMD: all workgroups of a bsz=1 launch (8 routes x 1408 / (2 NWV)) resident together.
// Every wave finds its route's expert itself and requests its weight rows at once (the shared
// halves' workgroups at entry), then each lane reads x for its own K chunks (as bf16, from L2
// / L1) instead of a copy staged in LDS: no LDS and no barrier, so nothing holds a wave's
// weight requests behind the other waves.
template <int RPW, int NWV>
__global__ __launch_bounds__(64 * NWV) __attribute__((amdgpu_waves_per_eu(6, 8))) void route_gateup_kernel(
    const RouteGateupArgs a) {
  const int bx = blockIdx.x % a.gu_blocks, route = blockIdx.x / a.gu_blocks;
  const int b = route / a.nr, s = route_slot(route % a.nr, a.nr);
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int i0 = (bx * NWV + wv) * RPW;
  if (i0 >= a.inter) return;  // inter % RPW == 0: a live wave owns RPW whole rows
  const int e = route_expert(a, b, s, bx == 0 && s == 0 && wv == 0, lane);
  const bf16_t *gp, *up;
  if (s < kTopK) {
    gp = a.wgu + (int64_t)e * 2 * a.inter * kH;
    up = gp + (int64_t)a.inter * kH;
  } else {
    const int half = s - kTopK;
    gp = a.shgu + (int64_t)half * a.inter * kH;
    up = a.shgu + (int64_t)(2 * a.inter + half * a.inter) * kH;
  }
  gp += (int64_t)i0 * kH;
  up += (int64_t)i0 * kH;
  uint4 wg[RPW][4], wu[RPW][4];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      wg[r][j] = ldg16_nt(gp + (int64_t)r * kH + (lane + 64 * j) * 8);
      wu[r][j] = ldg16_nt(up + (int64_t)r * kH + (lane + 64 * j) * 8);
    }
  // x after the weight requests (held across them it would not fit the 80 registers that
  // keep every workgroup of the launch resident)
  uint4 xr[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) xr[j] = ldg16(a.xn + (int64_t)b * kH + (lane + 64 * j) * 8);
  float ag[RPW], au[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) ag[r] = au[r] = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float xl[8];
    unpack8(xr[j], xl);
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      ag[r] += dot8(wg[r][j], xl);
      au[r] += dot8(wu[r][j], xl);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      ag[r] = xor_sum(ag[r], off);
      au[r] = xor_sum(au[r], off);
    }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < RPW; ++r)
      a.hbuf[((int64_t)b * a.hbuf_routes + s) * a.inter + i0 + r] = f2bf(swiglu_bf(ag[r], au[r]));
  }
}

// fp8 weights: the same work per route with every weight row in e4m3 (16 per 16-byte load,
// 2 loads per lane per row, 4 rows of gate and 4 of up per wave) and the row's fp32 scale
// applied to the fp32 dot product before the SwiGLU.
template <int RPW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 8))) void route_gateup_fp8_kernel(
    const RouteGateupArgs a) {
  __shared__ float xs[kH];
  const int bx = blockIdx.x % a.gu_blocks, route = blockIdx.x / a.gu_blocks;
  const int b = route / a.nr, s = route_slot(route % a.nr, a.nr);
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int i0 = (bx * 4 + wv) * RPW;
  const bool live = i0 < a.inter;  // inter % RPW == 0: a live wave owns RPW whole rows
  const uint4 x4 = ldg16(a.xn + (int64_t)b * kH + tid * 8);
  const int e = route_expert(a, b, s, bx == 0 && s == 0 && wv == 0, lane);
  const uint8_t *gp, *up;
  const float *gs, *us;
  if (s < kTopK) {
    gp = a.wgu8 + (int64_t)e * 2 * a.inter * kH;
    up = gp + (int64_t)a.inter * kH;
    gs = a.sgu + (int64_t)e * 2 * a.inter;
    us = gs + a.inter;
  } else {
    const int half = s - kTopK;
    gp = a.shgu8 + (int64_t)half * a.inter * kH;
    up = a.shgu8 + (int64_t)(2 * a.inter + half * a.inter) * kH;
    gs = a.sshgu + half * a.inter;
    us = a.sshgu + 2 * a.inter + half * a.inter;
  }
  const int ir = live ? i0 : 0;  // a dead wave's rows: in bounds, never used
  float sg[RPW], su[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    sg[r] = gs[ir + r];
    su[r] = us[ir + r];
  }
  gp += (int64_t)ir * kH;
  up += (int64_t)ir * kH;
  uint4 wg[RPW][2], wu[RPW][2];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      wg[r][j] = ldg16_nt(gp + (int64_t)r * kH + (lane + 64 * j) * 16);
      wu[r][j] = ldg16_nt(up + (int64_t)r * kH + (lane + 64 * j) * 16);
    }
  asm volatile("" ::: "memory");  // every weight request goes out before x is staged
  {
    float f[8];
    unpack8(x4, f);
#pragma unroll
    for (int i = 0; i < 8; ++i) xs[tid * 8 + i] = f[i];
  }
  __syncthreads();
  if (!live) return;
  float ag[RPW], au[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) ag[r] = au[r] = 0.f;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const float* xl = &xs[(lane + 64 * j) * 16];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      ag[r] += dot16_fp8(wg[r][j], xl);
      au[r] += dot16_fp8(wu[r][j], xl);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      ag[r] = xor_sum(ag[r], off);
      au[r] = xor_sum(au[r], off);
    }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < RPW; ++r)
      a.hbuf[((int64_t)b * a.hbuf_routes + s) * a.inter + i0 + r] = f2bf(swiglu_bf(ag[r] * sg[r], au[r] * su[r]));
  }
}

static int launch_route_gateup(RouteGateupArgs& a, int rows, hipStream_t st, const char* what) {
  constexpr int RPW = kGateRPW;
  DSV2_REQUIRE(a.inter % RPW == 0, DSV2_E_SHAPE, "%s: inter %% %d required", what, RPW);
  // 2-wave workgroups (2,816 at bsz=1; MI355X, C1 step: 1.3629 -> 1.3568 ms against 4 waves,
  // 1.401 with 8, 1.459 with 16, 1.400 with 1)
  constexpr int NWV = 2;
  a.gu_blocks = (a.inter + NWV * RPW - 1) / (NWV * RPW);
  const int64_t grid = (int64_t)rows * a.nr * a.gu_blocks;
  DSV2_REQUIRE(grid <= 0x7fffffff, DSV2_E_SHAPE, "%s: too many rows", what);
  hipLaunchKernelGGL((route_gateup_kernel<RPW, NWV>), dim3((unsigned)grid), dim3(64 * NWV), 0, st, a);
  return dsv2_launch_status(what);
}

extern "C" int dsv2_moe_route_gateup(const void* xn, int rows, const int32_t* ids, const void* w_gate_up,
                                     const void* sh_gate_up, int inter, void* hbuf, void* stream) {
  DSV2_REQUIRE(xn && ids && w_gate_up && hbuf, DSV2_E_NULL, "moe_route_gateup: null pointer");
  const int nr = sh_gate_up ? kTopK + 2 : kTopK;
  DSV2_REQUIRE(rows >= 0 && (int64_t)rows * nr <= 65535 && inter > 0 && inter % 8 == 0, DSV2_E_SHAPE,
               "moe_route_gateup: bad shape");
  DSV2_REQUIRE(dsv2_aligned16(xn) && dsv2_aligned16(w_gate_up) && (!sh_gate_up || dsv2_aligned16(sh_gate_up)),
               DSV2_E_ALIGN, "moe_route_gateup: alignment");
  if (rows == 0) return DSV2_OK;
  RouteGateupArgs a{};
  a.nr = nr;
  a.hbuf_routes = nr;
  a.inter = inter;
  a.xn = (const bf16_t*)xn;
  a.ids = const_cast<int32_t*>(ids);
  a.wgu = (const bf16_t*)w_gate_up;
  a.shgu = (const bf16_t*)sh_gate_up;
  a.hbuf = (bf16_t*)hbuf;
  return launch_route_gateup(a, rows, (hipStream_t)stream, "moe_route_gateup");
}

extern "C" int dsv2_moe_route_gateup_logits(const void* xn, int rows, const float* logits, float scaling,
                                            int32_t* ids, float* weights, const void* w_gate_up,
                                            const void* sh_gate_up, int inter, void* hbuf, void* stream) {
  DSV2_REQUIRE(xn && logits && ids && weights && w_gate_up && hbuf, DSV2_E_NULL,
               "moe_route_gateup_logits: null pointer");
  const int nr = sh_gate_up ? kTopK + 2 : kTopK;
  DSV2_REQUIRE(rows >= 0 && (int64_t)rows * nr <= 65535 && inter > 0 && inter % 8 == 0, DSV2_E_SHAPE,
               "moe_route_gateup_logits: bad shape");
  DSV2_REQUIRE(dsv2_aligned16(xn) && dsv2_aligned16(w_gate_up) && (!sh_gate_up || dsv2_aligned16(sh_gate_up)),
               DSV2_E_ALIGN, "moe_route_gateup_logits: alignment");
  if (rows == 0) return DSV2_OK;
  RouteGateupArgs a{};
  a.nr = nr;
  a.hbuf_routes = kTopK + 2;
  a.inter = inter;
  a.xn = (const bf16_t*)xn;
  a.ids = ids;
  a.logits = logits;
  a.scaling = scaling;
  a.wts = weights;
  a.wgu = (const bf16_t*)w_gate_up;
  a.shgu = (const bf16_t*)sh_gate_up;
  a.hbuf = (bf16_t*)hbuf;
  return launch_route_gateup(a, rows, (hipStream_t)stream, "moe_route_gateup_logits");
}

extern "C" int dsv2_moe_route_gateup_logits_fp8(const void* xn, int rows, const float* logits, float scaling,
                                                int32_t* ids, float* weights, const uint8_t* w_gate_up,
                                                const float* gate_up_scale, const uint8_t* sh_gate_up,
                                                const float* sh_gate_up_scale, int inter, void* hbuf, void* stream) {
  constexpr int RPW = 4;
  DSV2_REQUIRE(xn && logits && ids && weights && w_gate_up && gate_up_scale && hbuf, DSV2_E_NULL,
               "moe_route_gateup_logits_fp8: null pointer");
  DSV2_REQUIRE(!sh_gate_up == !sh_gate_up_scale, DSV2_E_NULL,
               "moe_route_gateup_logits_fp8: shared weights and their scales go together");
  const int nr = sh_gate_up ? kTopK + 2 : kTopK;
  DSV2_REQUIRE(rows >= 0 && (int64_t)rows * nr <= 65535 && inter > 0 && inter % RPW == 0, DSV2_E_SHAPE,
               "moe_route_gateup_logits_fp8: bad shape (inter %% 4 == 0)");
  DSV2_REQUIRE(dsv2_aligned16(xn) && dsv2_aligned16(w_gate_up) && (!sh_gate_up || dsv2_aligned16(sh_gate_up)),
               DSV2_E_ALIGN, "moe_route_gateup_logits_fp8: alignment");
  if (rows == 0) return DSV2_OK;
  RouteGateupArgs a{};
  a.nr = nr;
  a.hbuf_routes = kTopK + 2;
  a.inter = inter;
  a.xn = (const bf16_t*)xn;
  a.ids = ids;
  a.logits = logits;
  a.scaling = scaling;
  a.wts = weights;
  a.wgu8 = w_gate_up;
  a.sgu = gate_up_scale;
  a.shgu8 = sh_gate_up;
  a.sshgu = sh_gate_up_scale;
  a.hbuf = (bf16_t*)hbuf;
  a.gu_blocks = (inter + 4 * RPW - 1) / (4 * RPW);
  const int64_t grid = (int64_t)rows * nr * a.gu_blocks;
  hipLaunchKernelGGL(route_gateup_fp8_kernel<RPW>, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, a);
  return dsv2_launch_status("moe_route_gateup_logits_fp8");
}

// ---------------------------------------------------------------------------
// small family: down projection of every route of a token + weighted top-6 sum
// (+ shared halves, + residual), deterministic (no atomics). grid (2048/(4*RPW), rows)
// ---------------------------------------------------------------------------
template <int NR>
__global__ __launch_bounds__(256) void route_down_kernel(const bf16_t* __restrict__ hbuf,
                                                         const int32_t* __restrict__ ids,
                                                         const float* __restrict__ wts,
                                                         const bf16_t* __restrict__ wd,
                                                         const bf16_t* __restrict__ shd, int inter, int hbuf_routes,
                                                         const bf16_t* __restrict__ shared_y,
                                                         const bf16_t* __restrict__ res, bf16_t* __restrict__ out) {
  // workgroup: output rows j0, j0+1 of token b; wave w: routes 2w, 2w+1 (all chunks of K = inter)
  __shared__ float part[8][2];
  const int b = blockIdx.y;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int j0 = blockIdx.x * 2;
  const int nch = inter >> 3;
  constexpr int kMaxCh = 3;  // chunks per lane: ceil(176 / 64) for inter = 1408
  // Loads are issued in dependency order with no wait between independent ones: both
  // routes' expert ids (slots clamped), the residual / shared output (pinned, so they stay
  // ahead of the weights), then every weight and hbuf chunk (chunk indices clamped, masked
  // where used).
  int eid[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) eid[q] = ids[b * kTopK + min(2 * wv + q, kTopK - 1)];
  const int jr = j0 + (threadIdx.x & 1);
  bf16_t resb = 0, shb = 0;
  resb = (res ? res : hbuf)[res ? (int64_t)b * kH + jr : 0];
  shb = (shared_y ? shared_y : hbuf)[shared_y ? (int64_t)b * kH + jr : 0];
  if (2 * wv < NR) {
    const bf16_t* wrow[2];
    int64_t wstride[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int s = 2 * wv + q;
      if (s < kTopK) {
        wrow[q] = wd + (int64_t)min(max(eid[q], 0), kE - 1) * kH * inter + (int64_t)j0 * inter;
        wstride[q] = inter;
      } else {
        wrow[q] = shd + (int64_t)(s - kTopK) * inter + (int64_t)j0 * 2 * inter;
        wstride[q] = 2 * inter;
      }
    }
    uint4 w[2][2][kMaxCh], x[2][kMaxCh];
#pragma unroll
    for (int k = 0; k < kMaxCh; ++k) {
      const int c = min(lane + 64 * k, nch - 1);
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        x[q][k] = ldg16(hbuf + ((int64_t)b * hbuf_routes + 2 * wv + q) * inter + c * 8);
#pragma unroll
        for (int r = 0; r < 2; ++r) w[q][r][k] = ldg16_nt(wrow[q] + r * wstride[q] + c * 8);
      }
    }
    pin(resb);
    pin(shb);
    float acc[2][2];
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        float a = 0.f;
#pragma unroll
        for (int k = 0; k < kMaxCh; ++k) {
          float hx[8];
          unpack8(x[q][k], hx);
          const float d = dot8(w[q][r][k], hx);
          a += lane + 64 * k < nch ? d : 0.f;
        }
        acc[q][r] = a;
      }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int r = 0; r < 2; ++r) acc[q][r] = xor_sum(acc[q][r], off);
    if (lane == 0) {
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int r = 0; r < 2; ++r) part[2 * wv + q][r] = acc[q][r];
    }
  }
  __syncthreads();
  if (threadIdx.x < 2) {
    const int r = threadIdx.x;
    float routed = 0.f;
    const float rv = res ? bf2f(resb) : 0.f;
    const float shv = shared_y ? bf2f(shb) : 0.f;
#pragma unroll
    for (int s = 0; s < kTopK; ++s) routed += wts[b * kTopK + s] * rbf(part[s][r]);
    float y = rbf(routed);
    if (NR > kTopK) y = rbf(y + rbf(part[kTopK][r] + part[kTopK + 1][r]));
    else if (shared_y) y = rbf(y + shv);
    if (res) y = rbf(rv + y);
    out[(int64_t)b * kH + j0 + r] = f2bf(y);
  }
}

// fp8 weights: the same work with every down row in e4m3 (16 weights and 16 hbuf values per
// lane chunk, at most 2 chunks per lane) and the row's fp32 scale on the fp32 dot product.
template <int NR>
__global__ __launch_bounds__(256) void route_down_fp8_kernel(const bf16_t* __restrict__ hbuf,
                                                             const int32_t* __restrict__ ids,
                                                             const float* __restrict__ wts,
                                                             const uint8_t* __restrict__ wd,
                                                             const float* __restrict__ sd,
                                                             const uint8_t* __restrict__ shd,
                                                             const float* __restrict__ ssh, int inter,
                                                             int hbuf_routes, const bf16_t* __restrict__ res,
                                                             bf16_t* __restrict__ out) {
  __shared__ float part[8][2];
  const int b = blockIdx.y;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int j0 = blockIdx.x * 2;
  const int nch = inter >> 4;
  constexpr int kMaxCh = 2;  // chunks of 16 per lane: ceil(88 / 64) for inter = 1408
  int eid[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) eid[q] = ids[b * kTopK + min(2 * wv + q, kTopK - 1)];
  const int jr = j0 + (threadIdx.x & 1);
  bf16_t resb = (res ? res : hbuf)[res ? (int64_t)b * kH + jr : 0];
  if (2 * wv < NR) {
    const uint8_t* wrow[2];
    int64_t wstride[2];
    float sc[2][2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int s = 2 * wv + q;
      if (s < kTopK) {
        const int e = min(max(eid[q], 0), kE - 1);
        wrow[q] = wd + (int64_t)e * kH * inter + (int64_t)j0 * inter;
        wstride[q] = inter;
        sc[q][0] = sd[(int64_t)e * kH + j0];
        sc[q][1] = sd[(int64_t)e * kH + j0 + 1];
      } else {
        wrow[q] = shd + (int64_t)(s - kTopK) * inter + (int64_t)j0 * 2 * inter;
        wstride[q] = 2 * inter;
        sc[q][0] = ssh[j0];
        sc[q][1] = ssh[j0 + 1];
      }
    }
    uint4 w[2][2][kMaxCh], x[2][kMaxCh][2];
#pragma unroll
    for (int k = 0; k < kMaxCh; ++k) {
      const int c = min(lane + 64 * k, nch - 1);
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const bf16_t* hx = hbuf + ((int64_t)b * hbuf_routes + 2 * wv + q) * inter + c * 16;
        x[q][k][0] = ldg16(hx);
        x[q][k][1] = ldg16(hx + 8);
#pragma unroll
        for (int r = 0; r < 2; ++r) w[q][r][k] = ldg16_nt(wrow[q] + r * wstride[q] + c * 16);
      }
    }
    pin(resb);
    float acc[2][2];
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        float a = 0.f;
#pragma unroll
        for (int k = 0; k < kMaxCh; ++k) {
          float hx[16];
          unpack8(x[q][k][0], hx);
          unpack8(x[q][k][1], hx + 8);
          const float d = dot16_fp8(w[q][r][k], hx);
          a += lane + 64 * k < nch ? d : 0.f;
        }
        acc[q][r] = a;
      }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int r = 0; r < 2; ++r) acc[q][r] = xor_sum(acc[q][r], off);
    if (lane == 0) {
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int r = 0; r < 2; ++r) part[2 * wv + q][r] = acc[q][r] * sc[q][r];
    }
  }
  __syncthreads();
  if (threadIdx.x < 2) {
    const int r = threadIdx.x;
    float routed = 0.f;
    const float rv = res ? bf2f(resb) : 0.f;
#pragma unroll
    for (int s = 0; s < kTopK; ++s) routed += wts[b * kTopK + s] * rbf(part[s][r]);
    float y = rbf(routed);
    if (NR > kTopK) y = rbf(y + rbf(part[kTopK][r] + part[kTopK + 1][r]));
    if (res) y = rbf(rv + y);
    out[(int64_t)b * kH + j0 + r] = f2bf(y);
  }
}

extern "C" int dsv2_moe_route_down_fp8(const void* hbuf, int rows, const int32_t* ids, const float* weights,
                                       const uint8_t* w_down, const float* down_scale, const uint8_t* sh_down,
                                       const float* sh_down_scale, int inter, int hbuf_routes, const void* residual,
                                       void* out, void* stream) {
  DSV2_REQUIRE(hbuf && ids && weights && w_down && down_scale && out, DSV2_E_NULL, "moe_route_down_fp8: null pointer");
  DSV2_REQUIRE(!sh_down == !sh_down_scale, DSV2_E_NULL, "moe_route_down_fp8: shared weights and their scales go together");
  DSV2_REQUIRE(rows >= 0 && rows <= 65535 && inter > 0 && inter % 16 == 0 && inter <= 2 * 64 * 16, DSV2_E_SHAPE,
               "moe_route_down_fp8: bad shape (inter %% 16 == 0, inter <= 2048)");
  DSV2_REQUIRE(dsv2_aligned16(hbuf) && dsv2_aligned16(w_down) && (!sh_down || dsv2_aligned16(sh_down)),
               DSV2_E_ALIGN, "moe_route_down_fp8: alignment");
  DSV2_REQUIRE(hbuf_routes >= (sh_down ? kTopK + 2 : kTopK) && hbuf_routes <= kTopK + 2, DSV2_E_SHAPE,
               "moe_route_down_fp8: hbuf_routes must cover the routes read");
  if (rows == 0) return DSV2_OK;
  const dim3 grid(kH / 2, rows);
  if (sh_down)
    hipLaunchKernelGGL((route_down_fp8_kernel<kTopK + 2>), grid, dim3(256), 0, (hipStream_t)stream,
                       (const bf16_t*)hbuf, ids, weights, w_down, down_scale, sh_down, sh_down_scale, inter,
                       hbuf_routes, (const bf16_t*)residual, (bf16_t*)out);
  else
    hipLaunchKernelGGL((route_down_fp8_kernel<kTopK>), grid, dim3(256), 0, (hipStream_t)stream, (const bf16_t*)hbuf,
                       ids, weights, w_down, down_scale, nullptr, nullptr, inter, hbuf_routes,
                       (const bf16_t*)residual, (bf16_t*)out);
  return dsv2_launch_status("moe_route_down_fp8");
}

extern "C" int dsv2_moe_route_down(const void* hbuf, int rows, const int32_t* ids, const float* weights,
                                   const void* w_down, const void* sh_down, int inter, int hbuf_routes,
                                   const void* shared_y, const void* residual, void* out, void* stream) {
  DSV2_REQUIRE(hbuf && ids && weights && w_down && out, DSV2_E_NULL, "moe_route_down: null pointer");
  DSV2_REQUIRE(rows >= 0 && rows <= 65535 && inter > 0 && inter % 8 == 0 && inter <= 3 * 64 * 8, DSV2_E_SHAPE,
               "moe_route_down: bad shape (inter %% 8 == 0, inter <= 1536)");
  DSV2_REQUIRE(dsv2_aligned16(hbuf) && dsv2_aligned16(w_down) && (!sh_down || dsv2_aligned16(sh_down)),
               DSV2_E_ALIGN, "moe_route_down: alignment");
  DSV2_REQUIRE(!(sh_down && shared_y), DSV2_E_FLAGS, "moe_route_down: sh_down and shared_y are exclusive");
  DSV2_REQUIRE(hbuf_routes >= (sh_down ? kTopK + 2 : kTopK) && hbuf_routes <= kTopK + 2, DSV2_E_SHAPE,
               "moe_route_down: hbuf_routes must cover the routes read");
  if (rows == 0) return DSV2_OK;
  const dim3 grid(kH / 2, rows);
  if (sh_down)
    hipLaunchKernelGGL((route_down_kernel<kTopK + 2>), grid, dim3(256), 0, (hipStream_t)stream, (const bf16_t*)hbuf,
                       ids, weights, (const bf16_t*)w_down, (const bf16_t*)sh_down, inter, hbuf_routes, nullptr,
                       (const bf16_t*)residual, (bf16_t*)out);
  else
    hipLaunchKernelGGL((route_down_kernel<kTopK>), grid, dim3(256), 0, (hipStream_t)stream, (const bf16_t*)hbuf, ids,
                       weights, (const bf16_t*)w_down, nullptr, inter, hbuf_routes, (const bf16_t*)shared_y,
                       (const bf16_t*)residual, (bf16_t*)out);
  return dsv2_launch_status("moe_route_down");
}

// ---------------------------------------------------------------------------
// batch family bucketing: one workgroup of 16 waves.  Routes are processed in
// 64-route chunks; a route's slot = expert start + routes of the same expert in
// earlier chunks + earlier lanes of its own chunk, so the order is stable in the
// route index and the result is deterministic (no atomics).  Only the per-chunk counts
// live in LDS (96 KB at the 49,152-route maximum, the prefill's 8192-row chunks); a route's
// rank inside its chunk is recomputed from the same ballots when it is placed.
// ---------------------------------------------------------------------------
constexpr int kMaxRoutes = 49152;
constexpr int kMaxChunks = kMaxRoutes / 64;

// expert of route r (kE when r is past the routes), and its rank among the lanes of its
// 64-route chunk that hold the same expert; `last` is set on the chunk's last such lane
__device__ __forceinline__ int chunk_rank(int e, int lane, bool& last) {
  // lanes holding the same expert: intersect, over the 7 bits of e, the ballots that agree
  unsigned long long same = ~0ull;
#pragma unroll
  for (int bit = 0; bit < 7; ++bit) {
    const unsigned long long bl = __ballot((e >> bit) & 1);
    same &= ((e >> bit) & 1) ? bl : ~bl;
  }
  const unsigned long long below = (1ull << lane) - 1ull;
  last = __popcll(same & ~below) == 1;
  return __popcll(same & below);
}
__device__ __forceinline__ int route_rank(const int32_t* __restrict__ ids, int r, int R, int lane, int& e,
                                          bool& last) {
  e = r < R ? min(max(ids[r], 0), kE - 1) : kE;
  return chunk_rank(e, lane, last);
}

__global__ __launch_bounds__(1024) void bucket_kernel(const int32_t* __restrict__ ids, int R, int tile_tokens,
                                                      int32_t* __restrict__ sorted_routes,
                                                      int32_t* __restrict__ route_pos, int32_t* __restrict__ tiles,
                                                      int32_t* __restrict__ num_tiles) {
  __shared__ uint16_t hist[kMaxChunks][kE];  // per-chunk counts, then exclusive prefix over chunks
  __shared__ int start[kE], tstart[kE], total[kE];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int nchunks = (R + 63) / 64;
  // a wave's chunks wv and wv + 16 (every chunk up to 2,048 routes): their ids are requested
  // before the histogram is cleared (clamped indices; no routes: num_tiles' word, unused) and
  // their (expert, rank) kept for the placement pass instead of being read and ranked again
  const int32_t* idp = R > 0 ? ids : num_tiles;
  int ek[2], bk[2] = {0, 0};
#pragma unroll
  for (int k = 0; k < 2; ++k) ek[k] = idp[max(min((wv + 16 * k) * 64 + lane, R - 1), 0)];
  for (int i = tid; i < nchunks * kE; i += 1024) hist[i / kE][i % kE] = 0;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    pin(ek[k]);
    ek[k] = (wv + 16 * k) * 64 + lane < R ? min(max(ek[k], 0), kE - 1) : kE;
  }
  __syncthreads();
  for (int c = wv; c < nchunks; c += 16) {
    int e;
    bool last;
    int before;
    if (c == wv) {
      e = ek[0];
      before = bk[0] = chunk_rank(e, lane, last);
    } else if (c == wv + 16) {
      e = ek[1];
      before = bk[1] = chunk_rank(e, lane, last);
    } else {
      before = route_rank(ids, c * 64 + lane, R, lane, e, last);
    }
    if (c * 64 + lane < R && last) hist[c][e] = (uint16_t)(before + 1);
  }
  __syncthreads();
  if (tid < kE) {
    int run = 0;
    for (int c = 0; c < nchunks; ++c) {
      const int t = hist[c][tid];
      hist[c][tid] = (uint16_t)run;
      run += t;
    }
    total[tid] = run;
  }
  __syncthreads();
  if (wv == 0) {
    const int tot = total[lane];
    const int nt = (tot + tile_tokens - 1) / tile_tokens;
    int incl = tot, tincl = nt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int a = __shfl_up(incl, o, 64), bt = __shfl_up(tincl, o, 64);
      if (lane >= o) {
        incl += a;
        tincl += bt;
      }
    }
    start[lane] = incl - tot;
    tstart[lane] = tincl - nt;
    if (lane == 63) num_tiles[0] = tincl;
  }
  __syncthreads();
  for (int c = wv; c < nchunks; c += 16) {
    const int r = c * 64 + lane;
    int e, before;
    if (c == wv) {
      e = ek[0];
      before = bk[0];
    } else if (c == wv + 16) {
      e = ek[1];
      before = bk[1];
    } else {
      bool last;
      before = route_rank(ids, r, R, lane, e, last);
    }
    if (r < R) {
      const int p = start[e] + hist[c][e] + before;
      sorted_routes[p] = r;
      route_pos[r] = p;
    }
  }
  for (int e = wv; e < kE; e += 16) {
    const int tot = total[e];
    const int nt = (tot + tile_tokens - 1) / tile_tokens;
    for (int i = lane; i < nt; i += 64) {
      int4 t;
      t.x = e;
      t.y = start[e] + i * tile_tokens;
      t.z = min(tile_tokens, tot - i * tile_tokens);
      t.w = 0;
      reinterpret_cast<int4*>(tiles)[tstart[e] + i] = t;
    }
  }
}

extern "C" int dsv2_moe_bucket(const int32_t* ids, int rows, int tile_tokens, int32_t* sorted_routes,
                               int32_t* route_pos, int32_t* tiles, int32_t* num_tiles, void* stream) {
  DSV2_REQUIRE(ids && sorted_routes && route_pos && tiles && num_tiles, DSV2_E_NULL, "moe_bucket: null pointer");
  DSV2_REQUIRE(rows >= 0 && rows * kTopK <= kMaxRoutes && tile_tokens >= 1 && tile_tokens <= 256, DSV2_E_SHAPE,
               "moe_bucket: rows*6 must be <= %d (got %d)", kMaxRoutes, rows * kTopK);
  DSV2_REQUIRE(dsv2_aligned16(tiles), DSV2_E_ALIGN, "moe_bucket: tiles must be 16-byte aligned");
  hipLaunchKernelGGL(bucket_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, ids, rows * kTopK, tile_tokens,
                     sorted_routes, route_pos, tiles, num_tiles);
  return dsv2_launch_status("moe_bucket");
}

// ---------------------------------------------------------------------------
// bucketing over many workgroups (prefill chunks): the same counting sort as bucket_kernel,
// bit for bit, in three launches -- per-chunk histograms (one wave per 64-route chunk), the
// exclusive prefix over chunks per expert with the tile table (one workgroup), the stable
// scatter (one wave per chunk).  The histograms live in the caller's workspace (int32
// [chunks][64], then the 64 expert starts).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void bucket_hist_kernel(const int32_t* __restrict__ ids, int R,
                                                           int32_t* __restrict__ hist) {
  __shared__ int cnt[16][kE];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int c = blockIdx.x * 16 + wv, nchunks = (R + 63) / 64;
  const bool live = c < nchunks;  // per wave
  int e = kE, before = 0;
  bool last = false;
  if (live) before = route_rank(ids, c * 64 + lane, R, lane, e, last);
  cnt[wv][lane] = 0;
  __syncthreads();  // the lanes' count writes below land after every zero
  if (live && c * 64 + lane < R && last) cnt[wv][e] = before + 1;
  __syncthreads();
  if (live) hist[(int64_t)c * kE + lane] = cnt[wv][lane];
}

__global__ __launch_bounds__(1024) void bucket_scan_kernel(int R, int tile_tokens, int32_t* __restrict__ hist,
                                                           int32_t* __restrict__ tiles, int32_t* __restrict__ num_tiles) {
  __shared__ int start[kE], tstart[kE], total[kE];
  __shared__ int segtot[16][kE];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int nchunks = (R + 63) / 64;
  {
    // wave wv owns a segment of the chunks for all 64 experts (lane = expert): its counts are
    // requested at once (coalesced rows of hist), the segments' totals meet in LDS
    constexpr int kSegMax = kMaxChunks / 16;
    const int seg = (nchunks + 15) / 16, c0 = wv * seg;
    int v[kSegMax];
#pragma unroll
    for (int k = 0; k < kSegMax; ++k) {  // unconditional loads (clamped rows), masked values
      const int c = c0 + k;
      const int x = hist[(int64_t)min(c, max(nchunks - 1, 0)) * kE + lane];
      v[k] = (k < seg && c < nchunks) ? x : 0;
    }
    int loc = 0;
#pragma unroll
    for (int k = 0; k < kSegMax; ++k) loc += v[k];
    segtot[wv][lane] = loc;
    __syncthreads();
    int run = 0, all = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int t = segtot[j][lane];
      run += j < wv ? t : 0;
      all += t;
    }
#pragma unroll
    for (int k = 0; k < kSegMax; ++k) {
      const int c = c0 + k;
      if (k < seg && c < nchunks) hist[(int64_t)c * kE + lane] = run;
      run += v[k];
    }
    if (wv == 0) total[lane] = all;
  }
  __syncthreads();
  if (wv == 0) {
    const int tot = total[lane];
    const int nt = (tot + tile_tokens - 1) / tile_tokens;
    int incl = tot, tincl = nt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int a = __shfl_up(incl, o, 64), bt = __shfl_up(tincl, o, 64);
      if (lane >= o) {
        incl += a;
        tincl += bt;
      }
    }
    start[lane] = incl - tot;
    tstart[lane] = tincl - nt;
    hist[(int64_t)nchunks * kE + lane] = incl - tot;  // the expert starts, for the scatter
    if (lane == 63) num_tiles[0] = tincl;
  }
  __syncthreads();
  for (int e = wv; e < kE; e += 16) {
    const int tot = total[e];
    const int nt = (tot + tile_tokens - 1) / tile_tokens;
    for (int i = lane; i < nt; i += 64) {
      int4 t;
      t.x = e;
      t.y = start[e] + i * tile_tokens;
      t.z = min(tile_tokens, tot - i * tile_tokens);
      t.w = 0;
      reinterpret_cast<int4*>(tiles)[tstart[e] + i] = t;
    }
  }
}

__global__ __launch_bounds__(1024) void bucket_scatter_kernel(const int32_t* __restrict__ ids, int R,
                                                              const int32_t* __restrict__ hist,
                                                              int32_t* __restrict__ sorted_routes,
                                                              int32_t* __restrict__ route_pos) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int c = blockIdx.x * 16 + wv, nchunks = (R + 63) / 64;
  if (c >= nchunks) return;
  const int r = c * 64 + lane;
  int e;
  bool last;
  const int before = route_rank(ids, r, R, lane, e, last);
  if (r < R) {
    const int p = hist[(int64_t)nchunks * kE + e] + hist[(int64_t)c * kE + e] + before;
    sorted_routes[p] = r;
    route_pos[r] = p;
  }
}

extern "C" int64_t dsv2_moe_bucket_workspace_size(int rows) {
  const int64_t nchunks = ((int64_t)max(rows, 0) * kTopK + 63) / 64;
  return (nchunks + 1) * kE * (int64_t)sizeof(int32_t);
}

extern "C" int dsv2_moe_bucket_wide(const int32_t* ids, int rows, int tile_tokens, int32_t* sorted_routes,
                                    int32_t* route_pos, int32_t* tiles, int32_t* num_tiles, void* workspace,
                                    int64_t workspace_bytes, void* stream) {
  DSV2_REQUIRE(ids && sorted_routes && route_pos && tiles && num_tiles && workspace, DSV2_E_NULL,
               "moe_bucket_wide: null pointer");
  DSV2_REQUIRE(rows >= 0 && rows * kTopK <= kMaxRoutes && tile_tokens >= 1 && tile_tokens <= 256, DSV2_E_SHAPE,
               "moe_bucket_wide: rows*6 must be <= %d (got %d)", kMaxRoutes, rows * kTopK);
  DSV2_REQUIRE(workspace_bytes >= dsv2_moe_bucket_workspace_size(rows), DSV2_E_SHAPE,
               "moe_bucket_wide: workspace of %lld bytes, %lld needed", (long long)workspace_bytes,
               (long long)dsv2_moe_bucket_workspace_size(rows));
  DSV2_REQUIRE(dsv2_aligned16(tiles) && dsv2_aligned16(workspace), DSV2_E_ALIGN, "moe_bucket_wide: alignment");
  const int R = rows * kTopK, nchunks = (R + 63) / 64;
  int32_t* hist = reinterpret_cast<int32_t*>(workspace);
  const int groups = (nchunks + 15) / 16;
  hipStream_t st = (hipStream_t)stream;
  if (groups > 0) hipLaunchKernelGGL(bucket_hist_kernel, dim3(groups), dim3(1024), 0, st, ids, R, hist);
  hipLaunchKernelGGL(bucket_scan_kernel, dim3(1), dim3(1024), 0, st, R, tile_tokens, hist, tiles, num_tiles);
  if (groups > 0)
    hipLaunchKernelGGL(bucket_scatter_kernel, dim3(groups), dim3(1024), 0, st, ids, R, hist, sorted_routes, route_pos);
  return dsv2_launch_status("moe_bucket_wide");
}

// ---------------------------------------------------------------------------
// combine: one workgroup per token (256 threads x 8 elements)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void moe_combine_kernel(const bf16_t* __restrict__ ys,
                                                          const int32_t* __restrict__ route_pos,
                                                          const float* __restrict__ wts,
                                                          const bf16_t* __restrict__ shared,
                                                          const float* __restrict__ shared_parts,
                                                          const bf16_t* __restrict__ res, bf16_t* __restrict__ out,
                                                          const bf16_t* __restrict__ nw, float eps,
                                                          bf16_t* __restrict__ xn) {
  __shared__ float red[4];
  const int b = blockIdx.x, tid = threadIdx.x;
  // every operand is requested up front -- an absent one reads the start of ys instead and is
  // not used -- and the six expert rows right after their positions: two dependent round
  // trips per row instead of one per operand
  const bf16_t* shp = shared ? shared + (int64_t)b * kH : ys;
  const float* sp0 = shared_parts ? shared_parts + (int64_t)b * kH : reinterpret_cast<const float*>(ys);
  const float* sp1 = shared_parts ? shared_parts + ((int64_t)gridDim.x + b) * kH : reinterpret_cast<const float*>(ys);
  const bf16_t* rsp = res ? res + (int64_t)b * kH : ys;
  const bf16_t* nwp = nw ? nw : ys;
  int pr[kTopK];
  float wr[kTopK];
#pragma unroll
  for (int s = 0; s < kTopK; ++s) {
    pr[s] = route_pos[b * kTopK + s];
    wr[s] = wts[b * kTopK + s];
  }
  const uint4 shq = ldg16(shp + tid * 8);
  const float4 a0 = reinterpret_cast<const float4*>(sp0 + tid * 8)[0], a1 = reinterpret_cast<const float4*>(sp0 + tid * 8)[1];
  const float4 b0 = reinterpret_cast<const float4*>(sp1 + tid * 8)[0], b1 = reinterpret_cast<const float4*>(sp1 + tid * 8)[1];
  const uint4 rq = ldg16(rsp + tid * 8);
  const uint4 nq = ldg16(nwp + tid * 8);
  uint4 yq[kTopK];
#pragma unroll
  for (int s = 0; s < kTopK; ++s) yq[s] = ldg16(ys + (int64_t)pr[s] * kH + tid * 8);
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;
#pragma unroll
  for (int s = 0; s < kTopK; ++s) {
    float f[8];
    unpack8(yq[s], f);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] += wr[s] * f[i];
  }
  float y[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) y[i] = rbf(acc[i]);
  if (shared) {
    float f[8];
    unpack8(shq, f);
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = rbf(y[i] + f[i]);
  } else if (shared_parts) {  // shared = bf16(half 0 + half 1), the fp32 partials of its down GEMM
    const float sh[8] = {a0.x + b0.x, a0.y + b0.y, a0.z + b0.z, a0.w + b0.w,
                         a1.x + b1.x, a1.y + b1.y, a1.z + b1.z, a1.w + b1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = rbf(y[i] + rbf(sh[i]));
  }
  if (res) {
    float f[8];
    unpack8(rq, f);
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = rbf(f[i] + y[i]);
  }
  *reinterpret_cast<uint4*>(out + (int64_t)b * kH + tid * 8) = pack8(y);
  if (nw) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(y[i], y[i], ss);
    ss = block_sum<4>(ss, red);
    const float rs = rsqrtf(ss / static_cast<float>(kH) + eps);
    float g[8];
    unpack8(nq, g);
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = g[i] * rbf(y[i] * rs);
    *reinterpret_cast<uint4*>(xn + (int64_t)b * kH + tid * 8) = pack8(y);
  }
}

extern "C" int dsv2_moe_combine(const void* ysorted, const int32_t* route_pos, const float* weights, int rows,
                                const void* shared, const void* residual, void* out, const void* next_norm_w, float eps,
                                void* xn_out, void* stream) {
  DSV2_REQUIRE(ysorted && route_pos && weights && out && (!next_norm_w || xn_out), DSV2_E_NULL,
               "moe_combine: null pointer");
  DSV2_REQUIRE(rows >= 0, DSV2_E_SHAPE, "moe_combine: bad rows");
  DSV2_REQUIRE(dsv2_aligned16(ysorted) && dsv2_aligned16(out) && (!shared || dsv2_aligned16(shared)) &&
                   (!residual || dsv2_aligned16(residual)) && (!xn_out || dsv2_aligned16(xn_out)),
               DSV2_E_ALIGN, "moe_combine: alignment");
  if (rows == 0) return DSV2_OK;
  hipLaunchKernelGGL(moe_combine_kernel, dim3(rows), dim3(256), 0, (hipStream_t)stream, (const bf16_t*)ysorted,
                     route_pos, weights, (const bf16_t*)shared, nullptr, (const bf16_t*)residual, (bf16_t*)out,
                     (const bf16_t*)next_norm_w, eps, (bf16_t*)xn_out);
  return dsv2_launch_status("moe_combine");
}

extern "C" int dsv2_moe_combine_parts(const void* ysorted, const int32_t* route_pos, const float* weights, int rows,
                                      const float* shared_parts, const void* residual, void* out,
                                      const void* next_norm_w, float eps, void* xn_out, void* stream) {
  DSV2_REQUIRE(ysorted && route_pos && weights && shared_parts && out && (!next_norm_w || xn_out), DSV2_E_NULL,
               "moe_combine_parts: null pointer");
  DSV2_REQUIRE(rows >= 0, DSV2_E_SHAPE, "moe_combine_parts: bad rows");
  DSV2_REQUIRE(dsv2_aligned16(ysorted) && dsv2_aligned16(out) && dsv2_aligned16(shared_parts) &&
                   (!residual || dsv2_aligned16(residual)) && (!xn_out || dsv2_aligned16(xn_out)),
               DSV2_E_ALIGN, "moe_combine_parts: alignment");
  if (rows == 0) return DSV2_OK;
  hipLaunchKernelGGL(moe_combine_kernel, dim3(rows), dim3(256), 0, (hipStream_t)stream, (const bf16_t*)ysorted,
                     route_pos, weights, nullptr, shared_parts, (const bf16_t*)residual, (bf16_t*)out,
                     (const bf16_t*)next_norm_w, eps, (bf16_t*)xn_out);
  return dsv2_launch_status("moe_combine_parts");
}
