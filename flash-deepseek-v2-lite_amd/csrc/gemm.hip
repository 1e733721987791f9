// Grouped bf16 GEMM on CDNA4 matrix cores (v_mfma_f32_16x16x32_bf16).
//
// Output tile of a wave: 16 weight rows (MFMA M) x 16*TB tokens (MFMA N), fp32
// accumulators, K stepped by 32.  A operand = weight rows straight from HBM
// (16 B per lane per step: row li = lane&15, k-group kg = lane>>4), B operand =
// token rows (same k mapping; L2-resident).  A workgroup = 4 waves = 64 weight
// rows, so every weight byte of a (group, row-block) is fetched once per token
// tile.  Groups are experts (MoE), heads (MLA absorption) or a single dense
// matrix.  D layout: lane holds rows 4*kg..4*kg+3 of column li.
#include "common.h"

struct GemmArgs {
  const bf16_t* X;
  int64_t xs, xg;
  const int32_t* slot_row;  // MoE gate_up: token row of slot p = slot_row[p] / slot_div
  int slot_div;
  const int32_t* tiles;  // explicit {group, start, count, _} table (MoE) or null (implicit)
  const int32_t* ntiles;
  int rows, tiles_per_group;
  const bf16_t* W;
  int64_t wg;
  int N, K;
  const bf16_t* res;
  int64_t rs;
  void* Y;
  int64_t ys, yg;
  bool out_f32;
};

template <int TB, bool SWIGLU>
__global__ __launch_bounds__(256) void gemm_kernel(const GemmArgs a) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int li = lane & 15, kg = lane >> 4;
  int g, start, count;
  if (a.tiles) {
    if ((int)blockIdx.y >= a.ntiles[0]) return;
    const int4 t = reinterpret_cast<const int4*>(a.tiles)[blockIdx.y];
    g = t.x;
    start = t.y;
    count = t.z;
  } else {
    g = blockIdx.y / a.tiles_per_group;
    start = (blockIdx.y % a.tiles_per_group) * 16 * TB;
    count = min(16 * TB, a.rows - start);
  }
  const int n0 = blockIdx.x * 64 + wv * 16;
  const int K = a.K;
  const bf16_t* wrow = a.W + g * a.wg + (int64_t)(n0 + li) * K + kg * 8;
  const bf16_t* wrow_u = wrow + (int64_t)a.N * K;

  const bf16_t* xrow[TB];
  bool valid[TB];
#pragma unroll
  for (int tb = 0; tb < TB; ++tb) {
    const int j = tb * 16 + li;
    valid[tb] = j < count;
    int xr = 0;
    if (valid[tb]) xr = a.slot_row ? a.slot_row[start + j] / a.slot_div : start + j;
    xrow[tb] = a.X + g * a.xg + (int64_t)xr * a.xs + kg * 8;
  }

  floatx4_t acc[TB], accu[TB];
#pragma unroll
  for (int tb = 0; tb < TB; ++tb) acc[tb] = accu[tb] = floatx4_t{0.f, 0.f, 0.f, 0.f};

  const uint4 zero = {0u, 0u, 0u, 0u};
  constexpr int U = 4;
  int k0 = 0;
  for (; k0 + 32 * U <= K; k0 += 32 * U) {
    uint4 av[U], au[U], bv[U][TB];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      av[u] = ldg16(wrow + k0 + u * 32);
      if (SWIGLU) au[u] = ldg16(wrow_u + k0 + u * 32);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) bv[u][tb] = valid[tb] ? ldg16(xrow[tb] + k0 + u * 32) : zero;
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) {
        acc[tb] = mfma16x16x32(as_bf16x8(av[u]), as_bf16x8(bv[u][tb]), acc[tb]);
        if (SWIGLU) accu[tb] = mfma16x16x32(as_bf16x8(au[u]), as_bf16x8(bv[u][tb]), accu[tb]);
      }
  }
  for (; k0 < K; k0 += 32) {
    const uint4 av = ldg16(wrow + k0);
    uint4 au = zero;
    if (SWIGLU) au = ldg16(wrow_u + k0);
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      const uint4 bv = valid[tb] ? ldg16(xrow[tb] + k0) : zero;
      acc[tb] = mfma16x16x32(as_bf16x8(av), as_bf16x8(bv), acc[tb]);
      if (SWIGLU) accu[tb] = mfma16x16x32(as_bf16x8(au), as_bf16x8(bv), accu[tb]);
    }
  }

#pragma unroll
  for (int tb = 0; tb < TB; ++tb) {
    if (!valid[tb]) continue;
    const int slot = start + tb * 16 + li;
    const int n = n0 + 4 * kg;
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = SWIGLU ? swiglu_bf(acc[tb][e], accu[tb][e]) : rbf(acc[tb][e]);
    if (a.res) {
      const uint2 r2 = *reinterpret_cast<const uint2*>(a.res + slot * a.rs + n);
      v[0] = rbf(__uint_as_float(r2.x << 16) + v[0]);
      v[1] = rbf(__uint_as_float(r2.x & 0xffff0000u) + v[1]);
      v[2] = rbf(__uint_as_float(r2.y << 16) + v[2]);
      v[3] = rbf(__uint_as_float(r2.y & 0xffff0000u) + v[3]);
    }
    const int64_t off = g * a.yg + (int64_t)slot * a.ys + n;
    if (a.out_f32) {
      *reinterpret_cast<float4*>(reinterpret_cast<float*>(a.Y) + off) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
      uint2 o;
      o.x = pack2(v[0], v[1]);
      o.y = pack2(v[2], v[3]);
      *reinterpret_cast<uint2*>(reinterpret_cast<bf16_t*>(a.Y) + off) = o;
    }
  }
}

static int launch_gemm(const GemmArgs& a, int tb, bool swiglu, int grid_y, hipStream_t st) {
  const dim3 grid(a.N / 64, grid_y);
#define DSV2_GEMM(TBV)                                                        \
  if (swiglu)                                                                 \
    hipLaunchKernelGGL((gemm_kernel<TBV, true>), grid, dim3(256), 0, st, a);  \
  else                                                                        \
    hipLaunchKernelGGL((gemm_kernel<TBV, false>), grid, dim3(256), 0, st, a);
  if (tb == 1) {
    DSV2_GEMM(1)
  } else if (tb == 2) {
    DSV2_GEMM(2)
  } else {
    DSV2_GEMM(4)
  }
#undef DSV2_GEMM
  return dsv2_launch_status("gemm");
}

static int pick_tb(int rows) { return rows <= 16 ? 1 : (rows <= 32 ? 2 : 4); }

extern "C" int dsv2_gemm_bf16(const void* x, int64_t x_stride, int64_t x_gstride, int rows, int K, const void* W,
                              int64_t w_gstride, int N, int n_groups, const void* residual, int64_t res_stride,
                              void* y, int64_t y_stride, int64_t y_gstride, int flags, void* stream) {
  DSV2_REQUIRE(x && W && y, DSV2_E_NULL, "gemm: null pointer");
  DSV2_REQUIRE(rows >= 0 && K > 0 && K % 32 == 0 && N > 0 && N % 64 == 0 && n_groups >= 1, DSV2_E_SHAPE,
               "gemm: bad shape rows=%d K=%d N=%d groups=%d (K%%32, N%%64 required)", rows, K, N, n_groups);
  DSV2_REQUIRE((flags & ~(DSV2_LINEAR_SWIGLU | DSV2_LINEAR_OUT_F32)) == 0, DSV2_E_FLAGS, "gemm: unknown flags");
  DSV2_REQUIRE(!(residual && ((flags & DSV2_LINEAR_SWIGLU) || n_groups != 1)), DSV2_E_FLAGS,
               "gemm: residual needs a plain single-group GEMM");
  DSV2_REQUIRE(dsv2_aligned16(x) && dsv2_aligned16(W) && x_stride % 8 == 0 && x_gstride % 8 == 0 &&
                   w_gstride % 8 == 0 && y_stride % 4 == 0 && y_gstride % 4 == 0 &&
                   (!residual || res_stride % 4 == 0),
               DSV2_E_ALIGN, "gemm: 16-byte aligned x/W and 8-byte aligned rows of y required");
  if (rows == 0) return DSV2_OK;
  const int tb = pick_tb(rows);
  GemmArgs a{};
  a.X = (const bf16_t*)x;
  a.xs = x_stride;
  a.xg = x_gstride;
  a.slot_row = nullptr;
  a.slot_div = 1;
  a.tiles = nullptr;
  a.ntiles = nullptr;
  a.rows = rows;
  a.tiles_per_group = (rows + 16 * tb - 1) / (16 * tb);
  a.W = (const bf16_t*)W;
  a.wg = w_gstride;
  a.N = N;
  a.K = K;
  a.res = (const bf16_t*)residual;
  a.rs = res_stride;
  a.Y = y;
  a.ys = y_stride;
  a.yg = y_gstride;
  a.out_f32 = flags & DSV2_LINEAR_OUT_F32;
  const int64_t grid_y = (int64_t)a.tiles_per_group * n_groups;
  DSV2_REQUIRE(grid_y <= 65535, DSV2_E_SHAPE, "gemm: too many row tiles (%lld)", (long long)grid_y);
  return launch_gemm(a, tb, flags & DSV2_LINEAR_SWIGLU, (int)grid_y, (hipStream_t)stream);
}

static int tile_tb(int tile_tokens) { return tile_tokens == 16 ? 1 : (tile_tokens == 32 ? 2 : 4); }

extern "C" int dsv2_moe_grouped_gateup(const void* xn, const int32_t* sorted_routes, const int32_t* tiles,
                                       const int32_t* num_tiles, int max_tiles, int tile_tokens, const void* w_gate_up,
                                       int inter, void* hsorted, void* stream) {
  DSV2_REQUIRE(xn && sorted_routes && tiles && num_tiles && w_gate_up && hsorted, DSV2_E_NULL,
               "moe_grouped_gateup: null pointer");
  DSV2_REQUIRE(max_tiles >= 0 && max_tiles <= 65535 && inter > 0 && inter % 64 == 0 &&
                   (tile_tokens == 16 || tile_tokens == 32 || tile_tokens == 64),
               DSV2_E_SHAPE, "moe_grouped_gateup: bad shape (inter %% 64, tile_tokens in {16,32,64})");
  DSV2_REQUIRE(dsv2_aligned16(xn) && dsv2_aligned16(w_gate_up) && dsv2_aligned16(tiles), DSV2_E_ALIGN,
               "moe_grouped_gateup: alignment");
  if (max_tiles == 0) return DSV2_OK;
  GemmArgs a{};
  a.X = (const bf16_t*)xn;
  a.xs = 2048;
  a.xg = 0;
  a.slot_row = sorted_routes;
  a.slot_div = 6;
  a.tiles = tiles;
  a.ntiles = num_tiles;
  a.W = (const bf16_t*)w_gate_up;
  a.wg = (int64_t)2 * inter * 2048;
  a.N = inter;
  a.K = 2048;
  a.Y = hsorted;
  a.ys = inter;
  a.yg = 0;
  return launch_gemm(a, tile_tb(tile_tokens), true, max_tiles, (hipStream_t)stream);
}

extern "C" int dsv2_moe_grouped_down(const void* hsorted, const int32_t* tiles, const int32_t* num_tiles,
                                     int max_tiles, int tile_tokens, const void* w_down, int inter, void* ysorted,
                                     void* stream) {
  DSV2_REQUIRE(hsorted && tiles && num_tiles && w_down && ysorted, DSV2_E_NULL, "moe_grouped_down: null pointer");
  DSV2_REQUIRE(max_tiles >= 0 && max_tiles <= 65535 && inter > 0 && inter % 32 == 0 &&
                   (tile_tokens == 16 || tile_tokens == 32 || tile_tokens == 64),
               DSV2_E_SHAPE, "moe_grouped_down: bad shape");
  DSV2_REQUIRE(dsv2_aligned16(hsorted) && dsv2_aligned16(w_down) && dsv2_aligned16(tiles) && inter % 8 == 0,
               DSV2_E_ALIGN, "moe_grouped_down: alignment");
  if (max_tiles == 0) return DSV2_OK;
  GemmArgs a{};
  a.X = (const bf16_t*)hsorted;
  a.xs = inter;
  a.xg = 0;
  a.slot_row = nullptr;
  a.slot_div = 1;
  a.tiles = tiles;
  a.ntiles = num_tiles;
  a.W = (const bf16_t*)w_down;
  a.wg = (int64_t)2048 * inter;
  a.N = 2048;
  a.K = inter;
  a.Y = ysorted;
  a.ys = 2048;
  a.yg = 0;
  return launch_gemm(a, tile_tb(tile_tokens), false, max_tiles, (hipStream_t)stream);
}
