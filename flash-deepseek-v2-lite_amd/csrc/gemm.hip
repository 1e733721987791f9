// Grouped bf16 GEMM on CDNA4 matrix cores (v_mfma_f32_16x16x32_bf16) for the
// weight-streaming shapes of batched decode (tokens M <= 128 per tile, K up to 10944).
//
// A workgroup owns 16 output features (SwiGLU: 16 gate rows and the 16 matching up
// rows) for 16*TB tokens and streams those weight rows from HBM exactly once; its NW
// waves split K into contiguous ranges of 32-wide steps, and their fp32 partial tiles
// are summed through LDS in a fixed wave order (deterministic).  Per step a lane loads
// 16 B of weight row (lane & 15) at k-group (lane >> 4) (A operand) and 16 B of each
// token row (B operand, L2-resident); D layout: lane holds rows 4*kg..4*kg+3 of
// token column (lane & 15).  Grid: x = N / 16 feature tiles, y = token tiles x groups
// (or the MoE tile table).  Groups are experts (MoE), heads (MLA absorption) or one
// dense matrix.
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

template <int TB, bool SWIGLU, int NW, int U>
__global__ __launch_bounds__(NW * 64) void gemm_kernel(const GemmArgs a) {
  constexpr int R = SWIGLU ? 2 : 1;  // weight row blocks per tile (gate, up)
  __shared__ floatx4_t red[NW][R][TB][64];
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
  const int n0 = blockIdx.x * 16;
  const int K = a.K;
  const bf16_t* wrow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) wrow[r] = a.W + g * a.wg + (int64_t)(n0 + r * a.N + li) * K + kg * 8;

  // token rows past the tile read the tile's first row (always valid) and are not stored,
  // so every load below is unconditional (exact vmcnt waits, no masked loads)
  const bf16_t* xrow[TB];
#pragma unroll
  for (int tb = 0; tb < TB; ++tb) {
    const int j = tb * 16 + li < count ? tb * 16 + li : 0;
    const int xr = a.slot_row ? a.slot_row[start + j] / a.slot_div : start + j;
    xrow[tb] = a.X + g * a.xg + (int64_t)xr * a.xs + kg * 8;
  }

  floatx4_t acc[R][TB];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) acc[r][tb] = floatx4_t{0.f, 0.f, 0.f, 0.f};

  // K = nb batches of U 32-wide steps (the host picks U | K/32); wave wv takes the
  // contiguous batches [nb*wv/NW, nb*(wv+1)/NW), all loads of a batch before its MFMAs
  const int nb = (K >> 5) / U;
  const int b0 = (nb * wv) / NW, b1 = (nb * (wv + 1)) / NW;
  for (int bi = b0; bi < b1; ++bi) {
    const int s = bi * U;
    uint4 av[U][R], bv[U][TB];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int r = 0; r < R; ++r) av[u][r] = ldg16(wrow[r] + (s + u) * 32);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) bv[u][tb] = ldg16(xrow[tb] + (s + u) * 32);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) acc[r][tb] = mfma16x16x32(as_bf16x8(av[u][r]), as_bf16x8(bv[u][tb]), acc[r][tb]);
  }

  if (NW > 1) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) red[wv][r][tb][lane] = acc[r][tb];
    __syncthreads();
  }
  // epilogue: wave wv finishes token blocks wv, wv + NW, ... (sum over waves in order 0..NW-1)
  for (int tb = wv; tb < TB; tb += NW) {
    const int slot = start + tb * 16 + li;
    if (tb * 16 + li >= count) continue;
    floatx4_t sum[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      sum[r] = NW > 1 ? red[0][r][tb][lane] : acc[r][tb];
#pragma unroll
      for (int w = 1; w < NW; ++w) sum[r] += red[w][r][tb][lane];
    }
    const int n = n0 + 4 * kg;
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = SWIGLU ? swiglu_bf(sum[0][e], sum[R - 1][e]) : rbf(sum[0][e]);
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

// Token-rows-in-LDS shape (used when the launch has enough tiles): a workgroup owns 64
// weight rows (SwiGLU: 32 features = 32 gate + 32 up rows) of the tile, 8 waves = NRB
// feature blocks x NKQ contiguous k ranges.  Per chunk of CS 32-wide steps the tile's
// token rows are loaded once, with coalesced 16-byte loads, into LDS (double-buffered)
// and every wave takes its MFMA B fragments from there, so token traffic from L2 is one
// pass per 64 weight rows instead of one per 16.  Weight fragments stream straight from
// HBM, the next chunk's requested before the current one is multiplied.  Steps past K
// and token rows past the tile load clamped addresses and are zeroed, so every load is
// unconditional.  The NKQ partial tiles are summed through LDS in a fixed order.
template <int TB, bool SWIGLU, int CS>
__global__ __launch_bounds__(512) void gemm_xlds_kernel(const GemmArgs a) {
  constexpr int R = SWIGLU ? 2 : 1;    // row blocks per wave (gate, up)
  constexpr int NRB = SWIGLU ? 2 : 4;  // feature blocks of 16 per workgroup
  constexpr int NKQ = 8 / NRB;         // k ranges
  constexpr int TOK = 16 * TB;
  constexpr int XROW = CS * 32 + 8;  // LDS row in elements (+16 B pad: conflict-free B reads)
  constexpr int XBUF = NKQ * TOK * XROW;
  constexpr int RED = (NKQ - 1) * NRB * R * TB * 64 * 4;  // floats
  constexpr int LDS_BYTES = (2 * XBUF * 2 > RED * 4) ? 2 * XBUF * 2 : RED * 4;
  constexpr int UNITS = NKQ * TOK * CS * 4;  // 16-byte X units per chunk
  constexpr int UPT = UNITS / 512;
  static_assert(UNITS % 512 == 0, "X units must split evenly over the workgroup");
  __shared__ __attribute__((aligned(16))) uint8_t lds[LDS_BYTES];
  bf16_t* xbuf = reinterpret_cast<bf16_t*>(lds);
  floatx4_t* red = reinterpret_cast<floatx4_t*>(lds);

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int rb = wv % NRB, kq = wv / NRB;
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
    start = (blockIdx.y % a.tiles_per_group) * TOK;
    count = min(TOK, a.rows - start);
  }
  const int K = a.K, S = K >> 5;
  const int SP = ((S + NKQ - 1) / NKQ + CS - 1) / CS * CS;  // steps per k range (CS multiple)
  const int nch = SP / CS;
  const int f0 = blockIdx.x * 16 * NRB + rb * 16;
  const bf16_t* wrow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) wrow[r] = a.W + g * a.wg + (int64_t)(f0 + r * a.N + li) * K + kg * 8;

  // this thread's X units: fixed (range, token, 16-byte part) for every chunk
  const bf16_t* xsrc[UPT];
  int xkq[UPT], xpart[UPT], xdst[UPT];
  bool xok[UPT];
#pragma unroll
  for (int j = 0; j < UPT; ++j) {
    const int u = tid + 512 * j;
    const int uk = u / (TOK * CS * 4), rem = u % (TOK * CS * 4);
    const int tok = rem / (CS * 4), part = rem % (CS * 4);
    const int tk = tok < count ? tok : 0;
    const int row = a.slot_row ? a.slot_row[start + tk] / a.slot_div : start + tk;
    xsrc[j] = a.X + g * a.xg + (int64_t)row * a.xs + (part & 3) * 8;
    xkq[j] = uk;
    xpart[j] = part;
    xok[j] = tok < count;
    xdst[j] = (uk * TOK + tok) * XROW + (part >> 2) * 32 + (part & 3) * 8;
  }
  // chunk c of X (this thread's units) into registers / of this wave's weight fragments
#define XL_LOAD_X(c)                                                             \
  _Pragma("unroll") for (int j = 0; j < UPT; ++j) {                              \
    const int step_ = xkq[j] * SP + (c) * CS + (xpart[j] >> 2);                  \
    const uint4 v_ = ldg16(xsrc[j] + (int64_t)min(step_, S - 1) * 32);           \
    xr[j] = keep_if(xok[j] && step_ < S, v_);                                    \
  }
#define XL_STORE_X(buf) \
  _Pragma("unroll") for (int j = 0; j < UPT; ++j) *reinterpret_cast<uint4*>(xbuf + (buf) * XBUF + xdst[j]) = xr[j];
#define XL_LOAD_A(c, av)                                                         \
  _Pragma("unroll") for (int si = 0; si < CS; ++si) {                            \
    const int step_ = kq * SP + (c) * CS + si;                                   \
    _Pragma("unroll") for (int r = 0; r < R; ++r) {                              \
      const uint4 v_ = ldg16(wrow[r] + (int64_t)min(step_, S - 1) * 32);         \
      av[si][r] = keep_if(step_ < S, v_);                                        \
    }                                                                            \
  }

  floatx4_t acc[R][TB];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) acc[r][tb] = floatx4_t{0.f, 0.f, 0.f, 0.f};

  uint4 a0[CS][R], a1[CS][R], xr[UPT];
  XL_LOAD_A(0, a0)
  XL_LOAD_X(0)
  XL_STORE_X(0)
  __syncthreads();
  for (int c = 0; c < nch; ++c) {
    const bool more = c + 1 < nch;
    if (more) {
      XL_LOAD_A(c + 1, a1)
      XL_LOAD_X(c + 1)
    }
    const bf16_t* xb = xbuf + (c & 1) * XBUF + (kq * TOK + li) * XROW + kg * 8;
#pragma unroll
    for (int si = 0; si < CS; ++si)
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) {
        const bf16x8_t bfr = *reinterpret_cast<const bf16x8_t*>(xb + tb * 16 * XROW + si * 32);
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r][tb] = mfma16x16x32(as_bf16x8(a0[si][r]), bfr, acc[r][tb]);
      }
    if (more) {
      XL_STORE_X((c + 1) & 1)
    }
    __syncthreads();
#pragma unroll
    for (int si = 0; si < CS; ++si)
#pragma unroll
      for (int r = 0; r < R; ++r) a0[si][r] = a1[si][r];
  }

#undef XL_LOAD_X
#undef XL_STORE_X
#undef XL_LOAD_A
  // sum the k ranges in order 0, 1, ..., NKQ-1 (the X buffers are free after the last barrier)
  if (kq > 0) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) red[((((kq - 1) * NRB + rb) * R + r) * TB + tb) * 64 + lane] = acc[r][tb];
  }
  __syncthreads();
  if (kq != 0) return;
#pragma unroll
  for (int q = 1; q < NKQ; ++q)
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) acc[r][tb] += red[((((q - 1) * NRB + rb) * R + r) * TB + tb) * 64 + lane];
#pragma unroll
  for (int tb = 0; tb < TB; ++tb) {
    if (tb * 16 + li >= count) continue;
    const int slot = start + tb * 16 + li;
    const int n = f0 + 4 * kg;
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = SWIGLU ? swiglu_bf(acc[0][tb][e], acc[R - 1][tb][e]) : rbf(acc[0][tb][e]);
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

// features per workgroup of gemm_xlds_kernel
static int xlds_features(bool swiglu) { return swiglu ? 32 : 64; }

static int launch_gemm_xlds(const GemmArgs& a, int tb, bool swiglu, int grid_y, hipStream_t st) {
  const dim3 grid(a.N / xlds_features(swiglu), grid_y);
#define DSV2_XL(TBV, SWV, CSV) hipLaunchKernelGGL((gemm_xlds_kernel<TBV, SWV, CSV>), grid, dim3(512), 0, st, a)
  if (swiglu) {
    if (tb == 1) DSV2_XL(1, true, 4);
    else if (tb == 2) DSV2_XL(2, true, 4);
    else DSV2_XL(4, true, 2);
  } else {
    if (tb == 1) DSV2_XL(1, false, 8);
    else if (tb == 2) DSV2_XL(2, false, 8);
    else if (tb == 4) DSV2_XL(4, false, 4);
    else DSV2_XL(8, false, 2);
  }
#undef DSV2_XL
  return dsv2_launch_status("gemm");
}

// Launch shape by token blocks: NW waves split K in batches of U steps (U = 4 when it
// divides K/32, else 2).  The fp32 reduction buffer is NW*R*TB KB of LDS (<= 64 KB).
// Token tiles are at most 128 (TB = 8): larger row counts run as several tiles (their
// weights then come from L2 / Infinity Cache after the first).
static int launch_gemm(const GemmArgs& a, int tb, bool swiglu, int grid_y, hipStream_t st) {
  if ((a.tiles || (a.N % xlds_features(swiglu) == 0 && (int64_t)(a.N / xlds_features(swiglu)) * grid_y >= 512)) &&
      !(swiglu && tb == 8))
    return launch_gemm_xlds(a, tb, swiglu, grid_y, st);
  const dim3 grid(a.N / 16, grid_y);
  const bool u4 = ((a.K >> 5) % 4) == 0;
#define DSV2_GEMM(TBV, SWV, NWV)                                                                  \
  if (u4)                                                                                         \
    hipLaunchKernelGGL((gemm_kernel<TBV, SWV, NWV, 4>), grid, dim3(NWV * 64), 0, st, a);          \
  else                                                                                            \
    hipLaunchKernelGGL((gemm_kernel<TBV, SWV, NWV, 2>), grid, dim3(NWV * 64), 0, st, a);
  if (tb == 1) {
    if (swiglu) { DSV2_GEMM(1, true, 8) } else { DSV2_GEMM(1, false, 8) }
  } else if (tb == 2) {
    if (swiglu) { DSV2_GEMM(2, true, 8) } else { DSV2_GEMM(2, false, 8) }
  } else if (tb == 4) {
    if (swiglu) { DSV2_GEMM(4, true, 8) } else { DSV2_GEMM(4, false, 8) }
  } else {
    if (swiglu) { DSV2_GEMM(8, true, 4) } else { DSV2_GEMM(8, false, 8) }
  }
#undef DSV2_GEMM
  return dsv2_launch_status("gemm");
}

static int pick_tb(int rows) { return rows <= 16 ? 1 : (rows <= 32 ? 2 : (rows <= 64 ? 4 : 8)); }

extern "C" int dsv2_gemm_bf16(const void* x, int64_t x_stride, int64_t x_gstride, int rows, int K, const void* W,
                              int64_t w_gstride, int N, int n_groups, const void* residual, int64_t res_stride,
                              void* y, int64_t y_stride, int64_t y_gstride, int flags, void* stream) {
  DSV2_REQUIRE(x && W && y, DSV2_E_NULL, "gemm: null pointer");
  DSV2_REQUIRE(rows >= 0 && K > 0 && K % 64 == 0 && N > 0 && N % 16 == 0 && n_groups >= 1, DSV2_E_SHAPE,
               "gemm: bad shape rows=%d K=%d N=%d groups=%d (K%%64, N%%16 required)", rows, K, N, n_groups);
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
  DSV2_REQUIRE(max_tiles >= 0 && max_tiles <= 65535 && inter > 0 && inter % 16 == 0 &&
                   (tile_tokens == 16 || tile_tokens == 32 || tile_tokens == 64),
               DSV2_E_SHAPE, "moe_grouped_gateup: bad shape (inter %% 16, tile_tokens in {16,32,64})");
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
  DSV2_REQUIRE(max_tiles >= 0 && max_tiles <= 65535 && inter > 0 && inter % 64 == 0 &&
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
