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
#include "mla_rows.h"

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
  bool exact_f32;  // out_f32 without the bf16 round of the accumulator (router logits)
  // grouped launches: the shared-expert halves (a token tile of the launch's size per chunk
  // of `rows` and half, ahead of the table's tiles): half h reads token t at
  // X2 + h*x2g + t*x2s, its (gate) weight rows at W2 + h*w2g with row stride w2ld (SwiGLU:
  // up row = gate row + w2up), and writes Y2[h * y2g + t * y2s + n] (SwiGLU: bf16; plain:
  // the fp32 partial sum; no residual)
  const bf16_t* X2;
  int64_t x2s, x2g;
  const bf16_t* W2;
  int64_t w2g;
  int w2ld, w2up, s_tiles;
  void* Y2;
  int64_t y2s, y2g;
  // e4m3 weights (gemm_f8_kernel: W / W2 then hold e4m3 bytes): fp32 power-of-two scale of
  // weight row R of group g at S[g * sg + R] (shared half h: S2[h * s2g + R])
  const float* S;
  int64_t sg;
  const float* S2;
  int64_t s2g;
};

// A plain (non-SwiGLU) output before its residual add / store: the bf16 round of the fp32
// accumulator, or the accumulator itself for an exact fp32 output.
__device__ __forceinline__ float acc_out(const GemmArgs& a, float acc) { return a.exact_f32 ? acc : rbf(acc); }

// The residual of outputs (slot, n .. n+3), requested by a kernel before its weight stream: a
// load issued in the epilogue is one more dependent round trip at the end of every workgroup.
// Without a residual (or where `use` is false) it reads X's first 8 bytes, which are unused.
__device__ __forceinline__ uint2 gemm_res_load(const GemmArgs& a, bool use, int slot, int n) {
  return *reinterpret_cast<const uint2*>(use && a.res ? a.res + (int64_t)slot * a.rs + n : a.X);
}

// Four consecutive outputs (features n..n+3) of token slot `slot`: the residual r2 (loaded by
// gemm_res_load) added when the GEMM has one, then a bf16 or fp32 store.
__device__ __forceinline__ void gemm_store4r(const GemmArgs& a, int g, int slot, int n, float* v, uint2 r2) {
  if (a.res) {
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
    for (int e = 0; e < 4; ++e) v[e] = SWIGLU ? swiglu_bf(sum[0][e], sum[R - 1][e]) : acc_out(a, sum[0][e]);
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
//
// AST (CS == 4): weights are read in a row-contiguous pattern -- each load covers 4 rows x
// 256 B, four loads a wave's 16 rows x 128 k -- which streams ~35% faster from HBM on
// MI355X than the MFMA fragment order (16 rows x 64 B per load); the wave then passes
// them through its own 4 KB LDS tile to form the A fragments.
template <int TB, bool SWIGLU, int CS, bool AST, int DEPTH, int NRB, int XD = 1, bool NTA = false>
__global__ __launch_bounds__(512) void gemm_xlds_kernel(const GemmArgs a) {
  static_assert(!AST || CS == 4, "row-contiguous weight staging works on 128-k chunks");
  static_assert(XD >= 1 && DEPTH % XD == 0, "token-chunk stages must divide the unroll");
  constexpr int R = SWIGLU ? 2 : 1;    // row blocks per wave (gate, up)
  static_assert(NRB == 2 || NRB == 4, "feature blocks of 16 per workgroup");
  constexpr int NKQ = 8 / NRB;         // k ranges
  constexpr int TOK = 16 * TB;
  constexpr int XROW = CS * 32 + 8;  // LDS row in elements (+16 B pad: conflict-free B reads)
  constexpr int XBUF = NKQ * TOK * XROW;
  constexpr int RED = (NKQ - 1) * NRB * R * TB * 64 * 4;  // floats
  constexpr int AROW = 136;                             // A tile row (128 k + 8 pad), elements
  constexpr int ATILE = AST ? 8 * 16 * AROW : 0;         // elements (all waves)
  constexpr int MAIN = 2 * XBUF * 2 + ATILE * 2;
  constexpr int LDS_BYTES = (MAIN > RED * 4) ? MAIN : RED * 4;
  constexpr int UNITS = NKQ * TOK * CS * 4;  // 16-byte X units per chunk
  constexpr int UPT = UNITS / 512;
  static_assert(UNITS % 512 == 0, "X units must split evenly over the workgroup");
  __shared__ __attribute__((aligned(16))) uint8_t lds[LDS_BYTES];
  bf16_t* xbuf = reinterpret_cast<bf16_t*>(lds);
  floatx4_t* red = reinterpret_cast<floatx4_t*>(lds);
  bf16_t* atile = reinterpret_cast<bf16_t*>(lds) + 2 * XBUF + (threadIdx.x >> 6) * 16 * AROW;

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int rb = wv % NRB, kq = wv / NRB;
  const int li = lane & 15, kg = lane >> 4;
  int g, start, count;
  bool shared = false;  // a tile of one of the shared-expert halves (a.W2), grid rows 0 .. ns-1
  if (a.tiles) {
    const int ns = a.W2 ? 2 * a.s_tiles : 0;
    if ((int)blockIdx.y < ns) {
      shared = true;
      g = blockIdx.y / a.s_tiles;
      start = (blockIdx.y % a.s_tiles) * TOK;
      count = min(TOK, a.rows - start);
    } else {
      if ((int)blockIdx.y - ns >= a.ntiles[0]) return;
      const int4 t = reinterpret_cast<const int4*>(a.tiles)[blockIdx.y - ns];
      g = t.x;
      start = t.y;
      count = t.z;
    }
  } else {
    g = blockIdx.y / a.tiles_per_group;
    start = (blockIdx.y % a.tiles_per_group) * TOK;
    count = min(TOK, a.rows - start);
  }
  const int K = a.K, S = K >> 5;
  // steps per k range: a multiple of CS * DEPTH (steps past K are zero in the X tile)
  const int SP = ((S + NKQ - 1) / NKQ + CS * DEPTH - 1) / (CS * DEPTH) * (CS * DEPTH);
  const int nch = SP / CS;
  const int f0 = blockIdx.x * 16 * NRB + rb * 16;
  const bf16_t* const wbase = shared ? a.W2 + g * a.w2g : a.W + g * a.wg;
  const int64_t wld = shared ? a.w2ld : K;  // weight row stride
  const int upoff = shared ? a.w2up : a.N;  // SwiGLU: gate row -> up row
  const bf16_t* wrow[R];
#pragma unroll
  for (int r = 0; r < R; ++r)
    wrow[r] = AST ? wbase + (f0 + r * upoff + (lane >> 4)) * wld + (lane & 3) * 8
                  : wbase + (f0 + r * upoff + li) * wld + kg * 8;

  // this thread's X units: fixed (range, token, 16-byte part) for every chunk
  const bf16_t* xsrc[UPT];
  int xkq[UPT], xpart[UPT], xdst[UPT];
#pragma unroll
  for (int j = 0; j < UPT; ++j) {
    const int u = tid + 512 * j;
    const int uk = u / (TOK * CS * 4), rem = u % (TOK * CS * 4);
    const int tok = rem / (CS * 4), part = rem % (CS * 4);
    const int tk = tok < count ? tok : 0;
    if (shared) {
      xsrc[j] = a.X2 + g * a.x2g + (int64_t)(start + tk) * a.x2s + (part & 3) * 8;
    } else {
      const int row = a.slot_row ? a.slot_row[start + tk] / a.slot_div : start + tk;
      xsrc[j] = a.X + g * a.xg + (int64_t)row * a.xs + (part & 3) * 8;
    }
    xkq[j] = uk;
    xpart[j] = part;
    xdst[j] = (uk * TOK + tok) * XROW + (part >> 2) * 32 + (part & 3) * 8;
  }
  // chunk c of X (this thread's units) into registers / into LDS buffer buf.  Loaded values
  // are only masked when they are stored, so no load is waited for before its data is
  // needed.  Steps past K read step S-1 and are zeroed in the X tile only: the weight
  // fragments there are real (finite) weights multiplied by zero.  Token rows past the
  // tile hold row 0's values; their output columns are never stored.
#define XL_LOAD_X(c, xs)                                                         \
  _Pragma("unroll") for (int j = 0; j < UPT; ++j) {                              \
    const int step_ = xkq[j] * SP + (c) * CS + (xpart[j] >> 2);                  \
    xs[j] = ldg16(xsrc[j] + (int64_t)min(step_, S - 1) * 32);                    \
  }
#define XL_STORE_X(c, xs, buf)                                                   \
  _Pragma("unroll") for (int j = 0; j < UPT; ++j) {                              \
    const int step_ = xkq[j] * SP + (c) * CS + (xpart[j] >> 2);                  \
    *reinterpret_cast<uint4*>(xbuf + (buf) * XBUF + xdst[j]) = keep_if(step_ < S, xs[j]); \
  }
// AST: av[q][r] = rows 4q + (lane >> 4) of block r, k = chunk + (lane & 15) * 8
#define XL_LOAD_A(c, av)                                                                         \
  _Pragma("unroll") for (int si = 0; si < CS; ++si) {                                            \
    const int step_ = kq * SP + (c) * CS + (AST ? ((lane & 15) >> 2) : si);                      \
    _Pragma("unroll") for (int r = 0; r < R; ++r)                                                \
      av[si][r] = NTA ? ldg16_nt(wrow[r] + (AST ? si * 4 * wld : 0) + (int64_t)min(step_, S - 1) * 32) \
                      : ldg16(wrow[r] + (AST ? si * 4 * wld : 0) + (int64_t)min(step_, S - 1) * 32); \
  }

  floatx4_t acc[R][TB];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) acc[r][tb] = floatx4_t{0.f, 0.f, 0.f, 0.f};

  // Weight chunks are requested DEPTH - 1 chunks ahead of the one being multiplied, token
  // chunks XD ahead (a ring of XD register stages; chunk c + 1 goes to LDS at the end of
  // chunk c) and before the weight loads (loads complete in issue order, so the wait for a
  // token chunk before its LDS store leaves the later weight loads in flight).  The chunk
  // loop is unrolled by DEPTH (nch is a multiple of it) so every register buffer index is a
  // constant, and no load sits behind a branch: requests past the last chunk repeat it (L2
  // hits), so the compiler's wait counts stay exact.
  // the epilogue's residuals (k range 0's waves, token blocks tb) first: the wait for token
  // chunk 0 before its LDS store then covers them
  uint2 rpre[TB];
#pragma unroll
  for (int tb = 0; tb < TB; ++tb)
    rpre[tb] = gemm_res_load(a, kq == 0 && !shared && tb * 16 + li < count, start + tb * 16 + li, f0 + 4 * kg);
  uint4 ab[DEPTH][CS][R], xr[XD][UPT];
#pragma unroll
  for (int x = 0; x < XD; ++x) XL_LOAD_X(min(x, nch - 1), xr[x])
#pragma unroll
  for (int p = 0; p + 1 < DEPTH; ++p) XL_LOAD_A(min(p, nch - 1), ab[p])
  XL_STORE_X(0, xr[0], 0)
#pragma unroll
  for (int tb = 0; tb < TB; ++tb) {
    pin(rpre[tb].x);
    pin(rpre[tb].y);
  }
  __syncthreads();
  for (int c0 = 0; c0 < nch; c0 += DEPTH) {
#pragma unroll
    for (int i = 0; i < DEPTH; ++i) {
      const int c = c0 + i;
      XL_LOAD_X(min(c + XD, nch - 1), xr[i % XD])  // stage i % XD held chunk c, now in LDS
      XL_LOAD_A(min(c + DEPTH - 1, nch - 1), ab[(i + DEPTH - 1) % DEPTH])
      const bf16_t* xb = xbuf + (c & 1) * XBUF + (kq * TOK + li) * XROW + kg * 8;
      bf16x8_t afr[CS][R];
      if (AST) {
        // each row block's 16 rows x 128 k through the wave's LDS tile into MFMA fragments
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
          for (int q = 0; q < CS; ++q)
            *reinterpret_cast<uint4*>(atile + (4 * q + (lane >> 4)) * AROW + (lane & 15) * 8) = ab[i][q][r];
          __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
          for (int si = 0; si < CS; ++si)
            afr[si][r] = *reinterpret_cast<const bf16x8_t*>(atile + li * AROW + si * 32 + kg * 8);
          __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        }
      } else {
#pragma unroll
        for (int si = 0; si < CS; ++si)
#pragma unroll
          for (int r = 0; r < R; ++r) afr[si][r] = as_bf16x8(ab[i][si][r]);
      }
#pragma unroll
      for (int si = 0; si < CS; ++si)
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) {
          const bf16x8_t bfr = *reinterpret_cast<const bf16x8_t*>(xb + tb * 16 * XROW + si * 32);
#pragma unroll
          for (int r = 0; r < R; ++r) acc[r][tb] = mfma16x16x32(afr[si][r], bfr, acc[r][tb]);
        }
      // the last chunk's store fills the idle buffer with a repeat (never read)
      XL_STORE_X(c + 1, xr[(i + 1) % XD], (c + 1) & 1)
      __syncthreads();
    }
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
    for (int e = 0; e < 4; ++e) v[e] = SWIGLU ? swiglu_bf(acc[0][tb][e], acc[R - 1][tb][e]) : acc_out(a, acc[0][tb][e]);
    if (shared) {  // SwiGLU: bf16 row of the half's output; plain: the fp32 partial sum
      if (SWIGLU) {
        uint2 o;
        o.x = pack2(v[0], v[1]);
        o.y = pack2(v[2], v[3]);
        *reinterpret_cast<uint2*>(reinterpret_cast<bf16_t*>(a.Y2) + g * a.y2g + (int64_t)slot * a.y2s + n) = o;
      } else {
        *reinterpret_cast<float4*>(reinterpret_cast<float*>(a.Y2) + g * a.y2g + (int64_t)slot * a.y2s + n) =
            make_float4(acc[0][tb][0], acc[0][tb][1], acc[0][tb][2], acc[0][tb][3]);
      }
      continue;
    }
    gemm_store4r(a, g, slot, n, v, rpre[tb]);
  }
}

// gemm_store4r with the residual loaded at the store
__device__ __forceinline__ void gemm_store4(const GemmArgs& a, int g, int slot, int n, float* v) {
  gemm_store4r(a, g, slot, n, v, a.res ? *reinterpret_cast<const uint2*>(a.res + (int64_t)slot * a.rs + n) : uint2{0u, 0u});
}

// Direct-to-LDS ring shape for dense weights at 128+ tokens (the lm_head from 33) and for the
// expert-grouped MoE's 64-token tiles: a 4-wave workgroup owns 64
// features x 64 tokens (each wave 32 x 32, 2 x 2 MFMA blocks).  K streams in 64-wide chunks
// through a ring of kDmaStages 16 KB LDS stages filled by global_load_lds (16 bytes per
// lane straight into LDS, no register round trip): every load covers 8 rows x 128 B, and
// the lanes pick the 16-byte pieces so that the LDS copy is swizzled (piece c of row r at
// slot c ^ (r & 7)) and the MFMA fragment reads are conflict-free.  One barrier per chunk;
// the wait before it counts only this wave's newer ring loads (the workgroup fence of
// __syncthreads would drain the whole ring).  XCD-aware 1-D grid: the token tiles of one
// feature block are consecutive work items on one XCD, so their weight reads after the
// first hit that XCD's L2 (qkv_a at 256 tokens: 12.2 us vs 17.9 us for the token-rows-in-LDS
// shape; without the XCD grouping 18.3 us).
constexpr int kDmaStages = 4;
constexpr int kDmaGroupedWgs = 512;  // 256 CUs x 2 (64 KB of LDS each)

// xcd_blocked (the prefill shape): the work items, token-tile-major (all feature blocks of a
// token tile, then the next tile, an expert's tiles in a row), are cut into 8 contiguous
// ranges, one per XCD (workgroup i runs on XCD i % 8), and every item reads its K chunks in
// order.  The ~32 items an XCD runs at once then share each token chunk among the tile's
// feature blocks and each weight chunk among the expert's tiles in that XCD's L2; the decode
// order instead puts all token tiles of a feature block on one XCD, which at prefill sizes
// (token rows 3x the weight bytes) re-reads every token row from HBM on every XCD
// (8192 x 2048 x 2048: 80.4 -> 74.2 us; C3 prefill 4.27 -> 4.15 s).
struct DmaShape {
  int tiles, nwg, nfb;
  int xcd_blocked;
};


// SWIGLU: the 64 weight rows of a workgroup are, per 16 features, 16 gate rows then the 16
// matching up rows (32 features per workgroup); a wave's two row blocks are then one
// feature block's gate and up tiles, combined in its epilogue.
// Grouped (a.tiles, 64-token expert tiles): a grid of kDmaGroupedWgs workgroups loops over
// the live (tile, feature block) items only, so the table's dead tiles cost no workgroup
// launches; token rows are gathered through slot_row and the tile's expert selects the
// weights.
template <bool SWIGLU, int WM = 32, int WN = 32, int ST = kDmaStages, int RWV = 2>
__global__ __launch_bounds__(RWV * 128) void gemm_dma_kernel(const GemmArgs a, const DmaShape sh) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];  // ST stages of SB bytes
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, li = lane & 15, kg = lane >> 4;
  constexpr int NW = 2 * RWV;                // waves: RWV along the weight rows x 2 along the tokens
  constexpr int TM = RWV * WM, TN = 2 * WN;  // weight rows, tokens per workgroup
  constexpr int KC = 64, RB = 2 * KC;        // K per chunk; a chunk's bytes per row (8 pieces of 16 B)
  constexpr int RPL = 8;                     // rows per ring load (64 lanes x 16 B)
  constexpr int SB = (TM + TN) * RB;         // stage: TM weight rows, then TN token rows
  constexpr int LW = TM / (RPL * NW), LL = (TM + TN) / (RPL * NW);  // ring loads per wave per chunk: weights, all
  constexpr int XM = WM / 16, XN = WN / 16;  // MFMA blocks per wave
  constexpr int FPW = SWIGLU ? TM / 2 : TM;  // output features per workgroup
  static_assert(LL <= 8 && XM <= 4 && XN <= 8, "local arrays have literal sizes");
  // piece p of row r sits in slot p ^ (r & 7): the 16 rows one MFMA fragment reads hit
  // distinct banks in every group of 8 lanes
  auto swz = [](int r) { return r & 7; };
  // grouped: items j = tile * nfb + fb over the live tiles (the shared halves' tiles, then the
  // table's), consecutive items round-robin over the XCDs (keeping all token tiles of a
  // feature block on one XCD measured slower: fewer feature blocks than XCD slots balance)
  const int ns = a.W2 ? 2 * a.s_tiles : 0;
  const int live = a.tiles ? ns + min(a.ntiles[0], sh.tiles) : 0;  // sh.tiles: the table's size
  for (int it = 0;; ++it) {
    int fb, g = 0, t0, count;
    bool shared = false;
    if (a.tiles) {
      int j;
      if (sh.xcd_blocked) {  // XCD blockIdx % 8 runs items [x * per, (x + 1) * per)
        const int per = (live * sh.nfb + 7) / 8, jl = blockIdx.x / 8 + it * (gridDim.x / 8);
        if (jl >= per) break;
        j = (blockIdx.x % 8) * per + jl;
      } else {
        j = blockIdx.x + it * gridDim.x;
      }
      if (j >= live * sh.nfb) break;
      const int tile = j / sh.nfb;
      fb = j % sh.nfb;
      if (tile < ns) {  // a shared-expert half's tile of tokens
        shared = true;
        g = tile / a.s_tiles;
        t0 = (tile % a.s_tiles) * TN;
        count = min(TN, a.rows - t0);
      } else {
        const int4 tt = reinterpret_cast<const int4*>(a.tiles)[tile - ns];
        g = tt.x;
        t0 = tt.y;
        count = tt.z;
      }
    } else {
      if (it > 0) break;  // dense: one item per workgroup
      const int per = sh.nwg / 8;
      const int w = (blockIdx.x % 8) * per + blockIdx.x / 8;
      if (w >= sh.nfb * sh.tiles) break;
      const int tile = sh.xcd_blocked ? w / sh.nfb : w % sh.tiles;
      fb = sh.xcd_blocked ? w % sh.nfb : w / sh.tiles;
      t0 = tile * TN;
      count = min(TN, a.rows - t0);
    }
    const int f0 = fb * FPW;
    const int K = a.K, nch = K / KC;
    // this wave's LL ring loads per chunk, 8 rows x 128 B each: weight rows (TM / NW per wave,
    // j < LW) then token rows (TN / NW per wave); lane -> (row r, slot lane & 7), which holds
    // piece (lane & 7) ^ (r & 7)
    const bf16_t* const wbase = shared ? a.W2 + g * a.w2g : a.W + g * a.wg;
    const int64_t wld = shared ? a.w2ld : K;
    const int upoff = shared ? a.w2up : a.N;
    const bf16_t* src[8];
    int dst[8];
#pragma unroll
    for (int j = 0; j < LL; ++j) {
      const bool tok = j >= LW;
      const int r = (tok ? (TN / NW) * wv + RPL * (j - LW) : (TM / NW) * wv + RPL * j) + (lane >> 3);
      const int pc = (lane & 7) ^ swz(r);
      if (tok) {
        const int slot = t0 + (r < count ? r : 0);  // rows past the tile: the tile's first row
        if (shared) {
          src[j] = a.X2 + g * a.x2g + (int64_t)slot * a.x2s + pc * 8;
        } else {
          const int row = a.slot_row ? a.slot_row[slot] / a.slot_div : slot;
          src[j] = a.X + g * a.xg + (int64_t)row * a.xs + pc * 8;
        }
      } else if (SWIGLU) {
        src[j] = wbase + (f0 + (r >> 5) * 16 + ((r >> 4) & 1) * upoff + (r & 15)) * wld + pc * 8;
      } else {
        src[j] = wbase + (int64_t)min(f0 + r, a.N - 1) * wld + pc * 8;  // a ragged last block repeats row N-1
      }
      dst[j] = (tok ? TM * RB + ((TN / NW) * wv + RPL * (j - LW)) * RB : ((TM / NW) * wv + RPL * j) * RB);
    }
    // the item's K chunks start at a rotation that spreads the workgroups' concurrent requests
    // over the weight rows' address range instead of one column of 128 B lines (C3 grouped
    // gate_up 158.4 -> 153.6 us).  It depends on (expert or shared half, feature block) only:
    // an expert's results do not depend on which other tiles share the launch, and the token
    // tiles of one weight block read its chunks in the same order, so the ones that run
    // together share each chunk's fetch in L2 (a rotation per token tile as well made the
    // reference workload at bsz=256 -- 4 tiles per expert -- 1.5x slower)
    const int rot = sh.xcd_blocked ? 0 : (int)((unsigned)(fb * 7 + g * 13 + (shared ? 3 : 0)) % (unsigned)nch);
    auto issue = [&](int chunk, int buf) {
      int cc = min(chunk, nch - 1) + rot;  // past the last chunk: repeat it (never multiplied)
      if (cc >= nch) cc -= nch;
#pragma unroll
      for (int j = 0; j < LL; ++j)
        __builtin_amdgcn_global_load_lds(src[j] + cc * KC,
                                         (__attribute__((address_space(3))) void*)(lds + buf * SB + dst[j]), 16, 0, 0);
    };
    floatx4_t acc[4][8];
#pragma unroll
    for (int x = 0; x < XM; ++x)
#pragma unroll
      for (int y = 0; y < XN; ++y) acc[x][y] = floatx4_t{0.f, 0.f, 0.f, 0.f};
    const int wa = (wv % RWV) * WM, wt = (wv / RWV) * WN;  // this wave's WM weight rows x WN tokens
    // this wave's MFMA fragments of sub-step s (K 32 s .. 32 s + 31) of the chunk in stage st
    auto frags = [&](const uint8_t* st, int s, bf16x8_t* af, bf16x8_t* bfr) {
      const int pc = 4 * s + kg;
#pragma unroll
      for (int x = 0; x < XM; ++x) {
        const int r = wa + 16 * x + li;
        af[x] = *reinterpret_cast<const bf16x8_t*>(st + r * RB + ((pc ^ swz(r)) * 16));
      }
#pragma unroll
      for (int y = 0; y < XN; ++y) {
        const int t = wt + 16 * y + li;
        bfr[y] = *reinterpret_cast<const bf16x8_t*>(st + TM * RB + t * RB + ((pc ^ swz(t)) * 16));
      }
    };
    auto mfmas = [&](const bf16x8_t* af, const bf16x8_t* bfr) {
#pragma unroll
      for (int x = 0; x < XM; ++x)
#pragma unroll
        for (int y = 0; y < XN; ++y) acc[x][y] = mfma16x16x32(af[x], bfr[y], acc[x][y]);
    };
#pragma unroll
    for (int s = 0; s + 1 < ST; ++s) issue(s, s);
    for (int c0 = 0; c0 < nch; c0 += ST) {
#pragma unroll
      for (int i = 0; i < ST; ++i) {
        const int c = c0 + i;
        if (c >= nch) break;
        // this wave's loads of chunk c have landed (the LL of each newer chunk may not), then
        // every wave's: chunk c is complete in LDS and chunk c - 1's stage is free
        __builtin_amdgcn_s_waitcnt(vmcnt_only((ST - 2) * LL));
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if constexpr (ST == 2 && XM == 4 && XN == 8 && LL == 8) {
          // the prefill shape: the next chunk's 8 ring loads go out one per 4 MFMAs of the
          // first sub-step (sched_barrier pins the order) instead of as one burst that holds
          // up the wave's MFMA issue (8192 x 2816 x 2048: 132.3 -> 121.7 us)
          int cc = min(c + 1, nch - 1) + rot;
          if (cc >= nch) cc -= nch;
          const int buf = (i + 1) % ST;
          bf16x8_t af[4], bfr[8];
          frags(lds + i * SB, 0, af, bfr);
#pragma unroll
          for (int x = 0; x < XM; ++x)
#pragma unroll
            for (int y = 0; y < XN; ++y) {
              acc[x][y] = mfma16x16x32(af[x], bfr[y], acc[x][y]);
              if (y % 4 == 3) {
                const int j = x * 2 + y / 4;
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_global_load_lds(src[j] + cc * KC,
                                                 (__attribute__((address_space(3))) void*)(lds + buf * SB + dst[j]),
                                                 16, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
              }
            }
          frags(lds + i * SB, 1, af, bfr);
          mfmas(af, bfr);
        } else {
          issue(c + ST - 1, (i + ST - 1) % ST);
#pragma unroll
          for (int s = 0; s < KC / 32; ++s) {
            bf16x8_t af[4], bfr[8];
            frags(lds + i * SB, s, af, bfr);
            mfmas(af, bfr);
          }
        }
      }
    }
    // the repeats past the last chunk must land before the workgroup's LDS is released
    __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
    if (SWIGLU) {
      // the wave's row blocks alternate gate (x even) and up (x odd) of feature groups of 16
#pragma unroll
      for (int q = 0; q < XM / 2; ++q)
#pragma unroll
        for (int y = 0; y < XN; ++y) {
          if (wt + 16 * y + li >= count) continue;
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = swiglu_bf(acc[2 * q][y][e], acc[2 * q + 1][y][e]);
          const int n = f0 + (wa >> 1) + 16 * q + 4 * kg;
          if (shared) {
            uint2 o;
            o.x = pack2(v[0], v[1]);
            o.y = pack2(v[2], v[3]);
            *reinterpret_cast<uint2*>(reinterpret_cast<bf16_t*>(a.Y2) + g * a.y2g +
                                      (int64_t)(t0 + wt + 16 * y + li) * a.y2s + n) = o;
          } else {
            gemm_store4(a, g, t0 + wt + 16 * y + li, n, v);
          }
        }
    } else {
#pragma unroll
      for (int x = 0; x < XM; ++x)
#pragma unroll
        for (int y = 0; y < XN; ++y) {
          if (wt + 16 * y + li >= count || f0 + wa + 16 * x >= a.N) continue;
          if (shared) {  // fp32 partial of one half (the halves are summed by the consumer)
            float* yp = reinterpret_cast<float*>(a.Y2) + g * a.y2g + (int64_t)(t0 + wt + 16 * y + li) * a.y2s + f0 +
                        wa + 16 * x + 4 * kg;
            *reinterpret_cast<float4*>(yp) = make_float4(acc[x][y][0], acc[x][y][1], acc[x][y][2], acc[x][y][3]);
            continue;
          }
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = acc_out(a, acc[x][y][e]);
          gemm_store4(a, g, t0 + wt + 16 * y + li, f0 + wa + 16 * x + 4 * kg, v);
        }
    }
    __syncthreads();  // every wave is done with the ring before the next item refills it
  }
}

// grouped: max_tiles entries of a tile table of 64 (big: 256) tokens; dense: a.rows tokens.
// big: 256 weight rows x 256 tokens per 8-wave workgroup (each wave 64 x 128, 4 x 8 MFMA
// blocks), two 64 KB stages (a third does not fit the 160 KB of LDS), one workgroup per CU
// -- for expert tiles of hundreds of tokens (prefill), where the 64 x 64 shape re-reads each
// weight chunk once per 64 tokens and issues one MFMA per 2 KB of LDS reads (C3 prefill
// 7.1 s -> 6.0 s with 128 x 128 per 4-wave workgroup, 5.3 s with 256 x 128 per 8 waves and
// three 48 KB stages; with the later attention changes 4.76 s -> 4.43 s with 256 x 256).
constexpr int kBigRwv = 4, kBigStages = 2, kBigWn = 128;  // big: waves along the weight rows, ring stages,
constexpr int kBigTokens = 2 * kBigWn;                    // tokens per wave; tokens per workgroup
constexpr int kBigRows = 64 * kBigRwv;                 // weight rows per big workgroup
static void launch_dma(const GemmArgs& a, bool swiglu, hipStream_t st, int max_tiles = 0, bool big = false) {
  DmaShape sh;
  sh.xcd_blocked = big;
  const int tn = big ? kBigTokens : 64;
  // plain: a last feature block past N (N % 64 == 0) repeats row N-1 and stores nothing there
  sh.nfb = swiglu ? a.N / (big ? kBigRows / 2 : 32) : (a.N + (big ? kBigRows : 64) - 1) / (big ? kBigRows : 64);
  sh.tiles = a.tiles ? max_tiles : (a.rows + tn - 1) / tn;
  // grouped: resident workgroups (two per CU, big: one) looping over the live items
  sh.nwg = a.tiles ? (big ? kDmaGroupedWgs / 2 : kDmaGroupedWgs) : (sh.nfb * sh.tiles + 7) / 8 * 8;
  if (big) {
    constexpr int lds = kBigStages * (kBigRows + kBigTokens) * 128;
    if (swiglu)
      hipLaunchKernelGGL((gemm_dma_kernel<true, 64, kBigWn, kBigStages, kBigRwv>), dim3(sh.nwg),
                         dim3(128 * kBigRwv), lds, st, a, sh);
    else
      hipLaunchKernelGGL((gemm_dma_kernel<false, 64, kBigWn, kBigStages, kBigRwv>), dim3(sh.nwg),
                         dim3(128 * kBigRwv), lds, st, a, sh);
    return;
  }
  if (swiglu) hipLaunchKernelGGL(gemm_dma_kernel<true>, dim3(sh.nwg), dim3(256), kDmaStages * 16384, st, a, sh);
  else hipLaunchKernelGGL(gemm_dma_kernel<false>, dim3(sh.nwg), dim3(256), kDmaStages * 16384, st, a, sh);
}

// ---------------------------------------------------------------------------
// Expert-grouped MoE GEMMs on e4m3 weights (per-row power-of-two scales), bf16 activations.
// The shape of gemm_dma_kernel's decode form -- 4 waves, 64 weight rows x 2 WN tokens per
// workgroup, direct-to-LDS rings, resident workgroups looping over the live (tile, feature
// block) items, the shared-expert halves as extra tiles -- with the weight rows carried as
// e4m3 bytes (a K chunk of a row takes KC bytes of LDS instead of 2 KC) in a ring of their own
// (SW stages) beside the token ring (ST stages).
// A lane reads 16 e4m3 weights of one row per 64-wide half chunk (ds_read_b128: bytes
// 64 h + 16 kg .. + 15) and decodes them to two bf16 MFMA fragments (v_cvt_scalef32_pk_bf16_fp8,
// exact: e4m3 values are bf16 values), one per 32-wide MFMA step: step s takes K {64 h + 16 kg + 8 s
// .. + 7}, and the token fragments read the same K from their LDS rows.  The row's scale
// multiplies the fp32 accumulator in the epilogue (a power of two: the products are those of
// the dequantized bf16 weights).  The weight reads are native vector loads: as struct-typed
// uint4 loads they carried no TBAA tag, and the compiler then made every one of them wait for
// all ring loads in flight (vmcnt(0) each chunk: C3 gate_up 178 -> 128 us once fixed).
// LDS weight rows of 64 B: piece p (16 B) of row r at slot p ^ ((r >> 1) & 3); of 128 B:
// p ^ (r & 7) -- a 16-byte LDS read is served 8 lanes at a time over 32 four-byte banks, and
// the 8 rows such a group reads then fill all 8 sixteen-byte bank groups (slot p ^ ((r >> 2)
// & 3) left two rows on each: 9.7 M conflict cycles per launch at C3).
// Ring shapes per tile size (measured on MI355X, gate_up + shared halves, 26 layers' weights):
// 32-token tiles: 128-wide K chunks (8 KB of weights per stage), 3 weight + 3 token stages, 768
// resident workgroups (3 per CU) -- 256 rows 105.6 us, 64 rows 76.5 us, against 114.5 / 92.8 us
// with 64-wide chunks in 8 + 4 stages (2 per CU) and 152 / 131 us for the bf16 launches;
// 64-token tiles: 64-wide chunks, 8 + 4 stages, 512 workgroups (256 rows 125.9 us; 128-wide
// chunks need 96 KB of LDS there, one workgroup per CU, 160 us).
constexpr int kF8Wgs32 = 768, kF8Wgs64 = 512;

// 8 e4m3 bytes -> 8 bf16 by v_cvt_scalef32_pk_bf16_fp8 (two per instruction, scale 1: an e4m3
// value is a bf16 value, so the conversion is exact; the row scale is applied in fp32 later)
__device__ __forceinline__ bf16x8_t fp8x8_to_bf16x8(uint32_t w0, uint32_t w1) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, false);
  const bf16x2_t b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, true);
  const bf16x2_t c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, false);
  const bf16x2_t d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, true);
  return as_bf16x8(make_uint4(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                              __builtin_bit_cast(uint32_t, c), __builtin_bit_cast(uint32_t, d)));
}

template <bool SWIGLU, int WN, int KC, int SW, int ST>
__global__ __launch_bounds__(256) void gemm_f8_kernel(const GemmArgs a, const DmaShape sh) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, li = lane & 15, kg = lane >> 4;
  constexpr int NW = 4, TM = 64, TN = 2 * WN;   // waves; weight rows, tokens per workgroup
  constexpr int RW = KC, RB = 2 * KC;           // bytes per weight / token row per chunk (K = KC)
  constexpr int WSB = TM * RW, TSB = TN * RB;   // weight / token stage bytes
  constexpr int RLW = 1024 / RW, RLT = 1024 / RB;  // rows per 1 KB ring load: weights, tokens
  constexpr int LW = TM / (RLW * NW), LT = TN / (RLT * NW);  // ring loads per wave per chunk
  constexpr int LL = LW + LT;
  constexpr int XM = 2, XN = WN / 16;           // MFMA blocks per wave (32 rows x WN tokens)
  constexpr int FPW = SWIGLU ? TM / 2 : TM;     // output features per workgroup
  static_assert((KC == 64 || KC == 128) && LW >= 1 && LW <= 2 && LT >= 1 && LT <= 4 && XN >= 1 && XN <= 4 &&
                    SW % ST == 0, "shape");
  // weight slot swizzle: 64-B rows p ^ ((r >> 1) & 3), 128-B rows p ^ (r & 7) (8 distinct per 8 rows)
  auto wswz = [](int r) { return KC == 64 ? ((r >> 1) & 3) : (r & 7); };
  const uint8_t* const W8 = reinterpret_cast<const uint8_t*>(a.W);
  const uint8_t* const W28 = reinterpret_cast<const uint8_t*>(a.W2);
  const int ns = a.W2 ? 2 * a.s_tiles : 0;
  const int live = ns + min(a.ntiles[0], sh.tiles);
  for (int it = 0;; ++it) {
    const int j = blockIdx.x + it * gridDim.x;
    if (j >= live * sh.nfb) break;
    const int tile = j / sh.nfb, fb = j % sh.nfb;
    int g, t0, count;
    const bool shared = tile < ns;
    if (shared) {  // a shared-expert half's tile of tokens
      g = tile / a.s_tiles;
      t0 = (tile % a.s_tiles) * TN;
      count = min(TN, a.rows - t0);
    } else {
      const int4 tt = reinterpret_cast<const int4*>(a.tiles)[tile - ns];
      g = tt.x;
      t0 = tt.y;
      count = tt.z;
    }
    const int f0 = fb * FPW;
    const int K = a.K, nch = K / KC;
    const uint8_t* const wbase = shared ? W28 + g * a.w2g : W8 + g * a.wg;
    const int64_t wld = shared ? a.w2ld : K;
    const int upoff = shared ? a.w2up : a.N;
    const float* const sbase = shared ? a.S2 + g * a.s2g : a.S + g * a.sg;
    // weight row of tile row r (SwiGLU: per 16 features 16 gate rows then the 16 up rows)
    auto wrow = [&](int r) {
      return SWIGLU ? f0 + (r >> 5) * 16 + ((r >> 4) & 1) * upoff + (r & 15) : min(f0 + r, a.N - 1);
    };
    // the epilogue's scales (rows wa + 16 x + 4 kg + e), requested before the stream
    const int wa = (wv & 1) * 32, wt = (wv >> 1) * WN;
    float sc[2][4];  // literal sizes: the host stub of the template is kept
#pragma unroll
    for (int x = 0; x < XM; ++x)
#pragma unroll
      for (int e = 0; e < 4; ++e) sc[x][e] = sbase[wrow(wa + 16 * x + 4 * kg + e)];
    // ring loads: one of 16 weight rows x 64 B (lane -> row 16 wv + lane / 4, slot lane & 3),
    // LT of 8 token rows x 128 B
    // weight ring loads: LW of RLW rows x RW bytes (lane -> row, slot lane % (RW / 16))
    const uint8_t* wsrc[2];
#pragma unroll
    for (int q = 0; q < LW; ++q) {
      const int r = (TM / NW) * wv + RLW * q + lane / (RW / 16), slot = lane % (RW / 16);
      wsrc[q] = wbase + (int64_t)wrow(r) * wld + (slot ^ wswz(r)) * 16;
    }
    const int wdst = (TM / NW) * wv * RW;
    const uint8_t* tsrc[4];
#pragma unroll
    for (int q = 0; q < LT; ++q) {
      const int r = (TN / NW) * wv + RLT * q + lane / (RB / 16), pc = (lane % (RB / 16)) ^ (r & 7);
      const int slot = t0 + (r < count ? r : 0);  // rows past the tile: the tile's first row
      const bf16_t* x;
      if (shared) {
        x = a.X2 + g * a.x2g + (int64_t)slot * a.x2s;
      } else {
        const int row = a.slot_row ? a.slot_row[slot] / a.slot_div : slot;
        x = a.X + (int64_t)row * a.xs;
      }
      tsrc[q] = reinterpret_cast<const uint8_t*>(x + pc * 8);
    }
    const int tdst = ((TN / NW) * wv) * RB;
#pragma unroll
    for (int x = 0; x < XM; ++x)
#pragma unroll
      for (int e = 0; e < 4; ++e) pin(__float_as_uint(sc[x][e]));
    // K chunks start at a rotation per (expert or half, feature block), as gemm_dma_kernel
    const int rot = (int)((unsigned)(fb * 7 + g * 13 + (shared ? 3 : 0)) % (unsigned)nch);
    auto chunk_of = [&](int c) {  // past the last chunk: repeat it (never multiplied)
      int cc = min(c, nch - 1) + rot;
      return cc >= nch ? cc - nch : cc;
    };
    auto issue_w = [&](int c, int stage) {
      // (the chunk index in a local: with the call inside the builtin's argument hipcc drops
      // the kernel's host launch stub)
      const int cc = chunk_of(c);
#pragma unroll
      for (int q = 0; q < LW; ++q)
        __builtin_amdgcn_global_load_lds(wsrc[q] + cc * RW,
                                         (__attribute__((address_space(3))) void*)(lds + stage * WSB + wdst +
                                                                                   RLW * q * RW),
                                         16, 0, 0);
    };
    auto issue_t = [&](int c, int stage) {
      const int cc = chunk_of(c);
#pragma unroll
      for (int q = 0; q < LT; ++q)
        __builtin_amdgcn_global_load_lds(tsrc[q] + cc * RB,
                                         (__attribute__((address_space(3))) void*)(lds + SW * WSB + stage * TSB + tdst +
                                                                                   RLT * q * RB),
                                         16, 0, 0);
    };
    floatx4_t acc[2][4];
#pragma unroll
    for (int x = 0; x < XM; ++x)
#pragma unroll
      for (int y = 0; y < XN; ++y) acc[x][y] = floatx4_t{0.f, 0.f, 0.f, 0.f};
    // iteration c issues W(c + SW - 1), then T(c + ST - 1); the prologue runs the iterations
    // -(SW - 1) .. -1 of that schedule (a token chunk only from index 0), so before chunk c
    // every wave has exactly (ST - 2) iterations of loads issued after T(c), and T(c) landing
    // means W(c), issued before it, landed too (loads complete in issue order)
#pragma unroll
    for (int k = -(SW - 1); k < 0; ++k) {
      issue_w(k + SW - 1, k + SW - 1);
      if (k + ST - 1 >= 0) issue_t(k + ST - 1, k + ST - 1);
    }
    for (int c0 = 0; c0 < nch; c0 += SW) {
#pragma unroll
      for (int i = 0; i < SW; ++i) {
        const int c = c0 + i;
        if (c >= nch) break;
        __builtin_amdgcn_s_waitcnt(vmcnt_only((ST - 2) * LL));
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        issue_w(c + SW - 1, (i + SW - 1) % SW);
        issue_t(c + ST - 1, (i + ST - 1) % ST);
        const uint8_t* ws = lds + i * WSB;
        const uint8_t* ts = lds + SW * WSB + (i % ST) * TSB;
#pragma unroll
        for (int h = 0; h < KC / 64; ++h) {  // 64-wide halves of the chunk: one weight read, two MFMA steps
          bf16x8_t af[2][2];
#pragma unroll
          for (int x = 0; x < XM; ++x) {
            const int r = wa + 16 * x + li;
            // a native vector load: it keeps its TBAA tag, which lets the compiler tell it apart
            // from the ring loads in flight (as a struct-typed uint4 it waited for all of them)
            const u32x4_t w = *reinterpret_cast<const u32x4_t*>(ws + r * RW + (((4 * h + kg) ^ wswz(r)) * 16));
            af[0][x] = fp8x8_to_bf16x8(w[0], w[1]);
            af[1][x] = fp8x8_to_bf16x8(w[2], w[3]);
          }
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) {
            bf16x8_t bfr[4];
#pragma unroll
            for (int y = 0; y < XN; ++y) {
              const int t = wt + 16 * y + li;
              bfr[y] = *reinterpret_cast<const bf16x8_t*>(ts + t * RB + (((8 * h + 2 * kg + s2) ^ (t & 7)) * 16));
            }
#pragma unroll
            for (int x = 0; x < XM; ++x)
#pragma unroll
              for (int y = 0; y < XN; ++y) acc[x][y] = mfma16x16x32(af[s2][x], bfr[y], acc[x][y]);
          }
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
#pragma unroll
    for (int x = 0; x < XM; ++x)
#pragma unroll
      for (int y = 0; y < XN; ++y)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[x][y][e] *= sc[x][e];
    if (SWIGLU) {  // row block 0 of the wave holds 16 features' gate rows, block 1 their up rows
#pragma unroll
      for (int y = 0; y < XN; ++y) {
        if (wt + 16 * y + li >= count) continue;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = swiglu_bf(acc[0][y][e], acc[1][y][e]);
        const int n = f0 + (wa >> 1) + 4 * kg;
        if (shared) {
          uint2 o;
          o.x = pack2(v[0], v[1]);
          o.y = pack2(v[2], v[3]);
          *reinterpret_cast<uint2*>(reinterpret_cast<bf16_t*>(a.Y2) + g * a.y2g + (int64_t)(t0 + wt + 16 * y + li) * a.y2s +
                                    n) = o;
        } else {
          gemm_store4(a, g, t0 + wt + 16 * y + li, n, v);
        }
      }
    } else {
#pragma unroll
      for (int x = 0; x < XM; ++x)
#pragma unroll
        for (int y = 0; y < XN; ++y) {
          if (wt + 16 * y + li >= count || f0 + wa + 16 * x >= a.N) continue;
          if (shared) {  // fp32 partial of one half (the halves are summed by the consumer)
            float* yp = reinterpret_cast<float*>(a.Y2) + g * a.y2g + (int64_t)(t0 + wt + 16 * y + li) * a.y2s + f0 +
                        wa + 16 * x + 4 * kg;
            *reinterpret_cast<float4*>(yp) = make_float4(acc[x][y][0], acc[x][y][1], acc[x][y][2], acc[x][y][3]);
            continue;
          }
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = rbf(acc[x][y][e]);
          gemm_store4(a, g, t0 + wt + 16 * y + li, f0 + wa + 16 * x + 4 * kg, v);
        }
    }
    __syncthreads();  // every wave is done with the rings before the next item refills them
  }
}

// grouped e4m3 launch: 32- or 64-token tiles (WN 16 / 32), resident workgroups over the items
static void launch_f8(const GemmArgs& a, bool swiglu, int tile_tokens, int max_tiles, hipStream_t st) {
  DmaShape sh{};
  sh.nfb = swiglu ? a.N / 32 : (a.N + 63) / 64;
  sh.tiles = max_tiles;
  if (tile_tokens == 64) {
    constexpr int KC = 64, SW = 8, ST = 4;
    sh.nwg = kF8Wgs64;
    const int lds = SW * 64 * KC + ST * 64 * 2 * KC;
    if (swiglu) hipLaunchKernelGGL((gemm_f8_kernel<true, 32, KC, SW, ST>), dim3(sh.nwg), dim3(256), lds, st, a, sh);
    else hipLaunchKernelGGL((gemm_f8_kernel<false, 32, KC, SW, ST>), dim3(sh.nwg), dim3(256), lds, st, a, sh);
  } else {
    constexpr int KC = 128, SW = 3, ST = 3;
    sh.nwg = kF8Wgs32;
    const int lds = SW * 64 * KC + ST * 32 * 2 * KC;
    if (swiglu) hipLaunchKernelGGL((gemm_f8_kernel<true, 16, KC, SW, ST>), dim3(sh.nwg), dim3(256), lds, st, a, sh);
    else hipLaunchKernelGGL((gemm_f8_kernel<false, 16, KC, SW, ST>), dim3(sh.nwg), dim3(256), lds, st, a, sh);
  }
}

// One-shot shape for dense weights and few tokens (the row blocks alone cannot fill the
// chip): a workgroup owns RBW blocks of 16 features for one tile of 16*TB tokens, and
// KW waves per block split K into 128-wide chunks (wave kw takes chunks kw, kw + KW, ...,
// J of them).  Every wave requests all of its weight chunks at once, in the row-contiguous
// pattern (4 rows x 256 B per load) that streams fastest from HBM, and forms the MFMA A
// fragments through its own LDS tile; token fragments come from L2.  The KW partial tiles
// are summed through LDS in kw order.  The 1-D grid is laid out so the token tiles of one
// row block run on the same XCD (workgroups go round-robin over the 8 XCDs): the first
// tile's weight reads fill that XCD's L2 for the others.
struct OsShape {
  int rbw, kw, row_blocks, tiles, groups, nwg;
};

// bid: the workgroup's index in the launch's gemm_os part (blockIdx.x for gemm_os_kernel)
template <int TB, bool SWIGLU, int J>
__device__ __forceinline__ void gemm_os_body(const GemmArgs& a, const OsShape& sh, int bid) {
  constexpr int R = SWIGLU ? 2 : 1;
  constexpr int AROW = 136;  // LDS tile row (128 k + 8 pad), elements
  // dynamic LDS, os_lds_bytes(): per wave a 16 x AROW tile, reused for the partial tiles
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int li = lane & 15, kg = lane >> 4;
  // XCD-aware work index: XCD x = bid % 8 takes work items [x*per, (x+1)*per)
  const int per = sh.nwg / 8;
  const int w = (bid % 8) * per + bid / 8;
  const int total = sh.row_blocks * sh.tiles * sh.groups;
  if (w >= total) return;
  const int tile = w % sh.tiles, rbg = w / sh.tiles;  // tiles of one row block are adjacent
  const int g = rbg / sh.row_blocks, rblk = rbg % sh.row_blocks;
  const int rb = wv % sh.rbw, kw = wv / sh.rbw;
  const int start = tile * 16 * TB, count = min(16 * TB, a.rows - start);
  const int K = a.K, S = K >> 5;
  const int f0 = (rblk * sh.rbw + rb) * 16;

  // the residual of this wave's first output unit (u = wv below), ahead of the weight stream:
  // the wait for the first weight chunk then covers it
  const int u0b = wv % sh.rbw, u0t = wv / sh.rbw;
  const uint2 rpre = gemm_res_load(a, wv < sh.rbw * TB && u0t * 16 + li < count, start + u0t * 16 + li,
                                   (rblk * sh.rbw + u0b) * 16 + 4 * kg);
  // weight chunks: ab[j][q][r] = rows 4q + (lane >> 4) of block r, k = 128 c_j + (lane & 15) * 8
  uint4 ab[J][4][R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const bf16_t* wp = a.W + g * a.wg + (int64_t)(f0 + r * a.N + (lane >> 4)) * K + (lane & 3) * 8;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int step = (kw + j * sh.kw) * 4 + ((lane & 15) >> 2);
#pragma unroll
      for (int q = 0; q < 4; ++q) ab[j][q][r] = ldg16(wp + (int64_t)q * 4 * K + (int64_t)min(step, S - 1) * 32);
    }
  }
  // token rows in the same pattern: xrow[tb] + q*4 rows = token 16 tb + 4q + (lane >> 4)
  const bf16_t* xrow[TB][4];
#pragma unroll
  for (int tb = 0; tb < TB; ++tb)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int t0 = tb * 16 + 4 * q + (lane >> 4);
      const int t = t0 < count ? t0 : 0;
      xrow[tb][q] = a.X + g * a.xg + (int64_t)(start + t) * a.xs + (lane & 3) * 8;
    }
  floatx4_t acc[R][TB];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) acc[r][tb] = floatx4_t{0.f, 0.f, 0.f, 0.f};

  bf16_t* atile = reinterpret_cast<bf16_t*>(lds) + wv * 16 * AROW;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int s0 = (kw + j * sh.kw) * 4;
    const int step = s0 + ((lane & 15) >> 2);
    // token chunk rows (steps past K: clamped address, zeroed before the LDS store)
    uint4 bx[TB][4];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
      for (int q = 0; q < 4; ++q) bx[tb][q] = ldg16(xrow[tb][q] + (int64_t)min(step, S - 1) * 32);
    // weight and token 16 x 128 tiles through the wave's LDS tile into MFMA fragments
    bf16x8_t afr[4][R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<uint4*>(atile + (4 * q + (lane >> 4)) * AROW + (lane & 15) * 8) = ab[j][q][r];
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
      for (int si = 0; si < 4; ++si)
        afr[si][r] = *reinterpret_cast<const bf16x8_t*>(atile + li * AROW + si * 32 + kg * 8);
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    }
    if (j == 0) {
      pin(rpre.x);
      pin(rpre.y);
    }
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<uint4*>(atile + (4 * q + (lane >> 4)) * AROW + (lane & 15) * 8) = keep_if(step < S, bx[tb][q]);
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
      for (int si = 0; si < 4; ++si) {
        const bf16x8_t bfr = *reinterpret_cast<const bf16x8_t*>(atile + li * AROW + si * 32 + kg * 8);
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r][tb] = mfma16x16x32(afr[si][r], bfr, acc[r][tb]);
      }
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    }
  }

  // sum the KW partial tiles in kw order (the A tiles are dead after the barrier); the
  // RBW * TB (row block, token block) outputs are spread over the waves
  floatx4_t* red = reinterpret_cast<floatx4_t*>(lds);
  __syncthreads();
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) red[(((kw * sh.rbw + rb) * R + r) * TB + tb) * 64 + lane] = acc[r][tb];
  __syncthreads();
  const int nw = sh.rbw * sh.kw;
  for (int u = wv; u < sh.rbw * TB; u += nw) {
    const int urb = u % sh.rbw, tb = u / sh.rbw;
    if (tb * 16 + li >= count) continue;
    floatx4_t sum[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      sum[r] = red[((urb * R + r) * TB + tb) * 64 + lane];
      for (int q = 1; q < sh.kw; ++q) sum[r] += red[(((q * sh.rbw + urb) * R + r) * TB + tb) * 64 + lane];
    }
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = SWIGLU ? swiglu_bf(sum[0][e], sum[R - 1][e]) : acc_out(a, sum[0][e]);
    const int slot = start + tb * 16 + li, n = (rblk * sh.rbw + urb) * 16 + 4 * kg;
    if (u == wv)
      gemm_store4r(a, g, slot, n, v, rpre);
    else
      gemm_store4(a, g, slot, n, v);
  }
}

template <int TB, bool SWIGLU, int J>
__global__ __launch_bounds__(1024) void gemm_os_kernel(const GemmArgs a, const OsShape sh) {
  gemm_os_body<TB, SWIGLU, J>(a, sh, blockIdx.x);
}

// Shape of a one-shot launch for an implicit-tile GEMM, or rbw = 0 if it does not apply.
static OsShape os_shape(const GemmArgs& a, int tb, bool swiglu, int groups, int* j_out, int kwmax = 16) {
  OsShape sh{};
  const int nc = ((a.K >> 5) + 3) / 4;  // 128-wide chunks
  const int jmax = (swiglu || tb >= 4) ? 1 : 2;  // register budget of gemm_os_kernel
  int j = (nc + kwmax - 1) / kwmax;
  if (j > jmax) return sh;
  int kw = (nc + j - 1) / j;
  int rbw = 1;
  while (rbw * kw * 2 <= 8 && a.N % (16 * rbw * 2) == 0) rbw *= 2;  // at least ~8 waves when K is short
  if (a.N % (16 * rbw) != 0) return sh;
  sh.rbw = rbw;
  sh.kw = kw;
  sh.row_blocks = a.N / (16 * rbw);
  sh.tiles = a.tiles_per_group;
  sh.groups = groups;
  const int total = sh.row_blocks * sh.tiles * groups;
  sh.nwg = (total + 7) / 8 * 8;
  *j_out = j;
  return sh;
}

static int os_lds_bytes(const OsShape& sh, int tb, bool swiglu) {
  const int nw = sh.rbw * sh.kw;
  const int tiles = nw * 16 * 136 * 2, red = nw * (swiglu ? 2 : 1) * tb * 1024;
  return tiles > red ? tiles : red;
}

template <int TB, bool SWIGLU, int J>
static void launch_os_variant(const GemmArgs& a, const OsShape& sh, hipStream_t st) {
  hipLaunchKernelGGL((gemm_os_kernel<TB, SWIGLU, J>), dim3(sh.nwg), dim3(sh.rbw * sh.kw * 64),
                     os_lds_bytes(sh, TB, SWIGLU), st, a, sh);
}

// features per workgroup of gemm_xlds_kernel
static int xlds_features(bool swiglu) { return swiglu ? 32 : 64; }

template <int TB, bool SWIGLU, int CS, bool AST, int DEPTH, int NRB = (SWIGLU ? 2 : 4), int XD = 1, bool NTA = false>
static void launch_xlds_variant(const GemmArgs& a, int grid_y, hipStream_t st) {
  hipLaunchKernelGGL((gemm_xlds_kernel<TB, SWIGLU, CS, AST, DEPTH, NRB, XD, NTA>), dim3(a.N / (16 * NRB), grid_y),
                     dim3(512), 0, st, a);
}

static int launch_gemm_xlds(const GemmArgs& a, int tb, bool swiglu, int grid_y, hipStream_t st) {
  // Variants measured on MI355X for the expert-grouped MoE (64 experts, 16/32/64-token
  // tiles): row-contiguous weight staging wherever its LDS tiles fit next to the token
  // chunks; SwiGLU with 2+ token blocks takes 64 features (4 blocks x 2 k ranges) so each
  // token chunk in LDS serves twice the weight rows (bsz=256 gate_up 178 -> 140 us); with
  // 32-token tiles also non-temporal weight loads and two token chunks in flight (140 ->
  // 130 us; the same loads measured slower for 16-token tiles).  The down projection on
  // 32-token tiles takes the two token chunks in flight with ordinary weight loads (bsz=64
  // grouped down + shared halves 72.3 -> 67.8 us; with non-temporal loads 68.2).
  const bool wide = a.N % 64 == 0;
  if (swiglu) {
    if (tb == 1) launch_xlds_variant<1, true, 4, true, 2>(a, grid_y, st);
    else if (tb == 2 && wide) launch_xlds_variant<2, true, 4, true, 2, 4, 2, true>(a, grid_y, st);
    else if (tb == 2) launch_xlds_variant<2, true, 4, true, 2>(a, grid_y, st);
    else if (wide) launch_xlds_variant<4, true, 4, true, 2, 4>(a, grid_y, st);
    else launch_xlds_variant<4, true, 2, false, 2>(a, grid_y, st);
  } else {
    if (tb == 1) launch_xlds_variant<1, false, 4, true, 2>(a, grid_y, st);
    else if (tb == 2) launch_xlds_variant<2, false, 4, true, 2, 4, 2>(a, grid_y, st);
    else if (tb == 4) launch_xlds_variant<4, false, 4, false, 2>(a, grid_y, st);
    else launch_xlds_variant<8, false, 2, false, 2>(a, grid_y, st);
  }
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

// Dense (implicit-tile) shapes whose row blocks alone cannot fill the chip, measured on
// MI355X at 16..256 tokens: the one-shot kernel for short K and up to 64 tokens; the
// token-rows-in-LDS kernel (64-row workgroups sharing token chunks) for more tokens, with
// the largest token tile that still gives ~200 workgroups (SwiGLU: 64-token tiles); long K
// with few features on 16/32-token tiles.  Returns false (nothing launched) for shapes left
// to launch_gemm: huge N, long K with SwiGLU or groups, or N not a multiple of 16*rbw.
constexpr int kBigTileRows = 512;
static bool launch_dense_os(GemmArgs a, int groups, bool swiglu, hipStream_t st) {
  const int rows = a.rows, K = a.K;
  if (K > 4096 && !swiglu && groups == 1 && a.N % 64 == 0 && a.N < 16384) {
    // long K, few features (dense layer-0 down, K = 10944): token-rows-in-LDS tiles of 16 /
    // 32 tokens with row-contiguous weight staging (bsz=256: 51 us vs 97 us for the k-split
    // kernel's MFMA-fragment-order loads; bsz=64: 41 vs 62 us)
    const int tb = rows <= 64 ? 1 : 2;
    a.tiles_per_group = (rows + 16 * tb - 1) / (16 * tb);
    if (a.tiles_per_group > 65535) return false;
    if (tb == 1) launch_xlds_variant<1, false, 4, true, 2>(a, a.tiles_per_group, st);
    else launch_xlds_variant<2, false, 4, true, 2>(a, a.tiles_per_group, st);
    return true;
  }
  if (groups == 1 && K <= 4096 && rows >= kBigTileRows && a.N >= kBigRows &&
      a.N % (swiglu ? kBigRows / 2 : 64) == 0) {
    // prefill-size row counts: 128 weight rows x 128 tokens per workgroup
    launch_dma(a, swiglu, st, 0, true);
    return true;
  }
  if (!swiglu && groups == 1 && K <= 4096 && a.N % 64 == 0 &&
      ((rows > 128 && (a.N / 64) * ((rows + 63) / 64) >= 192) || (rows > 32 && a.N >= 16384))) {
    // direct-to-LDS ring: 128+ tokens with enough 64 x 64 tiles to fill the chip (qkv_a at
    // 256 tokens, 228 workgroups: 12.9 vs 16.1 us in the decode step; N = 2048 gives only 128
    // and stays on the token-rows-in-LDS shape's 32-token tiles, o_proj 12.9 vs 14.0 us), and
    // the lm_head (N = 102400) from 33 tokens (64: 104 vs 121 us; 256: 251 vs 301 us)
    launch_dma(a, false, st);
    return true;
  }
  if (swiglu && groups == 1 && K <= 4096 && a.N % 32 == 0 && rows > 128) {
    // SwiGLU on the ring (32 features x 64 tokens per workgroup): shared experts and the dense
    // layer-0 gate_up above 128 tokens (reference workload at 256 rows 39.3k -> 39.4k tok/s)
    launch_dma(a, true, st);
    return true;
  }
  if (K > 4096 || (int64_t)a.N * groups >= 16384) return false;
  if (swiglu && K > 512 && rows > 64 && a.N % 64 == 0) {
    // 64-token tiles, 64 features (gate + up rows) per workgroup, two token chunks in flight
    // (shared experts at 256 tokens: 22.4 us vs 28.8 us for the one-shot shape)
    a.tiles_per_group = (rows + 63) / 64;
    const int64_t gy = (int64_t)a.tiles_per_group * groups;
    if (gy > 65535) return false;
    launch_xlds_variant<4, true, 4, true, 2, 4, 2>(a, (int)gy, st);
    return true;
  }
  if (!swiglu && K > 512 && rows > 64 && a.N % 64 == 0) {
    int tb = 1;
    for (int t : {2, 4}) {
      const int64_t tiles = (rows + 16 * t - 1) / (16 * t);
      if ((int64_t)(a.N / 64) * tiles * groups >= 200) tb = t;
    }
    a.tiles_per_group = (rows + 16 * tb - 1) / (16 * tb);
    const int64_t gy = (int64_t)a.tiles_per_group * groups;
    if (gy > 65535) return false;
    if (tb == 1) launch_xlds_variant<1, false, 4, true, 2>(a, (int)gy, st);
    else if (tb == 2) launch_xlds_variant<2, false, 4, true, 2>(a, (int)gy, st);
    else launch_xlds_variant<4, false, 4, true, 2, 4, 2>(a, (int)gy, st);  // two token chunks in flight
    return true;
  }
  const int tb = K <= 512 ? (rows <= 64 ? 1 : 2) : (swiglu ? (rows <= 16 ? 1 : (rows <= 32 ? 2 : 4)) : (rows <= 16 ? 1 : 2));
  a.tiles_per_group = (rows + 16 * tb - 1) / (16 * tb);
  int j = 0;
  OsShape sh = os_shape(a, tb, swiglu, groups, &j, swiglu ? 16 : 8);
  if (!sh.rbw) sh = os_shape(a, tb, swiglu, groups, &j, 16);
  if (!sh.rbw || (int64_t)sh.nwg > (int64_t)1 << 30) return false;
#define DSV2_OS(TBV, JV)                                                          \
  (swiglu ? launch_os_variant<TBV, true, 1>(a, sh, st) : launch_os_variant<TBV, false, JV>(a, sh, st))
  if (tb == 1) { if (j == 1) DSV2_OS(1, 1); else DSV2_OS(1, 2); }
  else if (tb == 2) { if (j == 1) DSV2_OS(2, 1); else DSV2_OS(2, 2); }
  else DSV2_OS(4, 1);
#undef DSV2_OS
  return true;
}

extern "C" int dsv2_gemm_bf16(const void* x, int64_t x_stride, int64_t x_gstride, int rows, int K, const void* W,
                              int64_t w_gstride, int N, int n_groups, const void* residual, int64_t res_stride,
                              void* y, int64_t y_stride, int64_t y_gstride, int flags, void* stream) {
  DSV2_REQUIRE(x && W && y, DSV2_E_NULL, "gemm: null pointer");
  DSV2_REQUIRE(rows >= 0 && K > 0 && K % 64 == 0 && N > 0 && N % 16 == 0 && n_groups >= 1, DSV2_E_SHAPE,
               "gemm: bad shape rows=%d K=%d N=%d groups=%d (K%%64, N%%16 required)", rows, K, N, n_groups);
  DSV2_REQUIRE((flags & ~(DSV2_LINEAR_SWIGLU | DSV2_LINEAR_OUT_F32 | DSV2_LINEAR_OUT_F32_EXACT)) == 0, DSV2_E_FLAGS,
               "gemm: unknown flags");
  DSV2_REQUIRE(!(residual && ((flags & DSV2_LINEAR_SWIGLU) || n_groups != 1)), DSV2_E_FLAGS,
               "gemm: residual needs a plain single-group GEMM");
  DSV2_REQUIRE(!((flags & DSV2_LINEAR_OUT_F32_EXACT) && ((flags & DSV2_LINEAR_SWIGLU) || residual)), DSV2_E_FLAGS,
               "gemm: the exact fp32 output takes no SwiGLU and no residual");
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
  a.out_f32 = flags & (DSV2_LINEAR_OUT_F32 | DSV2_LINEAR_OUT_F32_EXACT);
  a.exact_f32 = flags & DSV2_LINEAR_OUT_F32_EXACT;
  const bool swiglu = flags & DSV2_LINEAR_SWIGLU;
  if (launch_dense_os(a, n_groups, swiglu, (hipStream_t)stream)) return dsv2_launch_status("gemm");
  const int64_t grid_y = (int64_t)a.tiles_per_group * n_groups;
  DSV2_REQUIRE(grid_y <= 65535, DSV2_E_SHAPE, "gemm: too many row tiles (%lld)", (long long)grid_y);
  return launch_gemm(a, tb, swiglu, (int)grid_y, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// Batch-family decode preparation in one launch: the absorbed queries
// q_lat[r, h, :512] = W_UK_h^T q_nope[r, h] (16 head groups, K = 128, N = 512: the one-shot
// GEMM's workgroups, with the shape and arithmetic dsv2_gemm_bf16 gives this product) and
// mla_prepare's per-row work (RoPE(q_pe), the token's new cache row), two rows per workgroup,
// after them.  Both parts only read qkva and write disjoint columns of q_out (and the cache),
// so they need no ordering: one launch instead of two dependent ones.
// ---------------------------------------------------------------------------
template <int TB>
__global__ __launch_bounds__(512) void mla_prepare_qlat_kernel(const GemmArgs a, const OsShape sh,
                                                               const MlaRowArgs m) {
  if ((int)blockIdx.x < sh.nwg) {
    gemm_os_body<TB, false, 1>(a, sh, blockIdx.x);
    return;
  }
  const int b = ((int)blockIdx.x - sh.nwg) * 2 + (int)(threadIdx.x >> 8);
  if (b < a.rows) mla_prepare_row(m, b, threadIdx.x & 255);
}

extern "C" int dsv2_mla_prepare_qlat(const void* qkva, int64_t qkva_stride, int rows, const int32_t* pos,
                                     const int64_t* base, const int32_t* cap, const void* kv_norm_w, float eps,
                                     const void* rope_cos, const void* rope_sin, int max_pos, const void* w_ukt,
                                     void* cache, void* q_out, int32_t* status, void* stream) {
  DSV2_REQUIRE(qkva && pos && base && cap && kv_norm_w && rope_cos && rope_sin && w_ukt && cache && q_out,
               DSV2_E_NULL, "mla_prepare_qlat: null pointer");
  DSV2_REQUIRE(rows >= 0 && rows <= 65535 && max_pos > 0 && qkva_stride >= 3648, DSV2_E_SHAPE,
               "mla_prepare_qlat: bad shape");
  DSV2_REQUIRE(dsv2_aligned16(qkva) && qkva_stride % 8 == 0 && dsv2_aligned16(kv_norm_w) && dsv2_aligned16(cache) &&
                   dsv2_aligned16(q_out) && dsv2_aligned16(w_ukt),
               DSV2_E_ALIGN, "mla_prepare_qlat: alignment");
  if (rows == 0) return DSV2_OK;
  constexpr int kHeadsQ = 16, kRowQ = 576, kLatQ = 512, kNopeQ = 128;
  GemmArgs a{};
  a.X = (const bf16_t*)qkva;  // q_nope of head g: columns 192 g .. 192 g + 127
  a.xs = qkva_stride;
  a.xg = 192;
  a.slot_div = 1;
  a.rows = rows;
  const int tb = rows <= 64 ? 1 : 2;  // dsv2_gemm_bf16's token tile for K <= 512
  a.tiles_per_group = (rows + 16 * tb - 1) / (16 * tb);
  a.W = (const bf16_t*)w_ukt;  // [16][512][128]
  a.wg = (int64_t)kLatQ * kNopeQ;
  a.N = kLatQ;
  a.K = kNopeQ;
  a.Y = q_out;
  a.ys = kHeadsQ * kRowQ;
  a.yg = kRowQ;
  int j = 0;
  const OsShape sh = os_shape(a, tb, false, kHeadsQ, &j, 8);
  DSV2_REQUIRE(sh.rbw * sh.kw == 8 && j == 1, DSV2_E_SHAPE, "mla_prepare_qlat: unexpected GEMM shape");
  const MlaRowArgs m{(const bf16_t*)qkva, qkva_stride, pos, base, cap, (const bf16_t*)kv_norm_w, eps,
                     (const bf16_t*)rope_cos, (const bf16_t*)rope_sin, max_pos, (bf16_t*)cache, (bf16_t*)q_out,
                     status};
  const dim3 grid(sh.nwg + (rows + 1) / 2);
  if (tb == 1)
    hipLaunchKernelGGL(mla_prepare_qlat_kernel<1>, grid, dim3(512), os_lds_bytes(sh, 1, false), (hipStream_t)stream,
                       a, sh, m);
  else
    hipLaunchKernelGGL(mla_prepare_qlat_kernel<2>, grid, dim3(512), os_lds_bytes(sh, 2, false), (hipStream_t)stream,
                       a, sh, m);
  return dsv2_launch_status("mla_prepare_qlat");
}

static int tile_tb(int tile_tokens) { return tile_tokens == 16 ? 1 : (tile_tokens == 32 ? 2 : 4); }

extern "C" int dsv2_moe_grouped_gateup(const void* xn, const int32_t* sorted_routes, const int32_t* tiles,
                                       const int32_t* num_tiles, int max_tiles, int tile_tokens, const void* w_gate_up,
                                       int inter, void* hsorted, void* stream) {
  DSV2_REQUIRE(xn && sorted_routes && tiles && num_tiles && w_gate_up && hsorted, DSV2_E_NULL,
               "moe_grouped_gateup: null pointer");
  DSV2_REQUIRE(max_tiles >= 0 && max_tiles <= 65535 && inter > 0 && inter % 16 == 0 &&
                   (tile_tokens == 16 || tile_tokens == 32 || tile_tokens == 64 || tile_tokens == kBigTokens),
               DSV2_E_SHAPE, "moe_grouped_gateup: bad shape (inter %% 16, tile_tokens in {16,32,64,256})");
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
  if ((tile_tokens == 64 && inter % 32 == 0) || (tile_tokens == kBigTokens && inter % (kBigRows / 2) == 0)) {
    // 64- and 256-token tiles on the direct-to-LDS ring (reference workload, 6 experts x 256
    // tokens: 45 us vs 71 us for the token-rows-in-LDS shape; x 64 tokens: 26.0 vs 26.8 us)
    launch_dma(a, true, (hipStream_t)stream, max_tiles, tile_tokens == kBigTokens);
    return dsv2_launch_status("moe_grouped_gateup");
  }
  DSV2_REQUIRE(tile_tokens != kBigTokens, DSV2_E_SHAPE, "moe_grouped_gateup: 256-token tiles need inter %% %d", kBigRows / 2);
  return launch_gemm(a, tile_tb(tile_tokens), true, max_tiles, (hipStream_t)stream);
}

extern "C" int dsv2_moe_grouped_gateup_shared(const void* xn, int rows, const int32_t* sorted_routes,
                                              const int32_t* tiles, const int32_t* num_tiles, int max_tiles,
                                              int tile_tokens, const void* w_gate_up, const void* sh_gate_up,
                                              int inter, void* hsorted, void* shared_out, void* stream) {
  DSV2_REQUIRE(xn && sorted_routes && tiles && num_tiles && w_gate_up && sh_gate_up && hsorted && shared_out,
               DSV2_E_NULL, "moe_grouped_gateup_shared: null pointer");
  DSV2_REQUIRE(rows >= 0 && max_tiles >= 0 && max_tiles <= 65535 && inter > 0 && inter % 64 == 0 &&
                   (tile_tokens == 16 || tile_tokens == 32 || tile_tokens == 64 || tile_tokens == kBigTokens) &&
                   (tile_tokens >= 64 || (int64_t)max_tiles + 2 * ((rows + tile_tokens - 1) / tile_tokens) <= 65535),
               DSV2_E_SHAPE, "moe_grouped_gateup_shared: bad shape (inter %% 64, tile_tokens in {16,32,64,256})");
  DSV2_REQUIRE(dsv2_aligned16(xn) && dsv2_aligned16(w_gate_up) && dsv2_aligned16(sh_gate_up) &&
                   dsv2_aligned16(tiles) && dsv2_aligned16(shared_out),
               DSV2_E_ALIGN, "moe_grouped_gateup_shared: alignment");
  if (rows == 0) return DSV2_OK;
  GemmArgs a{};
  a.X = (const bf16_t*)xn;
  a.xs = 2048;
  a.slot_row = sorted_routes;
  a.slot_div = 6;
  a.tiles = tiles;
  a.ntiles = num_tiles;
  a.rows = rows;
  a.W = (const bf16_t*)w_gate_up;
  a.wg = (int64_t)2 * inter * 2048;
  a.N = inter;
  a.K = 2048;
  a.Y = hsorted;
  a.ys = inter;
  a.X2 = (const bf16_t*)xn;
  a.x2s = 2048;
  a.W2 = (const bf16_t*)sh_gate_up;
  a.w2g = (int64_t)inter * 2048;
  a.w2ld = 2048;
  a.w2up = 2 * inter;
  a.s_tiles = (rows + tile_tokens - 1) / tile_tokens;
  a.Y2 = shared_out;
  a.y2s = 2 * inter;
  a.y2g = inter;
  if (tile_tokens >= 64) {
    launch_dma(a, true, (hipStream_t)stream, max_tiles, tile_tokens == kBigTokens);
    return dsv2_launch_status("moe_grouped_gateup_shared");
  }
  return launch_gemm(a, tile_tb(tile_tokens), true, 2 * a.s_tiles + max_tiles, (hipStream_t)stream);
}

extern "C" int dsv2_moe_grouped_down_shared(const void* hsorted, int rows, const int32_t* tiles,
                                            const int32_t* num_tiles, int max_tiles, int tile_tokens,
                                            const void* w_down, const void* shared_mid, const void* sh_down, int inter,
                                            void* ysorted, float* shared_parts, void* stream) {
  DSV2_REQUIRE(hsorted && tiles && num_tiles && w_down && shared_mid && sh_down && ysorted && shared_parts,
               DSV2_E_NULL, "moe_grouped_down_shared: null pointer");
  DSV2_REQUIRE(rows >= 0 && max_tiles >= 0 && max_tiles <= 65535 && inter > 0 && inter % 64 == 0 &&
                   (tile_tokens == 16 || tile_tokens == 32 || tile_tokens == 64 || tile_tokens == kBigTokens) &&
                   (tile_tokens >= 64 || (int64_t)max_tiles + 2 * ((rows + tile_tokens - 1) / tile_tokens) <= 65535),
               DSV2_E_SHAPE, "moe_grouped_down_shared: bad shape (inter %% 64, tile_tokens in {16,32,64,256})");
  DSV2_REQUIRE(dsv2_aligned16(hsorted) && dsv2_aligned16(w_down) && dsv2_aligned16(shared_mid) &&
                   dsv2_aligned16(sh_down) && dsv2_aligned16(tiles) && dsv2_aligned16(ysorted) &&
                   dsv2_aligned16(shared_parts),
               DSV2_E_ALIGN, "moe_grouped_down_shared: alignment");
  if (rows == 0) return DSV2_OK;
  GemmArgs a{};
  a.X = (const bf16_t*)hsorted;
  a.xs = inter;
  a.slot_div = 1;
  a.tiles = tiles;
  a.ntiles = num_tiles;
  a.rows = rows;
  a.W = (const bf16_t*)w_down;
  a.wg = (int64_t)2048 * inter;
  a.N = 2048;
  a.K = inter;
  a.Y = ysorted;
  a.ys = 2048;
  a.X2 = (const bf16_t*)shared_mid;
  a.x2s = 2 * inter;
  a.x2g = inter;
  a.W2 = (const bf16_t*)sh_down;
  a.w2g = inter;
  a.w2ld = 2 * inter;
  a.s_tiles = (rows + tile_tokens - 1) / tile_tokens;
  a.Y2 = shared_parts;
  a.y2s = 2048;
  a.y2g = (int64_t)rows * 2048;
  if (tile_tokens >= 64) {
    launch_dma(a, false, (hipStream_t)stream, max_tiles, tile_tokens == kBigTokens);
    return dsv2_launch_status("moe_grouped_down_shared");
  }
  return launch_gemm(a, tile_tb(tile_tokens), false, 2 * a.s_tiles + max_tiles, (hipStream_t)stream);
}

extern "C" int dsv2_moe_grouped_down(const void* hsorted, const int32_t* tiles, const int32_t* num_tiles,
                                     int max_tiles, int tile_tokens, const void* w_down, int inter, void* ysorted,
                                     void* stream) {
  DSV2_REQUIRE(hsorted && tiles && num_tiles && w_down && ysorted, DSV2_E_NULL, "moe_grouped_down: null pointer");
  DSV2_REQUIRE(max_tiles >= 0 && max_tiles <= 65535 && inter > 0 && inter % 64 == 0 &&
                   (tile_tokens == 16 || tile_tokens == 32 || tile_tokens == 64 || tile_tokens == kBigTokens),
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
  if (tile_tokens >= 64) {
    // 6 experts x 256 tokens: 24 us vs 35 us; x 64 tokens: 12.0 vs 16.3 us
    launch_dma(a, false, (hipStream_t)stream, max_tiles, tile_tokens == kBigTokens);
    return dsv2_launch_status("moe_grouped_down");
  }
  return launch_gemm(a, tile_tb(tile_tokens), false, max_tiles, (hipStream_t)stream);
}

// ---- e4m3 expert weights (batch family) ------------------------------------------------
extern "C" int dsv2_moe_grouped_gateup_shared_fp8(const void* xn, int rows, const int32_t* sorted_routes,
                                                  const int32_t* tiles, const int32_t* num_tiles, int max_tiles,
                                                  int tile_tokens, const void* w_gate_up8, const float* gu_scale,
                                                  const void* sh_gate_up8, const float* sh_gu_scale, int inter,
                                                  void* hsorted, void* shared_out, void* stream) {
  DSV2_REQUIRE(xn && sorted_routes && tiles && num_tiles && w_gate_up8 && gu_scale && sh_gate_up8 && sh_gu_scale &&
                   hsorted && shared_out,
               DSV2_E_NULL, "moe_grouped_gateup_shared_fp8: null pointer");
  DSV2_REQUIRE(rows >= 0 && max_tiles >= 0 && max_tiles <= 65535 && inter > 0 && inter % 64 == 0 &&
                   (tile_tokens == 32 || tile_tokens == 64),
               DSV2_E_SHAPE, "moe_grouped_gateup_shared_fp8: bad shape (inter %% 64, tile_tokens in {32,64})");
  DSV2_REQUIRE(dsv2_aligned16(xn) && dsv2_aligned16(w_gate_up8) && dsv2_aligned16(sh_gate_up8) &&
                   dsv2_aligned16(tiles) && dsv2_aligned16(shared_out) && dsv2_aligned16(hsorted),
               DSV2_E_ALIGN, "moe_grouped_gateup_shared_fp8: alignment");
  if (rows == 0) return DSV2_OK;
  GemmArgs a{};
  a.X = (const bf16_t*)xn;
  a.xs = 2048;
  a.slot_row = sorted_routes;
  a.slot_div = 6;
  a.tiles = tiles;
  a.ntiles = num_tiles;
  a.rows = rows;
  a.W = (const bf16_t*)w_gate_up8;  // e4m3 bytes: group and row strides below count bytes
  a.wg = (int64_t)2 * inter * 2048;
  a.N = inter;
  a.K = 2048;
  a.Y = hsorted;
  a.ys = inter;
  a.X2 = (const bf16_t*)xn;
  a.x2s = 2048;
  a.W2 = (const bf16_t*)sh_gate_up8;
  a.w2g = (int64_t)inter * 2048;
  a.w2ld = 2048;
  a.w2up = 2 * inter;
  a.s_tiles = (rows + tile_tokens - 1) / tile_tokens;
  a.Y2 = shared_out;
  a.y2s = 2 * inter;
  a.y2g = inter;
  a.S = gu_scale;
  a.sg = 2 * inter;
  a.S2 = sh_gu_scale;
  a.s2g = inter;
  launch_f8(a, true, tile_tokens, max_tiles, (hipStream_t)stream);
  return dsv2_launch_status("moe_grouped_gateup_shared_fp8");
}

extern "C" int dsv2_moe_grouped_down_shared_fp8(const void* hsorted, int rows, const int32_t* tiles,
                                                const int32_t* num_tiles, int max_tiles, int tile_tokens,
                                                const void* w_down8, const float* down_scale, const void* shared_mid,
                                                const void* sh_down8, const float* sh_down_scale, int inter,
                                                void* ysorted, float* shared_parts, void* stream) {
  DSV2_REQUIRE(hsorted && tiles && num_tiles && w_down8 && down_scale && shared_mid && sh_down8 && sh_down_scale &&
                   ysorted && shared_parts,
               DSV2_E_NULL, "moe_grouped_down_shared_fp8: null pointer");
  DSV2_REQUIRE(rows >= 0 && max_tiles >= 0 && max_tiles <= 65535 && inter > 0 && inter % 64 == 0 &&
                   (tile_tokens == 32 || tile_tokens == 64),
               DSV2_E_SHAPE, "moe_grouped_down_shared_fp8: bad shape (inter %% 64, tile_tokens in {32,64})");
  DSV2_REQUIRE(dsv2_aligned16(hsorted) && dsv2_aligned16(w_down8) && dsv2_aligned16(shared_mid) &&
                   dsv2_aligned16(sh_down8) && dsv2_aligned16(tiles) && dsv2_aligned16(ysorted) &&
                   dsv2_aligned16(shared_parts),
               DSV2_E_ALIGN, "moe_grouped_down_shared_fp8: alignment");
  if (rows == 0) return DSV2_OK;
  GemmArgs a{};
  a.X = (const bf16_t*)hsorted;
  a.xs = inter;
  a.slot_div = 1;
  a.tiles = tiles;
  a.ntiles = num_tiles;
  a.rows = rows;
  a.W = (const bf16_t*)w_down8;
  a.wg = (int64_t)2048 * inter;
  a.N = 2048;
  a.K = inter;
  a.Y = ysorted;
  a.ys = 2048;
  a.X2 = (const bf16_t*)shared_mid;
  a.x2s = 2 * inter;
  a.x2g = inter;
  a.W2 = (const bf16_t*)sh_down8;
  a.w2g = inter;
  a.w2ld = 2 * inter;
  a.s_tiles = (rows + tile_tokens - 1) / tile_tokens;
  a.Y2 = shared_parts;
  a.y2s = 2048;
  a.y2g = (int64_t)rows * 2048;
  a.S = down_scale;
  a.sg = 2048;
  a.S2 = sh_down_scale;
  a.s2g = 0;  // the two halves split K: the same output rows, the same scales
  launch_f8(a, false, tile_tokens, max_tiles, (hipStream_t)stream);
  return dsv2_launch_status("moe_grouped_down_shared_fp8");
}
