// Absorbed multi-head latent attention (MLA) for q_len = 1 over the compressed
// cache: one 576-wide bf16 row per token (512 normalised latent + 64 rotated
// k_pe), shared by all 16 heads.
//
//   prepare : kv-norm + RoPE(k_pe) -> cache row; RoPE(q_pe); q_lat = W_UK^T q_nope
//   decode  : split-KV flash decoding; per workgroup one (row, split); 32-token
//             tiles double-buffered in LDS, two more in flight in registers; S^T = K Q^T
//             and O^T += V^T P^T on v_mfma_f32_16x16x32_bf16 (16 heads = one MFMA
//             dimension), V^T fragments by transposed LDS reads
//   combine : log-sum-exp merge of the splits, then W_UV (fused GEMV) or bf16 o_lat
#include "common.h"
#include "mla_rows.h"

namespace {
constexpr int kHeads = 16;
constexpr int kRow = 576;       // cache row (elements)
constexpr int kLat = 512;       // latent part
constexpr int kQkvA = 3648;     // q (16*192) | latent (512) | k_pe (64)
constexpr int kTile = 32;       // tokens per LDS tile
constexpr int kLdsRow = kRow + 8;  // padded LDS row (elements): 1168 bytes
}  // namespace

// Workgroup (x, y) handles rows y*RB .. y*RB+RB-1.  With w_ukt != null workgroups x < 128
// each compute 64 of the 16*512 absorbed outputs (rows of W_UK_h^T, K = 128 split over 16
// lanes, weights requested first) and workgroup x == 128 writes the new cache rows
// (kv-norm + RoPE(k_pe)) and RoPE(q_pe) of its rows; without w_ukt workgroup 0 does the
// latter.  w_uv_pf != null (the spread small-batch path): the absorbing workgroups also
// bring mla_attend_kernel's W_UV rows into the L2 of the XCD that will read them.
template <bool ABSORB>
__global__ __launch_bounds__(256) void mla_prepare_kernel(const bf16_t* __restrict__ qkva, int64_t qs, int rows,
                                                          const int32_t* __restrict__ pos,
                                                          const int64_t* __restrict__ base,
                                                          const int32_t* __restrict__ cap,
                                                          const bf16_t* __restrict__ kvw, float eps,
                                                          const bf16_t* __restrict__ cosT,
                                                          const bf16_t* __restrict__ sinT, int max_pos,
                                                          const bf16_t* __restrict__ w_ukt, bf16_t* __restrict__ cache,
                                                          bf16_t* __restrict__ qout, int32_t* __restrict__ status,
                                                          const bf16_t* __restrict__ w_uv_pf) {
  constexpr int RB = ABSORB ? 8 : 1;  // RoPE/cache only: one row per workgroup
  const int tid = threadIdx.x;
  const int b0 = blockIdx.y * RB;
  const int nr = min(RB, rows - b0);
  if (ABSORB && blockIdx.x < 128) {
    const int gi = tid >> 4, k = tid & 15;
    const int row0 = blockIdx.x * 64 + gi * 4;  // 4 consecutive rows of one head
    const int h = row0 / kLat, j0 = row0 % kLat;
    uint4 wr[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) wr[q] = ldg16(w_ukt + (int64_t)(row0 + q) * 128 + k * 8);
    // Prefetch of the cached tokens of the block's first two rows for the attention launch
    // that follows (each head's workgroups re-read every cached row there): the 16
    // workgroups that share an XCD (block ids equal mod 8) each request every 16th token row
    // of the first 256, so each XCD's L2 holds them when the attention starts.  The values
    // only feed an empty asm after the absorption.
    constexpr int kPf = (16 * (kRow / 8) + 255) / 256;  // 16 rows of 72 chunks over 256 threads
    uint4 pf[2][kPf];
    const int slot = blockIdx.x >> 3;
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int b = b0 + min(rr, nr - 1);
      const int n = min(min(max(pos[b], 0), cap[b]), 256);  // rows [0, n) are already cached
      const int nt = n > slot ? (n - 1 - slot) / 16 + 1 : 0;  // tokens slot, slot + 16, ... < n
      const bf16_t* crow0 = cache + base[b] * kRow;
#pragma unroll
      for (int i = 0; i < kPf; ++i) {
        const int c = tid + 256 * i;
        const bool live = rr < nr && c < nt * (kRow / 8);
        const int t = live ? slot + 16 * (c / (kRow / 8)) : 0;
        pf[rr][i] = ldg16(crow0 + (int64_t)t * kRow + (live ? c % (kRow / 8) : 0) * 8);
      }
    }
    // W_UV: the attention workgroup bid = 4h + qq (on XCD bid % 8) reads rows h*128 + qq*32
    // .. +31; the 16 workgroups of this XCD take 16 rows each of its 8 such workgroups
    uint4 pu[4];
    if (w_uv_pf) {
      const int abid = (blockIdx.x & 7) + 8 * (slot >> 1);
      const int64_t row = (int64_t)(abid >> 2) * 128 + (abid & 3) * 32 + (slot & 1) * 16;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = tid + 256 * i;  // 16 rows x 64 chunks of 16 bytes
        pu[i] = ldg16(w_uv_pf + (row + (c >> 6)) * kLat + (c & 63) * 8);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) pu[i] = make_uint4(0u, 0u, 0u, 0u);
    }
    for (int r = 0; r < nr; ++r) {
      float qn[8];
      unpack8(ldg16(qkva + (b0 + r) * qs + h * 192 + k * 8), qn);
      float sdot[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) sdot[q] = dot8(wr[q], qn);
#pragma unroll
      for (int off = 8; off > 0; off >>= 1)
#pragma unroll
        for (int q = 0; q < 4; ++q) sdot[q] = xor_sum(sdot[q], off);
      if (k == 0) {
        uint2 o;
        o.x = pack2(sdot[0], sdot[1]);
        o.y = pack2(sdot[2], sdot[3]);
        *reinterpret_cast<uint2*>(qout + ((int64_t)(b0 + r) * kHeads + h) * kRow + j0) = o;
      }
    }
    uint32_t acc = 0;
#pragma unroll
    for (int rr = 0; rr < 2; ++rr)
#pragma unroll
      for (int i = 0; i < kPf; ++i) acc ^= pf[rr][i].x;
#pragma unroll
    for (int i = 0; i < 4; ++i) acc ^= pu[i].x;
    asm volatile("" ::"v"(acc));
    return;
  }
  const MlaRowArgs m{qkva, qs, pos, base, cap, kvw, eps, cosT, sinT, max_pos, cache, qout, status};
  for (int r = 0; r < nr; ++r) mla_prepare_row(m, b0 + r, tid);
}

// mla_prepare with absorption and the W_UV prefetch for mla_attend_kernel (dsv2_mla_spread)
void mla_prepare_absorb_launch(const void* qkva, int64_t qkva_stride, int rows, const int32_t* pos,
                              const int64_t* base, const int32_t* cap, const void* kv_norm_w, float eps,
                              const void* rope_cos, const void* rope_sin, int max_pos, const void* w_ukt,
                              const void* w_uv, void* cache, void* q_out, int32_t* status, hipStream_t stream) {
  hipLaunchKernelGGL(mla_prepare_kernel<true>, dim3(kHeads * kLat / 64 + 1, (rows + 7) / 8), dim3(256), 0, stream,
                     (const bf16_t*)qkva, qkva_stride, rows, pos, base, cap, (const bf16_t*)kv_norm_w, eps,
                     (const bf16_t*)rope_cos, (const bf16_t*)rope_sin, max_pos, (const bf16_t*)w_ukt, (bf16_t*)cache,
                     (bf16_t*)q_out, status, (const bf16_t*)w_uv);
}

extern "C" int dsv2_mla_prepare(const void* qkva, int64_t qkva_stride, int rows, const int32_t* pos,
                                const int64_t* base, const int32_t* cap, const void* kv_norm_w, float eps,
                                const void* rope_cos, const void* rope_sin, int max_pos, const void* w_ukt,
                                void* cache, void* q_out, int32_t* status, void* stream) {
  DSV2_REQUIRE(qkva && pos && base && cap && kv_norm_w && rope_cos && rope_sin && cache && q_out, DSV2_E_NULL,
               "mla_prepare: null pointer");
  DSV2_REQUIRE(rows >= 0 && rows <= 65535 && max_pos > 0 && qkva_stride >= kQkvA, DSV2_E_SHAPE,
               "mla_prepare: bad shape");
  DSV2_REQUIRE(dsv2_aligned16(qkva) && qkva_stride % 8 == 0 && dsv2_aligned16(kv_norm_w) && dsv2_aligned16(cache) &&
                   dsv2_aligned16(q_out) && (!w_ukt || dsv2_aligned16(w_ukt)),
               DSV2_E_ALIGN, "mla_prepare: alignment");
  if (rows == 0) return DSV2_OK;
  const dim3 grid(w_ukt ? kHeads * kLat / 64 + 1 : 1, w_ukt ? (rows + 7) / 8 : rows);
  if (w_ukt)
    hipLaunchKernelGGL(mla_prepare_kernel<true>, grid, dim3(256), 0, (hipStream_t)stream, (const bf16_t*)qkva,
                       qkva_stride, rows, pos, base, cap, (const bf16_t*)kv_norm_w, eps, (const bf16_t*)rope_cos,
                       (const bf16_t*)rope_sin, max_pos, (const bf16_t*)w_ukt, (bf16_t*)cache, (bf16_t*)q_out, status,
                       nullptr);
  else
    hipLaunchKernelGGL(mla_prepare_kernel<false>, grid, dim3(256), 0, (hipStream_t)stream, (const bf16_t*)qkva,
                       qkva_stride, rows, pos, base, cap, (const bf16_t*)kv_norm_w, eps, (const bf16_t*)rope_cos,
                       (const bf16_t*)rope_sin, max_pos, nullptr, (bf16_t*)cache, (bf16_t*)q_out, status,
                       nullptr);
  return dsv2_launch_status("mla_prepare");
}

// ---------------------------------------------------------------------------
// split-KV decode
// ---------------------------------------------------------------------------
// DIRECT (one split per row, split_tokens covering every row): the workgroup's softmax is
// the row's, so it writes o_lat = O / l as bf16 (out [rows, 16 * 512], row stride os) --
// the value dsv2_mla_combine computes from a single split, bit for bit -- and no partials.
template <bool DIRECT>
__global__ __launch_bounds__(256, 2) void mla_decode_kernel(const bf16_t* __restrict__ q,
                                                            const bf16_t* __restrict__ cache,
                                                            const int64_t* __restrict__ base,
                                                            const int32_t* __restrict__ pos,
                                                            const int32_t* __restrict__ cap, int split_tokens,
                                                            int max_splits, float scale_log2,
                                                            float* __restrict__ part_o, float* __restrict__ part_ml,
                                                            bf16_t* __restrict__ out, int64_t os) {
  __shared__ __attribute__((aligned(16))) bf16_t lds[2][kTile * kLdsRow];
  __shared__ floatx4_t spart[4][64];  // per-wave partial S^T (one 16-token block, half of K)
  const int s = blockIdx.x, b = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, li = lane & 15, kg = lane >> 4;
  // S^T = K Q^T is split over the waves: wave w scores 16-token block w >> 1 of every tile
  // over k steps [9*(w & 1), 9*(w & 1) + 9) of the 18; the pair's partials meet in LDS.
  // Q^T fragments (B operand) of those steps: head li, dims kk*32 + kg*8 .. +8.  They depend
  // on the row only and are requested first; the row's position, capacity and cache base
  // then come in one round trip, ahead of the split's range check.
  const int sblk = wv >> 1, k0 = (wv & 1) * 9;
  bf16x8_t qf[9];
  {
    const bf16_t* qh = q + ((int64_t)b * kHeads + li) * kRow + kg * 8 + k0 * 32;
#pragma unroll
    for (int kk = 0; kk < 9; ++kk) qf[kk] = as_bf16x8(ldg16(qh + kk * 32));
  }
  const int pb = pos[b], cb = cap[b];
  const int64_t bb = base[b];
  const int len = min(pb + 1, cb);  // never past the row's own slots
  const int t_begin = s * split_tokens;
  if (t_begin >= len) {
    if (DIRECT) {  // a row with no cached token (capacity 0): zeros, as the combine writes
#pragma unroll
      for (int j = 0; j < 4; ++j) *reinterpret_cast<uint4*>(out + b * os + tid * 32 + j * 8) = make_uint4(0, 0, 0, 0);
    }
    return;
  }
  const int t_end = min(len, t_begin + split_tokens);
  const int ntiles = (t_end - t_begin + kTile - 1) / kTile;
  const bf16_t* crow = cache + bb * kRow;

  // Two register stages: tile it + 2 is requested while tile it + 1 is still in flight
  // (cache rows are read once per step: non-temporal loads, which stream ~15% faster here).
  // Requests past the last tile repeat it (L2 hits, never stored), so every load is
  // unconditional and the waits count the newer stage's 9 loads exactly.
  uint4 stage[2][9];
  const int last = t_begin + (ntiles - 1) * kTile;
  auto load_tile = [&](int st, int t0) {
    t0 = min(t0, last);
#pragma unroll
    for (int i = 0; i < 9; ++i) {
      const int c = tid + 256 * i;
      const int tok = c / 72, off = (c % 72) * 8;
      const int tt = min(t0 + tok, t_end - 1);
      stage[st][i] = ldg16_nt(crow + (int64_t)tt * kRow + off);
    }
  };
  auto store_tile = [&](int st, int buf) {
#pragma unroll
    for (int i = 0; i < 9; ++i) {
      const int c = tid + 256 * i;
      const int tok = c / 72, off = (c % 72) * 8;
      *reinterpret_cast<uint4*>(&lds[buf][tok * kLdsRow + off]) = stage[st][i];
    }
  };

  // every workgroup walks its tiles in token order, whatever its row: the online softmax's
  // rounding depends on the order, and rows holding the same sequence must give the same
  // bits.  (Rows streamed together at one cache stride can camp on the same HBM channels;
  // CompressedKVCache staggers the rows' bases against that.)
  auto tile_t0 = [&](int it) {  // first token of tile it; past the end: the last tile
    return t_begin + min(it, ntiles - 1) * kTile;
  };
  load_tile(0, tile_t0(0));
  load_tile(1, tile_t0(1));
  store_tile(0, 0);
  __syncthreads();

  float m_run = -INFINITY, l_run = 0.f;
  floatx4_t acc[8];
#pragma unroll
  for (int mb = 0; mb < 8; ++mb) acc[mb] = floatx4_t{0.f, 0.f, 0.f, 0.f};

  // one tile: register stage u (= tile parity) and LDS buffer u
  auto tile_step = [&](const int u, const int it) {
    const int t0 = tile_t0(it);
    load_tile(u, tile_t0(it + 2));
    const bf16_t* L = lds[u];

    // S^T for two 16-token blocks: sc[blk][e] = score(token blk*16 + 4kg + e, head li)
    {
      floatx4_t sp = floatx4_t{0.f, 0.f, 0.f, 0.f};
      const bf16_t* kr = L + (sblk * 16 + li) * kLdsRow + kg * 8 + k0 * 32;
#pragma unroll
      for (int kk = 0; kk < 9; ++kk) sp = mfma16x16x32(*reinterpret_cast<const bf16x8_t*>(kr + kk * 32), qf[kk], sp);
      spart[wv][lane] = sp;
    }
    __syncthreads();
    floatx4_t sc[2];
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) sc[blk] = spart[2 * blk][lane] + spart[2 * blk + 1][lane];
    float p[8];
    float mx = -INFINITY;  // of the raw scores (scale_log2 > 0 keeps the order)
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int tok = t0 + blk * 16 + 4 * kg + e;
        const float v = tok < t_end ? sc[blk][e] : -INFINITY;
        p[blk * 4 + e] = v;
        mx = fmaxf(mx, v);
      }
    mx = xor16_max(mx);
    mx = xor32_max(mx);
    // lazy rescaling: the running maximum m (log2 units) moves, and O and l are rescaled,
    // only where the tile's maximum exceeds it by more than 8, so p = 2^(s - m) <= 256
    // (bf16 and the fp32 sums hold it) while most tiles skip the rescale; (O, l, m) stay a
    // consistent triple for the combine.  The first tile always moves m (it holds a token).
    const float tm = mx * scale_log2;
    const bool grow = tm > m_run + 8.f;
    if (__any(grow)) {
      const float m_new = grow ? tm : m_run;
      const float alpha = exp2f(m_run - m_new);  // 0 from m = -inf, 1 where m stays
      l_run *= alpha;
      m_run = m_new;
#pragma unroll
      for (int mb = 0; mb < 8; ++mb) acc[mb] *= alpha;
    }
    float rsum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      p[i] = exp2f(fmaf(p[i], scale_log2, -m_run));
      rsum += p[i];
    }
    rsum = xor16_sum(rsum);
    rsum = xor32_sum(rsum);
    l_run += rsum;

    // P^T (B operand): head li, tokens {4kg+e} then {16+4kg+e}; the V^T A operand takes the
    // same tokens of dim d0 + li through two transposed LDS reads (ds_read_b64_tr_b16): in
    // each 16-lane group, lane i receives element i % 4 of the 8 bytes that lane 4e + i / 4
    // addressed (e = 0..3), so lane (li, kg) addresses token 4kg + li/4 (then 16 + 4kg + li/4),
    // dims d0 + 4(li % 4) .. +3, and receives V[4kg + e][d0 + li] (then V[16 + 4kg + e][..]).
    const bf16x8_t pb = as_bf16x8(pack8(p));
    const bf16_t* vp = L + (4 * kg + (li >> 2)) * kLdsRow + wv * 128 + 4 * (li & 3);
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
      const uint2 lo = lds_read_tr16(vp + mb * 16), hi = lds_read_tr16(vp + mb * 16 + 16 * kLdsRow);
      acc[mb] = mfma16x16x32(as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y)), pb, acc[mb]);
    }
    if (it + 1 < ntiles) {
      // buffer u ^ 1 was last read in tile it - 1, which every wave finished before the
      // barrier that ended it; one barrier after the store publishes tile it + 1.
      store_tile(u ^ 1, u ^ 1);
      __syncthreads();
    }
  };
  // two tiles per pass, so each register stage stays in its own registers across the back edge
  for (int it = 0;; it += 2) {
    tile_step(0, it);
    if (it + 1 >= ntiles) break;
    tile_step(1, it + 1);
    if (it + 2 >= ntiles) break;
  }
  // O^T layout: lane holds head li, dims wv*128 + mb*16 + 4kg + e
  if (DIRECT) {
    const float inv = 1.0f / l_run;  // the combine's weight of a lone split: exp2(0) / l
    bf16_t* ob = out + b * os + li * kLat + wv * 128 + 4 * kg;
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
      uint2 v;
      v.x = pack2(__builtin_fmaf(inv, acc[mb][0], 0.f), __builtin_fmaf(inv, acc[mb][1], 0.f));
      v.y = pack2(__builtin_fmaf(inv, acc[mb][2], 0.f), __builtin_fmaf(inv, acc[mb][3], 0.f));
      *reinterpret_cast<uint2*>(ob + mb * 16) = v;
    }
    return;
  }
  float* po = part_o + (((int64_t)b * max_splits + s) * kHeads + li) * kLat + wv * 128 + 4 * kg;
#pragma unroll
  for (int mb = 0; mb < 8; ++mb)
    *reinterpret_cast<float4*>(po + mb * 16) = make_float4(acc[mb][0], acc[mb][1], acc[mb][2], acc[mb][3]);
  if (wv == 0 && kg == 0) {
    float* pm = part_ml + (((int64_t)b * max_splits + s) * kHeads + li) * 2;
    pm[0] = m_run;
    pm[1] = l_run;
  }
}

extern "C" int dsv2_mla_decode(const void* q, const void* cache, const int64_t* base, const int32_t* pos,
                               const int32_t* cap, int rows, int split_tokens, int max_splits, float softmax_scale,
                               float* part_o, float* part_ml, void* stream) {
  DSV2_REQUIRE(q && cache && base && pos && cap && part_o && part_ml, DSV2_E_NULL, "mla_decode: null pointer");
  DSV2_REQUIRE(rows >= 0 && rows <= 65535 && split_tokens > 0 && split_tokens % kTile == 0 && max_splits > 0 &&
                   max_splits <= 64,
               DSV2_E_SHAPE, "mla_decode: bad shape (split_tokens %% 32, 1 <= max_splits <= 64)");
  DSV2_REQUIRE(dsv2_aligned16(q) && dsv2_aligned16(cache) && dsv2_aligned16(part_o), DSV2_E_ALIGN,
               "mla_decode: alignment");
  if (rows == 0) return DSV2_OK;
  const float scale_log2 = softmax_scale * 1.4426950408889634f;
  hipLaunchKernelGGL(mla_decode_kernel<false>, dim3(max_splits, rows), dim3(256), 0, (hipStream_t)stream,
                     (const bf16_t*)q, (const bf16_t*)cache, base, pos, cap, split_tokens, max_splits, scale_log2, part_o,
                     part_ml, nullptr, 0);
  return dsv2_launch_status("mla_decode");
}

extern "C" int dsv2_mla_decode_rows(const void* q, const void* cache, const int64_t* base, const int32_t* pos,
                                    const int32_t* cap, int rows, float softmax_scale, void* olat, int64_t olat_stride,
                                    void* stream) {
  DSV2_REQUIRE(q && cache && base && pos && cap && olat, DSV2_E_NULL, "mla_decode_rows: null pointer");
  DSV2_REQUIRE(rows >= 0 && rows <= 65535, DSV2_E_SHAPE, "mla_decode_rows: bad rows");
  DSV2_REQUIRE(dsv2_aligned16(q) && dsv2_aligned16(cache) && dsv2_aligned16(olat) && olat_stride % 8 == 0 &&
                   olat_stride >= kHeads * kLat,
               DSV2_E_ALIGN, "mla_decode_rows: alignment (16-byte o_lat rows of >= 8192 elements)");
  if (rows == 0) return DSV2_OK;
  const float scale_log2 = softmax_scale * 1.4426950408889634f;
  // one split per row covering all of it (2^30 tokens would be 1.2 TB of one row's cache)
  hipLaunchKernelGGL(mla_decode_kernel<true>, dim3(1, rows), dim3(256), 0, (hipStream_t)stream, (const bf16_t*)q,
                     (const bf16_t*)cache, base, pos, cap, 1 << 30, 1, scale_log2, nullptr, nullptr, (bf16_t*)olat,
                     olat_stride);
  return dsv2_launch_status("mla_decode_rows");
}

// ---------------------------------------------------------------------------
// combine (+ W_UV)
// ---------------------------------------------------------------------------
template <bool UV>
__global__ __launch_bounds__(256) void mla_combine_kernel(const float* __restrict__ part_o,
                                                          const float* __restrict__ part_ml,
                                                          const int32_t* __restrict__ pos,
                                                          const int32_t* __restrict__ cap, int split_tokens,
                                                          int max_splits, const bf16_t* __restrict__ w_uv,
                                                          bf16_t* __restrict__ out, int64_t os) {
  __shared__ float olat[kLat];
  __shared__ float wsp[64];
  const int b = blockIdx.x, h = blockIdx.y, part = blockIdx.z, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int pb = pos[b], cb = cap[b];  // one round trip for both
  const int len = min(pb + 1, cb);     // the tokens dsv2_mla_decode attended
  const int ns = min((len + split_tokens - 1) / split_tokens, max_splits);
  // W_UV rows of this workgroup (part*32 + wv*8 .. +8) are requested before the merge
  uint4 wr[8];
  if (UV) {
    const bf16_t* wp = w_uv + ((int64_t)h * 128 + part * 32 + wv * 8) * kLat + lane * 8;
#pragma unroll
    for (int r = 0; r < 8; ++r) wr[r] = ldg16(wp + (int64_t)r * kLat);
  }
  // every split's (m, l) pair (lane = split; wave 0 merges them), then the first 8 splits'
  // partial outputs, all requested before the merge, so its wait covers the pairs only;
  // further splits come 8 loads at a time (split indices clamped into [0, ns), masked where
  // used; a row with nothing cached, ns = 0, reads its first split's slot and writes zeros)
  const float* pm = part_ml + ((int64_t)b * max_splits * kHeads + h) * 2;
  float2 ml = *reinterpret_cast<const float2*>(pm + (int64_t)max(min(lane, ns - 1), 0) * kHeads * 2);
  const float* po = part_o + ((int64_t)b * max_splits * kHeads + h) * kLat + 2 * tid;
  float2 pv[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
    pv[j] = *reinterpret_cast<const float2*>(po + (int64_t)max(min(j, ns - 1), 0) * kHeads * kLat);
  // the pair used here, in the entry block: hipcc would otherwise sink its load into wave 0's
  // branch, behind the partial-output loads
  asm volatile("" : "+v"(ml.x), "+v"(ml.y));
  if (wv == 0) {
    const float m = lane < ns ? ml.x : -INFINITY;
    const float M = wave_max(m);
    const float w = lane < ns ? exp2f(m - M) : 0.f;
    const float l = lane < ns ? ml.y : 0.f;
    const float Lsum = wave_sum(w * l);
    wsp[lane] = w / Lsum;
  }
  __syncthreads();
  float o0 = 0.f, o1 = 0.f;
  for (int s0 = 0; s0 < ns; s0 += 8) {
    if (s0 > 0) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        pv[j] = *reinterpret_cast<const float2*>(po + (int64_t)min(s0 + j, ns - 1) * kHeads * kLat);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (s0 + j < ns) {
        o0 = __builtin_fmaf(wsp[s0 + j], pv[j].x, o0);
        o1 = __builtin_fmaf(wsp[s0 + j], pv[j].y, o1);
      }
    }
  }
  if (!UV) {
    if (part == 0) *reinterpret_cast<uint32_t*>(out + b * os + h * kLat + 2 * tid) = pack2(o0, o1);
    return;
  }
  olat[2 * tid] = o0;
  olat[2 * tid + 1] = o1;
  __syncthreads();
  float xo[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) xo[e] = olat[lane * 8 + e];
  float r[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = dot8(wr[i], xo);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = xor_sum(r[i], off);
  if (lane == 0) *reinterpret_cast<uint4*>(out + b * os + h * 128 + part * 32 + wv * 8) = pack8(r);
}

extern "C" int dsv2_mla_combine(const float* part_o, const float* part_ml, const int32_t* pos, const int32_t* cap,
                                int rows, int split_tokens, int max_splits, const void* w_uv, void* out,
                                int64_t out_stride, void* stream) {
  DSV2_REQUIRE(part_o && part_ml && pos && cap && out, DSV2_E_NULL, "mla_combine: null pointer");
  DSV2_REQUIRE(rows >= 0 && rows <= 65535 && split_tokens > 0 && max_splits > 0 && max_splits <= 64, DSV2_E_SHAPE,
               "mla_combine: bad shape");
  DSV2_REQUIRE(out_stride % 8 == 0 && dsv2_aligned16(out) && (!w_uv || dsv2_aligned16(w_uv)), DSV2_E_ALIGN,
               "mla_combine: alignment");
  if (rows == 0) return DSV2_OK;
  if (w_uv)
    hipLaunchKernelGGL(mla_combine_kernel<true>, dim3(rows, kHeads, 4), dim3(256), 0, (hipStream_t)stream, part_o,
                       part_ml, pos, cap, split_tokens, max_splits, (const bf16_t*)w_uv, (bf16_t*)out, out_stride);
  else
    hipLaunchKernelGGL(mla_combine_kernel<false>, dim3(rows, kHeads), dim3(256), 0, (hipStream_t)stream, part_o,
                       part_ml, pos, cap, split_tokens, max_splits, nullptr, (bf16_t*)out, out_stride);
  return dsv2_launch_status("mla_combine");
}
