// Absorbed-MLA decode for a few rows (the small family).  Constants shared by the kernels.
#include "common.h"

namespace {
constexpr int kRow = 576, kLat = 512;
constexpr int kAbsBlocks = 8;  // q_nope rows of a head in blocks of 16: partial absorbed queries per head
}

// ---------------------------------------------------------------------------------------
// Spread absorbed-MLA attention for a few rows: per row 64 workgroups of 512 threads, one per
// (head h, quarter qq of W_UV_h's 128 output rows).  Each attends all of the row's cached
// tokens and applies its 32 W_UV rows (requested at entry); no communication between
// workgroups.  A token is spread over 16 lanes (lane li holds latent chunks li, li+16, li+32,
// li+48 of 8 elements and rope elements 4li .. 4li+3), so a wave scores 4 tokens per
// instruction: q.k by v_dot2_f32_bf16 on the packed bf16 pairs, a 16-lane DPP sum, an online
// softmax per 16-lane row, p.v by v_dot2_f32_bf16 over the row's two tokens with p rounded
// to bf16 (the reference also rounds its softmax weights to bf16 before p.v).  Each wave
// takes 8 consecutive tokens per batch (2 per row), three batches in flight.  The 32 row
// states of the workgroup merge in LDS.
//   mla_attend_kernel: after mla_prepare (absorbed, rotated q and the new cache row written).
//   mla_quad_kernel (dsv2_mla_fused): the whole MLA in one launch -- each of a head's four
//     workgroups also absorbs q_h (all 512 latent rows of W_UK_h^T, shared through its
//     XCD's L2), builds the new token's row (stored by one workgroup) and attends it from
//     LDS, so the four need nothing from each other.
namespace {
constexpr int kAttWaves = 8, kAttTB = 2;  // tokens per 16-lane row per batch (p.v pairs them)
constexpr int kAttRows = kAttWaves * 4;   // 16-lane rows per workgroup
constexpr int kAttStep = kAttWaves * 4 * kAttTB;  // tokens per workgroup per batch
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
struct __attribute__((aligned(16))) AttLds {
  float wo[kAttRows][kLat];
  bf16_t wuv[kAttRows][kLat];  // the workgroup's 32 W_UV rows (wave wv: rows 4 wv .. 4 wv + 3)
  float wm[kAttRows], wl[kAttRows];
  float olat[kLat];
};

// the rows of this lane's 16-lane row in the batch starting at token T: T + wv*8 + 4u + rg,
// clamped to n_ld - 1 (masked at use); the loads stay here, ahead of the batch consumed next
__device__ __forceinline__ void att_load(AttTok (&S)[kAttTB], const bf16_t* crow0, int T, int n_ld, int wv, int li,
                                         int rg) {
#pragma unroll
  for (int u = 0; u < kAttTB; ++u) {
    const bf16_t* rp = crow0 + (int64_t)min(T + wv * 4 * kAttTB + 4 * u + rg, n_ld - 1) * kRow;
#pragma unroll
    for (int j = 0; j < 4; ++j) S[u].c[j] = ldg16(rp + (li + 16 * j) * 8);
    S[u].r = *reinterpret_cast<const uint2*>(rp + kLat + 4 * li);
  }
  asm volatile("" ::: "memory");
}

struct AttRow {
  float m, l, o[32];
};

// score of one token against q (this lane's share, summed over the 16-lane row)
__device__ __forceinline__ float att_score(const AttTok& t, const uint4 (&qc)[4], uint2 qr) {
  float a0 = dot2bf(t.r.x, qr.x, 0.f), a1 = dot2bf(t.r.y, qr.y, 0.f);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    a0 = dot2bf(t.c[j].x, qc[j].x, a0);
    a1 = dot2bf(t.c[j].y, qc[j].y, a1);
    a0 = dot2bf(t.c[j].z, qc[j].z, a0);
    a1 = dot2bf(t.c[j].w, qc[j].w, a1);
  }
  return row16_sum(a0 + a1);
}

// online softmax over the row's two tokens of a batch (token index T + tw + 4u + rg, live
// below n)
__device__ __forceinline__ void att_consume(AttRow& R, const AttTok (&S)[kAttTB], const uint4 (&qc)[4], uint2 qr,
                                            int tok0, int n, float scale_log2) {
  float sc[kAttTB];
  float mx = R.m;
#pragma unroll
  for (int u = 0; u < kAttTB; ++u) {
    const float sv = att_score(S[u], qc, qr);
    sc[u] = (tok0 + 4 * u < n) ? sv * scale_log2 : -INFINITY;
    mx = fmaxf(mx, sc[u]);
  }
  const bool live = mx != -INFINITY;  // a row past n has seen no token yet
  const float alpha = live ? exp2f(R.m - mx) : 1.f;
  R.m = mx;
  R.l *= alpha;
#pragma unroll
  for (int i = 0; i < 32; ++i) R.o[i] *= alpha;
  // p.v over the two tokens by v_dot2_f32_bf16: p rounded to bf16 (l summed over the rounded
  // values), each value pair gathered by v_perm_b32
  const uint32_t pp = live ? pack2(exp2f(sc[0] - R.m), exp2f(sc[1] - R.m)) : 0u;
  R.l += __uint_as_float(pp << 16) + __uint_as_float(pp & 0xffff0000u);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t a4[4] = {S[0].c[j].x, S[0].c[j].y, S[0].c[j].z, S[0].c[j].w};
    const uint32_t b4[4] = {S[1].c[j].x, S[1].c[j].y, S[1].c[j].z, S[1].c[j].w};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      R.o[8 * j + 2 * w] = dot2bf(__builtin_amdgcn_perm(b4[w], a4[w], 0x05040100u), pp, R.o[8 * j + 2 * w]);
      R.o[8 * j + 2 * w + 1] = dot2bf(__builtin_amdgcn_perm(b4[w], a4[w], 0x07060302u), pp, R.o[8 * j + 2 * w + 1]);
    }
  }
}

// The attention of one (row, head, W_UV quarter): cached rows [0, n) of crow0 (first three
// batches already requested into ta / tb / tc), plus -- when xt != null, in the workgroup's
// 16-lane row 0 -- one more token whose bf16 row xt[576] is in LDS; the 32 row states merged
// in LDS, then y = W_UV rows (wave wv's 4 rows in sh.wuv, stored by att_stash_wuv) . o_lat,
// stored as bf16 at outp[wv*4 .. +3].
__device__ __forceinline__ void att_finish(AttTok (&ta)[kAttTB], AttTok (&tb)[kAttTB], AttTok (&tc)[kAttTB],
                                           const bf16_t* crow0, int n, int n_ld, const uint4 (&qc)[4], uint2 qr,
                                           const bf16_t* xt, float scale_log2, AttLds& sh,
                                           bf16_t* outp) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, li = lane & 15, rg = lane >> 4;
  const int tw = wv * 4 * kAttTB;
  AttRow R;
  R.m = -INFINITY;
  R.l = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) R.o[i] = 0.f;
  // a ring of three batches (192 tokens requested at entry: the bsz=1 contexts of a few
  // hundred tokens wait for one load round trip, not one per batch pair).  Each pass but the
  // last consumes its three batches and refills each slot unconditionally (past the end the
  // rows are clamped and masked), so the same loads are pending at every loop entry and each
  // wait is for one batch; the last pass -- its batches already in flight -- loads nothing
  if (n > 0)
    for (int t0 = 0;; t0 += 3 * kAttStep) {
      if (t0 + 3 * kAttStep >= n) {
        att_consume(R, ta, qc, qr, t0 + tw + rg, n, scale_log2);
        if (t0 + kAttStep < n) att_consume(R, tb, qc, qr, t0 + kAttStep + tw + rg, n, scale_log2);
        if (t0 + 2 * kAttStep < n) att_consume(R, tc, qc, qr, t0 + 2 * kAttStep + tw + rg, n, scale_log2);
        break;
      }
      att_consume(R, ta, qc, qr, t0 + tw + rg, n, scale_log2);
      att_load(ta, crow0, t0 + 3 * kAttStep, n_ld, wv, li, rg);
      att_consume(R, tb, qc, qr, t0 + kAttStep + tw + rg, n, scale_log2);
      att_load(tb, crow0, t0 + 4 * kAttStep, n_ld, wv, li, rg);
      att_consume(R, tc, qc, qr, t0 + 2 * kAttStep + tw + rg, n, scale_log2);
      att_load(tc, crow0, t0 + 5 * kAttStep, n_ld, wv, li, rg);
    }
  if (xt && wv == 0 && rg == 0) {  // the extra token, in row 0
    AttTok t;
#pragma unroll
    for (int j = 0; j < 4; ++j) t.c[j] = *reinterpret_cast<const uint4*>(xt + (li + 16 * j) * 8);
    t.r = *reinterpret_cast<const uint2*>(xt + kLat + 4 * li);
    const float sv = att_score(t, qc, qr) * scale_log2;
    const float mx = fmaxf(R.m, sv);
    const float alpha = exp2f(R.m - mx);
    const float pu = rbf(exp2f(sv - mx));
    R.m = mx;
    R.l = R.l * alpha + pu;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float f[8];
      unpack8(t.c[j], f);
#pragma unroll
      for (int i = 0; i < 8; ++i) R.o[8 * j + i] = __builtin_fmaf(pu, f[i], R.o[8 * j + i] * alpha);
    }
  }
  const int row = wv * 4 + rg;
  if (li == 0) {
    sh.wm[row] = R.m;
    sh.wl[row] = R.l;
  }
  // the row state as 16-byte LDS writes: lane li's 8 latent elements (li + 16j) * 8 .. + 7 are
  // one 32-byte chunk, and lanes li with bit 2 set write its second half first, so the 8 lanes
  // a write serves at once cover all 32 banks (element-wise writes put the 64 lanes of a wave
  // on 4 banks: 1.8 us of the workgroup's 8 us at bsz=1, MI355X)
  const int hs = (li >> 2) & 1;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int hh = k ^ hs;
      floatx4_t v;
      v[0] = hh ? R.o[8 * j + 4] : R.o[8 * j];
      v[1] = hh ? R.o[8 * j + 5] : R.o[8 * j + 1];
      v[2] = hh ? R.o[8 * j + 6] : R.o[8 * j + 2];
      v[3] = hh ? R.o[8 * j + 7] : R.o[8 * j + 3];
      *reinterpret_cast<floatx4_t*>(&sh.wo[row][(li + 16 * j) * 8 + 4 * hh]) = v;
    }
  __syncthreads();
  // merge the rows: wave 0 turns the 32 row maxima into weights 2^(m_w - M) / L once (a row
  // that saw no token carries m = -inf: weight 0; row 0 always sees a token -- token 0, or
  // the extra one -- so M is finite), then every thread sums its latent element
  if (wv == 0) {
    const float mw = lane < kAttRows ? sh.wm[lane] : -INFINITY;
    float M = mw;
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) M = xor_max(M, off);
    const float sw = exp2f(mw - M);
    float L = lane < kAttRows ? sh.wl[lane] * sw : 0.f;
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) L = xor_sum(L, off);
    if (lane < kAttRows) sh.wm[lane] = sw / L;
  }
  __syncthreads();
  {
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < kAttRows; ++w) acc = __builtin_fmaf(sh.wo[w][tid], sh.wm[w], acc);
    sh.olat[tid] = acc;
  }
  __syncthreads();
  float xo[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) xo[i] = sh.olat[lane * 8 + i];
  float yr[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const u32x4_t w4 = *reinterpret_cast<const u32x4_t*>(&sh.wuv[wv * 4 + r][lane * 8]);
    yr[r] = wave_sum_dpp(dot8(make_uint4(w4[0], w4[1], w4[2], w4[3]), xo));
  }
  if (lane == 0) {
    uint2 w;
    w.x = pack2(yr[0], yr[1]);
    w.y = pack2(yr[2], yr[3]);
    *reinterpret_cast<uint2*>(outp + wv * 4) = w;
  }
}

// wave wv's 4 of the workgroup's 32 W_UV rows (h's output rows qq*32 + wv*4 ..), this lane's
// 16 bytes of each, requested at entry and parked in LDS (att_stash_wuv) before the attention
// so that no registers are held across it
__device__ __forceinline__ void att_load_wuv(uint4 (&wuv)[4], const bf16_t* w_uv, int h, int qq, int wv, int lane) {
  const bf16_t* wp = w_uv + ((int64_t)h * 128 + qq * 32 + wv * 4) * kLat + lane * 8;
#pragma unroll
  for (int r = 0; r < 4; ++r) wuv[r] = ldg16(wp + (int64_t)r * kLat);
}
__device__ __forceinline__ void att_stash_wuv(AttLds& sh, const uint4 (&wuv)[4], int wv, int lane) {
#pragma unroll
  for (int r = 0; r < 4; ++r)
    *reinterpret_cast<u32x4_t*>(&sh.wuv[wv * 4 + r][lane * 8]) = u32x4_t{wuv[r].x, wuv[r].y, wuv[r].z, wuv[r].w};
}
}  // namespace

__global__ __launch_bounds__(512) void mla_attend_kernel(const bf16_t* __restrict__ q,
                                                         const bf16_t* __restrict__ cache,
                                                         const int64_t* __restrict__ base,
                                                         const int32_t* __restrict__ pos,
                                                         const int32_t* __restrict__ cap,
                                                         const bf16_t* __restrict__ w_uv, float scale_log2,
                                                         bf16_t* __restrict__ out, int64_t os) {
  __shared__ AttLds sh;
  const int b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int li = lane & 15, rg = lane >> 4;
  const int h = blockIdx.x >> 2, qq = blockIdx.x & 3;
  // tokens attended: the cached rows [0, n) including the new one (n = pos + 1 at most cap)
  const int pr = pos[b], cp = cap[b];
  const int n = max(1, pr < 0 ? 1 : min(pr + 1, cp));
  const bf16_t* crow0 = cache + base[b] * kRow;
  const bf16_t* qh = q + ((int64_t)b * 16 + h) * kRow;
  uint4 qc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) qc[j] = ldg16(qh + (li + 16 * j) * 8);
  const uint2 qr = *reinterpret_cast<const uint2*>(qh + kLat + 4 * li);
  uint4 wuv[4];
  att_load_wuv(wuv, w_uv, h, qq, wv, lane);
  AttTok ta[kAttTB], tb[kAttTB], tc[kAttTB];
  att_load(ta, crow0, 0, n, wv, li, rg);
  att_load(tb, crow0, kAttStep, n, wv, li, rg);
  att_load(tc, crow0, 2 * kAttStep, n, wv, li, rg);
  att_stash_wuv(sh, wuv, wv, lane);
  att_finish(ta, tb, tc, crow0, n, n, qc, qr, nullptr, scale_log2, sh,
             out + (int64_t)b * os + h * 128 + qq * 32);
}

// PARTS: q_lat is the sum of qkva_absorb_kernel's 8 fp32 partial products per head
// (qlat_part[row][h][i][512]) instead of each workgroup absorbing q_h itself.
template <bool PARTS>
__global__ __launch_bounds__(512) void mla_quad_kernel(const bf16_t* __restrict__ qkva, int64_t qs,
                                                       const int32_t* __restrict__ pos,
                                                       const int64_t* __restrict__ base,
                                                       const int32_t* __restrict__ cap,
                                                       const bf16_t* __restrict__ kvw, float eps,
                                                       const bf16_t* __restrict__ cosT,
                                                       const bf16_t* __restrict__ sinT, int max_pos,
                                                       const bf16_t* __restrict__ w_ukt,
                                                       const float* __restrict__ qlat_part,
                                                       const bf16_t* __restrict__ w_uv, bf16_t* __restrict__ cache,
                                                       float scale_log2, bf16_t* __restrict__ out, int64_t os,
                                                       int32_t* __restrict__ status) {
  __shared__ AttLds sh;
  __shared__ __attribute__((aligned(16))) bf16_t qv[kRow];    // q_lat (bf16) | rotated q_pe
  __shared__ __attribute__((aligned(16))) bf16_t nrow[kRow];  // the new token's cache row
  const int b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int li = lane & 15, rg = lane >> 4;
  // a head's four workgroups sit on one XCD (block ids equal mod 8): its W_UK^T rows are
  // read from HBM once per XCD
  const int bid = blockIdx.x;
  const int h = (bid & 7) + 8 * (bid >> 5), qq = (bid >> 3) & 3;
  const bf16_t* q = qkva + b * qs;
  // the new token goes to slot pos; the row owns slots [0, cap): a position at or past cap
  // attends the cap cached rows plus the new one, is not stored, and sets
  // DSV2_DEVERR_CACHE_FULL
  const int pr = pos[b], cp = cap[b];
  const bool fits = pr >= 0 && pr < cp;
  const int p = pr < 0 ? 0 : (pr > cp ? cp : pr);  // cached rows read: [0, p)
  const int pc = p >= max_pos ? max_pos - 1 : p;
  const bf16_t* crow0 = cache + base[b] * kRow;

  // ---- entry loads: W_UK^T_h, q_nope_h, the W_UV rows, the new row's inputs, 3 batches ----
  // absorption: thread (gi = tid / 16, k = tid % 16) owns latent rows gi + 32u, K slice k
  const int gi = tid >> 4, k = tid & 15;
  uint4 qn4 = {0u, 0u, 0u, 0u};
  uint4 wk[16];
  float qp[kAbsBlocks];
  if (PARTS) {
    // thread tid sums latent element tid of the head's partial products
    const float* pp = qlat_part + ((int64_t)b * 16 + h) * kAbsBlocks * kLat + tid;
#pragma unroll
    for (int i = 0; i < kAbsBlocks; ++i) qp[i] = pp[i * kLat];
  } else {
    qn4 = ldg16(q + h * 192 + k * 8);
    const bf16_t* wp = w_ukt + ((int64_t)h * kLat + gi) * 128 + k * 8;
#pragma unroll
    for (int u = 0; u < 16; ++u) wk[u] = ldg16(wp + (int64_t)u * 32 * 128);
  }
  uint4 wuv[4];
  att_load_wuv(wuv, w_uv, h, qq, wv, lane);
  // the new row's inputs (used by waves 0 and 1), requested by every wave without a branch and
  // turned into floats only after the token batches are requested: unpacked inside a branch
  // they made waves 0 and 1 wait for every load so far first (one more load round trip)
  const uint4 kv4 = ldg16(q + 3072 + lane * 8);
  const uint4 kw4 = ldg16(kvw + lane * 8);
  uint32_t rr[6];  // RoPE pair (k_pe: wave 0, q_pe: the other waves), cos pair, sin pair
  {
    const int l32 = lane & 31;
    const bf16_t* rp = wv == 0 ? q + 3584 : q + h * 192 + 128;
    rr[0] = rp[2 * l32];
    rr[1] = rp[2 * l32 + 1];
    rr[2] = cosT[(int64_t)pc * 64 + l32];
    rr[3] = cosT[(int64_t)pc * 64 + 32 + l32];
    rr[4] = sinT[(int64_t)pc * 64 + l32];
    rr[5] = sinT[(int64_t)pc * 64 + 32 + l32];
  }
  const int n_ld = max(p, 1);
  AttTok ta[kAttTB], tb[kAttTB], tc[kAttTB];
  att_load(ta, crow0, 0, n_ld, wv, li, rg);
  att_load(tb, crow0, kAttStep, n_ld, wv, li, rg);
  att_load(tc, crow0, 2 * kAttStep, n_ld, wv, li, rg);
  float rf[6];
#pragma unroll
  for (int i = 0; i < 6; ++i) {
    uint32_t u = rr[i];
    asm volatile("" : "+v"(u));
    rf[i] = __uint_as_float(u << 16);
  }
  const float re = rf[0], ro = rf[1], c0 = rf[2], c1 = rf[3], s0 = rf[4], s1 = rf[5];

  // ---- absorption: q_lat[c] = bf16(W_UK^T_h[c, :] . q_nope_h) ------------------------------
  if (PARTS) {
    qv[tid] = f2bf(((qp[0] + qp[1]) + (qp[2] + qp[3])) + ((qp[4] + qp[5]) + (qp[6] + qp[7])));
  } else {
    float qn[8];
    unpack8(qn4, qn);
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const float v = row16_sum(dot8(wk[u], qn));
      if (k == 0) qv[gi + 32 * u] = f2bf(v);
    }
  }
  // ---- the new row (wave 0) and RoPE(q_pe) (wave 1) ---------------------------------------
  if (wv == 0) {
    float f[8], g[8];
    unpack8(kv4, f);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(f[i], f[i], ss);
    ss = wave_sum_dpp(ss);
    const float rs = rsqrtf(ss / static_cast<float>(kLat) + eps);
    unpack8(kw4, g);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = g[i] * rbf(f[i] * rs);
    const uint4 c8 = pack8(f);
    *reinterpret_cast<uint4*>(nrow + lane * 8) = c8;
    const bool store = h == 0 && qq == 0 && fits;
    if (h == 0 && qq == 0 && !fits && lane == 0 && status) atomicOr(status, DSV2_DEVERR_CACHE_FULL);
    bf16_t* crow = cache + (base[b] + p) * kRow;
    if (store) *reinterpret_cast<uint4*>(crow + lane * 8) = c8;
    if (lane < 32) {
      const bf16_t v0 = f2bf(re * c0 - ro * s0), v1 = f2bf(ro * c1 + re * s1);
      nrow[kLat + lane] = v0;
      nrow[kLat + 32 + lane] = v1;
      if (store) {
        crow[kLat + lane] = v0;
        crow[kLat + 32 + lane] = v1;
      }
    }
  } else if (wv == 1 && lane < 32) {
    qv[kLat + lane] = f2bf(re * c0 - ro * s0);
    qv[kLat + 32 + lane] = f2bf(ro * c1 + re * s1);
  }
  att_stash_wuv(sh, wuv, wv, lane);
  __syncthreads();
  uint4 qc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) qc[j] = *reinterpret_cast<const uint4*>(qv + (li + 16 * j) * 8);
  const uint2 qr = *reinterpret_cast<const uint2*>(qv + kLat + 4 * li);
  att_finish(ta, tb, tc, crow0, p, n_ld, qc, qr, nrow, scale_log2, sh,
             out + (int64_t)b * os + h * 128 + qq * 32);
}

// ---------------------------------------------------------------------------------------
// The q | kv_a projection of one row (RMSNorm prologue) with the W_UK absorption of q_nope
// spread over the projection's own workgroups, so the small-batch MLA needs no prepare
// launch.  Workgroup w (512 threads, row blockIdx.y) owns projection rows 16w .. 16w+15,
// wave v rows 16w + 2v, +1; each lane streams 4 chunks of 8 elements of each of its rows
// (non-temporal) against x' in LDS, as gemv_k2048_kernel does (8 waves of 2 rows: 6.2 us per
// launch on MI355X against 7.0 us for 4 waves of 4).  The 12 workgroups of head h
// (w = 12h + i) hold its 192 q rows: i < 8 are the q_nope rows 16i .. 16i+15, whose bf16
// outputs q_d each workgroup multiplies into its 16 rows of W_UK_h (each lane 8 latent
// elements of the wave's 2 rows, requested at entry) -- partial[c] = sum_d W_UK_h[d, c] q_d
// over the 16 rows (fp32, fixed order), written to qlat_part[row][h][i][512].  The last 36
// workgroups hold the latent and k_pe rows.  Every workgroup also pulls an even share of the
// row's first 256 cached tokens into its XCD's L2 for the attention launch that follows
// (without it the C1 step is 1% slower).
namespace {
constexpr int kQkvRows = 3648, kQWgs = 16 * 12, kQkvWgs = kQkvRows / 16;
}

__global__ __launch_bounds__(512) void qkva_absorb_kernel(const bf16_t* __restrict__ x, int64_t xs,
                                                          const bf16_t* __restrict__ nw, float eps,
                                                          const bf16_t* __restrict__ W,
                                                          const bf16_t* __restrict__ w_uk, bf16_t* __restrict__ qkva,
                                                          int64_t qs, float* __restrict__ qlat_part,
                                                          const bf16_t* __restrict__ cache,
                                                          const int64_t* __restrict__ base,
                                                          const int32_t* __restrict__ pos,
                                                          const int32_t* __restrict__ cap) {
  __shared__ float xl[2048];
  __shared__ float red[8];
  __shared__ float pw[8][kLat];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int b = blockIdx.y, w = blockIdx.x;
  const int n0 = 16 * w + 2 * wv;
  const int h = w / 12, blk = w % 12;
  const bool absorb = w < kQWgs && blk < kAbsBlocks;  // uniform over the workgroup
  const bf16_t* xr = x + b * xs;
  // the row's position, capacity and cache base (for the prefetch below), in one round trip
  const int pb = pos[b], cb = cap[b];
  const int64_t bb = base[b];
  // entry loads, in the order they are consumed: x and the norm weights (waves 4..7 repeat
  // waves 0..3's chunks), W_UK (absorbing workgroups; the others re-read head 0's first rows,
  // an L2 hit), then the weight rows
  const int tc = tid & 255;
  const uint4 xv4 = ldg16(xr + tc * 8);
  const uint4 g4 = ldg16((nw ? nw : xr) + tc * 8);  // no norm: a harmless read of x
  uint4 wk[2];
  {
    const bf16_t* wp = w_uk + ((int64_t)(absorb ? h : 0) * 128 + (absorb ? 16 * blk + 2 * wv : 0)) * kLat + lane * 8;
#pragma unroll
    for (int j = 0; j < 2; ++j) wk[j] = ldg16(wp + (int64_t)j * kLat);
  }
  uint4 wr[2][4];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int u = 0; u < 4; ++u) wr[r][u] = ldg16_nt(W + (int64_t)(n0 + r) * 2048 + (lane + 64 * u) * 8);
  // the prefetch share: tokens slot, slot + S, ... of the first min(n, 256) (workgroups w
  // with equal w % 8 share an XCD; S of them per XCD)
  constexpr int kSlots = (kQkvWgs + 7) / 8;
  constexpr int kPfRows = (256 + kSlots - 1) / kSlots;
  constexpr int kPf = (kPfRows * (kRow / 8) + 511) / 512;
  uint4 pf[kPf];
  {
    const int slot = w >> 3;
    const int n = min(min(max(pb, 0), cb), 256);
    const int nt = n > slot ? (n - 1 - slot) / kSlots + 1 : 0;
    const bf16_t* crow0 = cache + bb * kRow;
#pragma unroll
    for (int i = 0; i < kPf; ++i) {
      const int c = tid + 512 * i;
      const bool live = c < nt * (kRow / 8);
      const int t = live ? slot + kSlots * (c / (kRow / 8)) : 0;
      pf[i] = ldg16(crow0 + (int64_t)t * kRow + (live ? c % (kRow / 8) : 0) * 8);
    }
  }
  pin(xv4.x);
  pin(g4.x);
  // x' = w * bf16(x * rsqrt(mean x^2 + eps)) (nw == null: x' = x) -> LDS (fp32)
  {
    float f[8], g8[8];
    unpack8(xv4, f);
    if (nw) {  // uniform
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(f[i], f[i], ss);
      ss = wave_sum(ss);
      if (lane == 0) red[wv] = ss;
      __syncthreads();
      const float rn = rsqrtf((red[0] + red[1] + red[2] + red[3]) / 2048.f + eps);  // waves 0..3: all of x
      unpack8(g4, g8);
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] = rbf(g8[i] * rbf(f[i] * rn));
    }
    if (tid < 256) {
#pragma unroll
      for (int i = 0; i < 8; ++i) xl[tid * 8 + i] = f[i];
    }
    __syncthreads();
  }
  float acc[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    acc[r] = 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[r] += dot8(wr[r][u], &xl[(lane + 64 * u) * 8]);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
#pragma unroll
    for (int r = 0; r < 2; ++r) acc[r] = xor_sum(acc[r], off);
  float qd[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) qd[r] = rbf(acc[r]);
  if (lane == 0) {
    *reinterpret_cast<uint32_t*>(qkva + b * qs + n0) = pack2(qd[0], qd[1]);
  }
  if (absorb) {
    float f[8], p[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) p[e] = 0.f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      unpack8(wk[j], f);
#pragma unroll
      for (int e = 0; e < 8; ++e) p[e] = __builtin_fmaf(f[e], qd[j], p[e]);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) pw[wv][lane * 8 + e] = p[e];
    __syncthreads();
    const int c = tid;
    float s0 = pw[0][c];
#pragma unroll
    for (int v = 1; v < 8; ++v) s0 += pw[v][c];
    qlat_part[(((int64_t)b * 16 + h) * kAbsBlocks + blk) * kLat + c] = s0;
  }
  uint32_t sink = 0;
#pragma unroll
  for (int i = 0; i < kPf; ++i) sink ^= pf[i].x;
  asm volatile("" ::"v"(sink));
}

extern "C" int dsv2_qkva_absorb_bf16(const void* x, int64_t x_stride, int rows, const void* w_qkva, const void* norm_w,
                                     float eps, const void* w_uk, void* qkva, int64_t qkva_stride, float* qlat_part,
                                     const void* cache, const int64_t* base, const int32_t* pos, const int32_t* cap,
                                     void* stream) {
  DSV2_REQUIRE(x && w_qkva && w_uk && qkva && qlat_part && cache && base && pos && cap, DSV2_E_NULL,
               "qkva_absorb: null pointer");
  DSV2_REQUIRE(rows >= 0 && rows <= 65535 && x_stride >= 2048 && qkva_stride >= kQkvRows, DSV2_E_SHAPE,
               "qkva_absorb: bad shape");
  DSV2_REQUIRE(dsv2_aligned16(x) && x_stride % 8 == 0 && dsv2_aligned16(w_qkva) && (!norm_w || dsv2_aligned16(norm_w)) &&
                   dsv2_aligned16(w_uk) && dsv2_aligned16(cache) && dsv2_aligned16(qkva) && qkva_stride % 8 == 0 &&
                   dsv2_aligned16(qlat_part),
               DSV2_E_ALIGN, "qkva_absorb: alignment");
  if (rows == 0) return DSV2_OK;
  hipLaunchKernelGGL(qkva_absorb_kernel, dim3(kQkvWgs, rows), dim3(512), 0, (hipStream_t)stream, (const bf16_t*)x,
                     x_stride, (const bf16_t*)norm_w, eps, (const bf16_t*)w_qkva, (const bf16_t*)w_uk, (bf16_t*)qkva,
                     qkva_stride, qlat_part, (const bf16_t*)cache, base, pos, cap);
  return dsv2_launch_status("qkva_absorb");
}

extern "C" int dsv2_mla_attend_parts(const void* qkva, int64_t qkva_stride, int rows, const int32_t* pos,
                                     const int64_t* base, const int32_t* cap, const void* kv_norm_w, float eps,
                                     const void* rope_cos, const void* rope_sin, int max_pos, const float* qlat_part,
                                     const void* w_uv, void* cache, float softmax_scale, void* out,
                                     int64_t out_stride, int32_t* status, void* stream) {
  DSV2_REQUIRE(qkva && pos && base && cap && kv_norm_w && rope_cos && rope_sin && qlat_part && w_uv && cache && out,
               DSV2_E_NULL, "mla_attend_parts: null pointer");
  DSV2_REQUIRE(rows >= 0 && rows <= 65535 && max_pos > 0 && qkva_stride >= kQkvRows && out_stride >= 2048,
               DSV2_E_SHAPE, "mla_attend_parts: bad shape");
  DSV2_REQUIRE(dsv2_aligned16(qkva) && qkva_stride % 8 == 0 && dsv2_aligned16(kv_norm_w) && dsv2_aligned16(cache) &&
                   dsv2_aligned16(qlat_part) && dsv2_aligned16(w_uv) && dsv2_aligned16(out) && out_stride % 8 == 0,
               DSV2_E_ALIGN, "mla_attend_parts: alignment");
  if (rows == 0) return DSV2_OK;
  hipLaunchKernelGGL(mla_quad_kernel<true>, dim3(64, rows), dim3(512), 0, (hipStream_t)stream, (const bf16_t*)qkva,
                     qkva_stride, pos, base, cap, (const bf16_t*)kv_norm_w, eps, (const bf16_t*)rope_cos,
                     (const bf16_t*)rope_sin, max_pos, nullptr, qlat_part, (const bf16_t*)w_uv, (bf16_t*)cache,
                     softmax_scale * 1.4426950408889634f, (bf16_t*)out, out_stride, status);
  return dsv2_launch_status("mla_attend_parts");
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

extern "C" int dsv2_mla_fused(const void* qkva, int64_t qkva_stride, int rows, const int32_t* pos, const int64_t* base,
                             const int32_t* cap, const void* kv_norm_w, float eps, const void* rope_cos,
                             const void* rope_sin, int max_pos, const void* w_ukt, const void* w_uv, void* cache,
                             float softmax_scale, void* out, int64_t out_stride, int32_t* status, void* stream) {
  DSV2_REQUIRE(qkva && pos && base && cap && kv_norm_w && rope_cos && rope_sin && w_ukt && w_uv && cache && out,
               DSV2_E_NULL, "mla_fused: null pointer");
  DSV2_REQUIRE(rows >= 0 && rows <= 65535 && max_pos > 0 && qkva_stride >= 3648 && out_stride >= 2048, DSV2_E_SHAPE,
               "mla_fused: bad shape");
  DSV2_REQUIRE(dsv2_aligned16(qkva) && qkva_stride % 8 == 0 && dsv2_aligned16(kv_norm_w) && dsv2_aligned16(cache) &&
                   dsv2_aligned16(w_ukt) && dsv2_aligned16(w_uv) && dsv2_aligned16(out) && out_stride % 8 == 0,
               DSV2_E_ALIGN, "mla_fused: alignment");
  if (rows == 0) return DSV2_OK;
  hipLaunchKernelGGL(mla_quad_kernel<false>, dim3(64, rows), dim3(512), 0, (hipStream_t)stream, (const bf16_t*)qkva,
                     qkva_stride, pos, base, cap, (const bf16_t*)kv_norm_w, eps, (const bf16_t*)rope_cos,
                     (const bf16_t*)rope_sin, max_pos, (const bf16_t*)w_ukt, nullptr, (const bf16_t*)w_uv,
                     (bf16_t*)cache, softmax_scale * 1.4426950408889634f, (bf16_t*)out, out_stride, status);
  return dsv2_launch_status("mla_fused");
}

