// Prefill attention of DeepSeek-V2's MLA in its expanded form (the prompt's attention, run
// before the q_len = 1 decode path): per head h, softmax(scale * q . k) v over the causal
// prefix, with
//   q = [q_nope (128, from the qkv_a output) | RoPE(q_pe) (64, from mla_prepare)]
//   k = [k_nope = W_UK_h c (128, expanded) | RoPE(k_pe) (64, the cache row's tail)]
//   v = W_UV_h c (128, expanded)
// where c is the kv-normalised latent of the compressed cache.  The expanded form needs
// 320 multiply-adds per (query, key, head) against 1088 for the absorbed (latent) form the
// decode step uses, which pays off when every cached token is attended by many queries.
//
// One 256-thread workgroup per (tile of <= 128 consecutive query tokens of one sequence,
// head); wave w owns queries 32w .. 32w + 31 of the tile, two 16-query blocks that share
// every K and V^T fragment the wave reads from LDS.  Keys go in 32-token tiles,
// double-buffered in LDS (the next tile's 16-byte chunks in registers meanwhile):
//   S^T = K Q^T   two 16-key blocks x 6 k-steps of v_mfma_f32_16x16x32_bf16 (queries = N)
//   online softmax per query (column), fp32, the causal mask key <= query position on the
//                   tiles that cross the diagonal, lazy rescaling of O and l
//   O^T += V^T P^T  8 x 16 value dims; V^T fragments by transposed LDS reads
//                   (ds_read_b64_tr_b16), P^T packed to bf16 in the order the reads give.
#include "common.h"

namespace {
constexpr int kKT = 32;   // keys per tile
constexpr int kQK = 192;  // q.k dims: 128 nope + 64 rope
constexpr int kVD = 128;  // value dims
constexpr int kHeads = 16;
constexpr int kCacheRow = 576;
constexpr int kKC = kQK / 8, kVC = kVD / 8;      // 16-byte chunks per key: K 16 nope + 8 rope, V 16
constexpr int kStageK = kKT * kKC * 16;          // a stage: the tile's K rows (384 B each), then
constexpr int kStage = kStageK + kKT * kVC * 16;  // its V rows (256 B each): 20 KB
constexpr int kStages = 3;
constexpr int kLoads = kKT * (kKC + kVC) / 256;  // 16-byte ring loads per thread per tile: 5
// chunk c of key row r sits in slot swz(c, r) (an involution within each aligned group of 8
// chunks): the 16 rows one K fragment reads, and the 4 rows of a transposed V read, fall in
// different banks
__device__ __forceinline__ int swz(int c, int r) { return (c & ~7) | ((c ^ r) & 7); }
constexpr int kQB = 2;                             // 16-query blocks per wave
constexpr int kQT = 4 * 16 * kQB;                  // queries per workgroup tile
}  // namespace

__global__ __launch_bounds__(256, 2) void mla_prefill_kernel(
    const bf16_t* __restrict__ qkva, int64_t qs, const bf16_t* __restrict__ qrope, int64_t qrs,
    const bf16_t* __restrict__ cache, int64_t cache_rows, const bf16_t* __restrict__ knope,
    const bf16_t* __restrict__ vexp, int64_t exp_lo, int64_t exp_rows, int rows, const int4* __restrict__ tiles,
    float scale_log2, bf16_t* __restrict__ out, int64_t os) {
  __shared__ __attribute__((aligned(16))) uint8_t ring[kStages * kStage];
  // 1-D grid over (head, tile) items cut into 8 contiguous ranges, one per XCD (workgroup i
  // runs on XCD i % 8): the query tiles of one (sequence, head) run on one XCD at about the
  // same time and sweep the same keys from key 0, so each key tile comes from HBM once per
  // XCD and from that XCD's L2 for the rest; tiles are taken last first (a sequence's last
  // tiles attend the most keys), which shortens the launch's tail
  const int n_tiles = gridDim.x / kHeads;
  const int item = (blockIdx.x % 8) * (gridDim.x / 8) + blockIdx.x / 8;
  const int h = item / n_tiles;
  const int4 tl = tiles[n_tiles - 1 - item % n_tiles];
  // every index derived from the tile table is clamped into the buffers the host described
  // (a malformed table gives wrong numbers, never an access outside them)
  const int r0 = min(max(tl.x, 0), rows - 1), nr = min(max(tl.y, 1), min(kQT, rows - r0)), p0 = max(tl.z, 0);
  const int64_t sb = tl.w;  // cache row of position 0 of the tile's sequence
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, li = lane & 15, kg = lane >> 4;
  int jq[kQB], qp[kQB];
  bf16x8_t qf[kQB][6];
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    jq[qb] = wv * 16 * kQB + 16 * qb + li;  // this lane's query (column) of block qb in the tile
    const int r = r0 + min(jq[qb], nr - 1);  // its row (queries past the tile repeat the last one)
    qp[qb] = p0 + jq[qb];                    // its position
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      qf[qb][kk] = as_bf16x8(ldg16(qkva + (int64_t)r * qs + h * 192 + kk * 32 + kg * 8));
#pragma unroll
    for (int kk = 4; kk < 6; ++kk)
      qf[qb][kk] = as_bf16x8(ldg16(qrope + (int64_t)r * qrs + h * kCacheRow + 512 + (kk - 4) * 32 + kg * 8));
  }
  const int nkv = p0 + nr;  // keys [0, nkv) of the sequence
  const int ntiles = (nkv + kKT - 1) / kKT;

  // K/V tiles stream straight into a 3-stage LDS ring (global_load_lds, 16 B per lane): ring
  // load i of wave wv fills slots 64 (4i + wv) .. + 63 of a stage, slot s holding K chunk
  // slot s % 24 of key s / 24 (s < 768), else V chunk slot (s - 768) % 16 of key
  // (s - 768) / 16; each lane fetches the chunk that belongs in its slot
  int lkey[kLoads], lchunk[kLoads];
#pragma unroll
  for (int i = 0; i < kLoads; ++i) {
    const int sl = 64 * (4 * i + wv) + lane;
    const bool kpart = sl < kKT * kKC;
    const int s2 = kpart ? sl : sl - kKT * kKC, per = kpart ? kKC : kVC;
    lkey[i] = s2 / per;
    lchunk[i] = swz(s2 % per, lkey[i]) + (kpart ? 0 : kKC);  // 0..23 K, 24..39 V
  }
  auto issue = [&](int t, int stage) {
    const int t0 = t * kKT;
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int64_t row = sb + min(t0 + lkey[i], nkv - 1);  // past the prefix: the last key (masked)
      const int64_t crow = min(max(row, (int64_t)0), cache_rows - 1);
      const int64_t erow = min(max(row - exp_lo, (int64_t)0), exp_rows - 1);
      const int part = lchunk[i];
      const bf16_t* src;
      if (part < 16)
        src = knope + erow * (kHeads * kVD) + h * kVD + part * 8;
      else if (part < 24)
        src = cache + crow * kCacheRow + 512 + (part - 16) * 8;
      else
        src = vexp + erow * (kHeads * kVD) + h * kVD + (part - 24) * 8;
      __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(ring + stage * kStage +
                                                                                          (4 * i + wv) * 1024),
                                       16, 0, 0);
    }
  };
  // tiles past the last one repeat its keys into a stage nobody reads: every wave then has
  // exactly kLoads newer loads in flight at each wait
  issue(0, 0);
  issue(1, 1);

  float m_run[kQB], l_run[kQB];
  floatx4_t acc[kQB][8];
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    m_run[qb] = -INFINITY;
    l_run[qb] = 0.f;
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) acc[qb][mb] = floatx4_t{0.f, 0.f, 0.f, 0.f};
  }

  for (int it = 0; it < ntiles; ++it) {
    const int t0 = it * kKT;
    // this wave's loads of tile it have landed (tile it + 1's may not), then every wave's:
    // the tile is complete and tile it - 1's stage is free for tile it + 2
    __builtin_amdgcn_s_waitcnt(vmcnt_only(kLoads));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    issue(it + 2, (it + 2) % kStages);
    const uint8_t* const kst = ring + (it % kStages) * kStage;
    const uint8_t* const vst = kst + kStageK;
    // S^T: sc[qb][blk][e] = score(key t0 + blk*16 + 4kg + e, query jq[qb]); each K fragment
    // serves both query blocks
    floatx4_t sc[kQB][2];
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      floatx4_t sp[kQB];
#pragma unroll
      for (int qb = 0; qb < kQB; ++qb) sp[qb] = floatx4_t{0.f, 0.f, 0.f, 0.f};
      const int krow = blk * 16 + li;
      const uint8_t* kr = kst + krow * (kKC * 16);
#pragma unroll
      for (int kk = 0; kk < 6; ++kk) {
        const bf16x8_t kf = *reinterpret_cast<const bf16x8_t*>(kr + swz(4 * kk + kg, krow) * 16);
#pragma unroll
        for (int qb = 0; qb < kQB; ++qb) sp[qb] = mfma16x16x32(kf, qf[qb][kk], sp[qb]);
      }
#pragma unroll
      for (int qb = 0; qb < kQB; ++qb) sc[qb][blk] = sp[qb];
    }
    // the causal mask only on tiles that reach past the wave's first query position
    const bool diag = t0 + kKT - 1 > p0 + wv * 16 * kQB;
    bf16x8_t pb[kQB];
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
      float p[8];
      float mx = -INFINITY;  // of the raw scores (scale_log2 > 0 keeps the order)
#pragma unroll
      for (int blk = 0; blk < 2; ++blk)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int kp = t0 + blk * 16 + 4 * kg + e;
          const float v = !diag || kp <= qp[qb] ? sc[qb][blk][e] : -INFINITY;
          p[blk * 4 + e] = v;
          mx = fmaxf(mx, v);
        }
      mx = xor16_max(mx);
      mx = xor32_max(mx);
      // lazy rescaling: the running maximum m (log2 units) moves, and O and l are rescaled,
      // only where the tile's maximum exceeds it by more than 8, so p = 2^(s - m) <= 256
      // (bf16 and the fp32 sums hold it) while most tiles skip the rescale; O / l does not
      // depend on the m chosen.  The first tile always moves m (key 0 is in every query's
      // first tile); a query all of whose keys in a tile are masked has mx = -inf there.
      const float tm = mx * scale_log2;
      const bool grow = tm > m_run[qb] + 8.f;
      if (__any(grow)) {
        const float m_new = grow ? tm : m_run[qb];
        const float alpha = exp2f(m_run[qb] - m_new);  // 0 from m = -inf, 1 where m stays
        l_run[qb] *= alpha;
        m_run[qb] = m_new;
#pragma unroll
        for (int mb = 0; mb < 8; ++mb) acc[qb][mb] *= alpha;
      }
      float rsum = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        p[i] = exp2f(fmaf(p[i], scale_log2, -m_run[qb]));
        rsum += p[i];
      }
      rsum = xor16_sum(rsum);
      rsum = xor32_sum(rsum);
      l_run[qb] += rsum;
      pb[qb] = as_bf16x8(pack8(p));
    }
    // O^T += V^T P^T: lane (li, kg) addresses key 4kg + li/4 (then 16 + 4kg + li/4), dims
    // 16mb + 4(li % 4) .. +3, and receives V[4kg + e][16mb + li] (then V[16 + 4kg + e][..]),
    // the keys of its P^T column in the same order; each V^T fragment serves both blocks
    const int vr = 4 * kg + (li >> 2);  // then vr + 16
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
      const int vc = 2 * mb + ((li & 3) >> 1), vo = (li & 1) * 8;  // chunk, byte in it
      const uint2 lo = lds_read_tr16(reinterpret_cast<const bf16_t*>(vst + vr * (kVC * 16) + swz(vc, vr) * 16 + vo));
      const uint2 hi =
          lds_read_tr16(reinterpret_cast<const bf16_t*>(vst + (vr + 16) * (kVC * 16) + swz(vc, vr + 16) * 16 + vo));
      const bf16x8_t vf = as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
#pragma unroll
      for (int qb = 0; qb < kQB; ++qb) acc[qb][mb] = mfma16x16x32(vf, pb[qb], acc[qb][mb]);
    }
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_only(0));  // the repeats land before the LDS is released
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    if (jq[qb] >= nr) continue;
    const float inv = 1.f / l_run[qb];
    bf16_t* o = out + (int64_t)(r0 + jq[qb]) * os + h * kVD + 4 * kg;
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
      uint2 w;
      w.x = pack2(acc[qb][mb][0] * inv, acc[qb][mb][1] * inv);
      w.y = pack2(acc[qb][mb][2] * inv, acc[qb][mb][3] * inv);
      *reinterpret_cast<uint2*>(o + mb * 16) = w;
    }
  }
}

extern "C" int dsv2_mla_prefill_attention(const void* qkva, int64_t qkva_stride, const void* q_rope,
                                          int64_t q_rope_stride, int rows, const void* cache, int64_t cache_rows,
                                          const void* k_nope, const void* v, int64_t exp_lo, int64_t exp_rows,
                                          const int32_t* tiles, int n_tiles, float softmax_scale, void* out,
                                          int64_t out_stride, void* stream) {
  DSV2_REQUIRE(qkva && q_rope && cache && k_nope && v && tiles && out, DSV2_E_NULL,
               "mla_prefill_attention: null pointer");
  DSV2_REQUIRE(n_tiles >= 0 && n_tiles <= 0x7ffffff && exp_lo >= 0 && qkva_stride >= 3648 &&
                   q_rope_stride >= kHeads * kCacheRow && out_stride >= kHeads * kVD && rows >= 0 &&
                   cache_rows > 0 && exp_rows > 0,
               DSV2_E_SHAPE, "mla_prefill_attention: bad shape");
  DSV2_REQUIRE(dsv2_aligned16(qkva) && dsv2_aligned16(q_rope) && dsv2_aligned16(cache) && dsv2_aligned16(k_nope) &&
                   dsv2_aligned16(v) && dsv2_aligned16(tiles) && dsv2_aligned16(out) && qkva_stride % 8 == 0 &&
                   q_rope_stride % 8 == 0 && out_stride % 4 == 0,
               DSV2_E_ALIGN, "mla_prefill_attention: alignment");
  if (n_tiles == 0 || rows == 0) return DSV2_OK;
  hipLaunchKernelGGL(mla_prefill_kernel, dim3(n_tiles * kHeads), dim3(256), 0, (hipStream_t)stream,
                     (const bf16_t*)qkva, qkva_stride, (const bf16_t*)q_rope, q_rope_stride, (const bf16_t*)cache,
                     cache_rows, (const bf16_t*)k_nope, (const bf16_t*)v, exp_lo, exp_rows, rows, (const int4*)tiles,
                     softmax_scale * 1.4426950408889634f, (bf16_t*)out, out_stride);
  return dsv2_launch_status("mla_prefill_attention");
}
