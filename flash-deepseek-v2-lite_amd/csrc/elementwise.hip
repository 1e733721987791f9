// Elementwise / bookkeeping kernels of the decode step and the library's error plumbing.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

static thread_local char g_err[512] = "";

void dsv2_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int dsv2_launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    dsv2_set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return static_cast<int>(e);
  }
  return DSV2_OK;
}

// ---------------------------------------------------------------------------
// RMSNorm: one workgroup per row, 8 bf16 per thread per pass.
// y = bf16(w * bf16(x * rsqrt(mean(x^2) + eps)))  (HF rounding points)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rmsnorm_kernel(const bf16_t* __restrict__ x, int64_t x_stride,
                                                      const bf16_t* __restrict__ w, bf16_t* __restrict__ y,
                                                      int64_t y_stride, int cols, float eps) {
  __shared__ float red[4];
  const int r = blockIdx.x;
  const bf16_t* xr = x + r * x_stride;
  bf16_t* yr = y + r * y_stride;
  const int nch = cols >> 3;
  float ss = 0.f;
  for (int c = threadIdx.x; c < nch; c += 256) {
    float f[8];
    unpack8(ldg16(xr + c * 8), f);
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(f[i], f[i], ss);
  }
  ss = block_sum<4>(ss, red);
  const float rs = rsqrtf(ss / static_cast<float>(cols) + eps);
  for (int c = threadIdx.x; c < nch; c += 256) {
    float f[8], g[8];
    unpack8(ldg16(xr + c * 8), f);
    unpack8(ldg16(w + c * 8), g);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = g[i] * rbf(f[i] * rs);
    *reinterpret_cast<uint4*>(yr + c * 8) = pack8(f);
  }
}

extern "C" int dsv2_rmsnorm_bf16(const void* x, int64_t x_stride, const void* w, void* y, int64_t y_stride,
                                 int rows, int cols, float eps, void* stream) {
  DSV2_REQUIRE(x && w && y, DSV2_E_NULL, "rmsnorm: null pointer");
  DSV2_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0 && cols <= 8192, DSV2_E_SHAPE, "rmsnorm: bad shape %d x %d",
               rows, cols);
  DSV2_REQUIRE(dsv2_aligned16(x) && dsv2_aligned16(y) && dsv2_aligned16(w) && x_stride % 8 == 0 &&
                   y_stride % 8 == 0,
               DSV2_E_ALIGN, "rmsnorm: pointers/strides must be 16-byte aligned");
  if (rows == 0) return DSV2_OK;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, (hipStream_t)stream, (const bf16_t*)x, x_stride,
                     (const bf16_t*)w, (bf16_t*)y, y_stride, cols, eps);
  return dsv2_launch_status("rmsnorm");
}

// ---------------------------------------------------------------------------
__global__ void residual_add_kernel(const bf16_t* __restrict__ a, const bf16_t* __restrict__ b,
                                    bf16_t* __restrict__ o, int64_t nch) {
  const int64_t c = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (c >= nch) return;
  float fa[8], fb[8];
  unpack8(ldg16(a + c * 8), fa);
  unpack8(ldg16(b + c * 8), fb);
#pragma unroll
  for (int i = 0; i < 8; ++i) fa[i] += fb[i];
  *reinterpret_cast<uint4*>(o + c * 8) = pack8(fa);
}

extern "C" int dsv2_residual_add_bf16(const void* a, const void* b, void* out, int64_t n, void* stream) {
  DSV2_REQUIRE(a && b && out, DSV2_E_NULL, "residual_add: null pointer");
  DSV2_REQUIRE(n >= 0 && n % 8 == 0, DSV2_E_SHAPE, "residual_add: n=%lld must be a multiple of 8", (long long)n);
  DSV2_REQUIRE(dsv2_aligned16(a) && dsv2_aligned16(b) && dsv2_aligned16(out), DSV2_E_ALIGN,
               "residual_add: pointers must be 16-byte aligned");
  if (n == 0) return DSV2_OK;
  const int64_t nch = n / 8;
  hipLaunchKernelGGL(residual_add_kernel, dim3((unsigned)((nch + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const bf16_t*)a, (const bf16_t*)b, (bf16_t*)out, nch);
  return dsv2_launch_status("residual_add");
}

// fp16 variant: o = fp16(fp32(a) + fp32(b)) with round-to-nearest-even conversions
__global__ void residual_add_f16_kernel(const uint4* __restrict__ a, const uint4* __restrict__ b,
                                        uint4* __restrict__ o, int64_t nch) {
  typedef _Float16 halfx8_t __attribute__((ext_vector_type(8)));
  const int64_t c = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (c >= nch) return;
  const halfx8_t va = __builtin_bit_cast(halfx8_t, a[c]), vb = __builtin_bit_cast(halfx8_t, b[c]);
  halfx8_t r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = static_cast<_Float16>(static_cast<float>(va[i]) + static_cast<float>(vb[i]));
  o[c] = __builtin_bit_cast(uint4, r);
}

extern "C" int dsv2_residual_add_f16(const void* a, const void* b, void* out, int64_t n, void* stream) {
  DSV2_REQUIRE(a && b && out, DSV2_E_NULL, "residual_add_f16: null pointer");
  DSV2_REQUIRE(n >= 0 && n % 8 == 0, DSV2_E_SHAPE, "residual_add_f16: n=%lld must be a multiple of 8",
               (long long)n);
  DSV2_REQUIRE(dsv2_aligned16(a) && dsv2_aligned16(b) && dsv2_aligned16(out), DSV2_E_ALIGN,
               "residual_add_f16: pointers must be 16-byte aligned");
  if (n == 0) return DSV2_OK;
  const int64_t nch = n / 8;
  hipLaunchKernelGGL(residual_add_f16_kernel, dim3((unsigned)((nch + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const uint4*)a, (const uint4*)b, (uint4*)out, nch);
  return dsv2_launch_status("residual_add_f16");
}

// ---------------------------------------------------------------------------
__global__ void silu_mul_kernel(const bf16_t* __restrict__ g, const bf16_t* __restrict__ u,
                                bf16_t* __restrict__ o, int64_t nch) {
  const int64_t c = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (c >= nch) return;
  float fg[8], fu[8];
  unpack8(ldg16(g + c * 8), fg);
  unpack8(ldg16(u + c * 8), fu);
#pragma unroll
  for (int i = 0; i < 8; ++i) fg[i] = silu_f(fg[i]) * fu[i];
  *reinterpret_cast<uint4*>(o + c * 8) = pack8(fg);
}

extern "C" int dsv2_silu_mul_bf16(const void* gate, const void* up, void* out, int64_t n, void* stream) {
  DSV2_REQUIRE(gate && up && out, DSV2_E_NULL, "silu_mul: null pointer");
  DSV2_REQUIRE(n >= 0 && n % 8 == 0, DSV2_E_SHAPE, "silu_mul: n=%lld must be a multiple of 8", (long long)n);
  DSV2_REQUIRE(dsv2_aligned16(gate) && dsv2_aligned16(up) && dsv2_aligned16(out), DSV2_E_ALIGN,
               "silu_mul: pointers must be 16-byte aligned");
  if (n == 0) return DSV2_OK;
  const int64_t nch = n / 8;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((nch + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const bf16_t*)gate, (const bf16_t*)up, (bf16_t*)out, nch);
  return dsv2_launch_status("silu_mul");
}

// ---------------------------------------------------------------------------
__global__ void prepare_inputs_kernel(const int64_t* __restrict__ cache_position, const int64_t* __restrict__ index,
                                      int64_t* __restrict__ mask, int64_t* __restrict__ position_ids, int max_len) {
  const int b = blockIdx.y;
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t pos = cache_position[0];
  if (j < max_len) {
    const int64_t idx = index ? index[j] : j;
    mask[(int64_t)b * max_len + j] = (idx <= pos) ? 1 : 0;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) position_ids[b] = pos;
}

extern "C" int dsv2_prepare_decode_inputs(const int64_t* cache_position, const int64_t* attention_mask_index,
                                          int64_t* attention_mask, int64_t* position_ids, int batch, int max_len,
                                          void* stream) {
  DSV2_REQUIRE(cache_position && attention_mask && position_ids, DSV2_E_NULL, "prepare_decode_inputs: null pointer");
  DSV2_REQUIRE(batch >= 0 && max_len > 0 && batch <= 65535, DSV2_E_SHAPE, "prepare_decode_inputs: bad shape");
  if (batch == 0) return DSV2_OK;
  hipLaunchKernelGGL(prepare_inputs_kernel, dim3((max_len + 255) / 256, batch), dim3(256), 0, (hipStream_t)stream,
                     cache_position, attention_mask_index, attention_mask, position_ids, max_len);
  return dsv2_launch_status("prepare_decode_inputs");
}

// ---------------------------------------------------------------------------
__global__ void copy_token_rows_kernel(const uint4* __restrict__ src, int64_t src_bstride16, uint4* __restrict__ dst,
                                       int64_t dst_bstride16, int64_t row16, const int64_t* __restrict__ cache_position,
                                       int64_t max_tokens, int32_t* __restrict__ status) {
  const int b = blockIdx.y;
  const int64_t pos = cache_position[0];
  if (pos < 0 || pos >= max_tokens) {  // past the cache: nothing is written, the status is flagged
    if (status && threadIdx.x == 0 && blockIdx.x == 0) atomicOr(status, DSV2_DEVERR_CACHE_FULL);
    return;
  }
  for (int64_t c = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; c < row16; c += (int64_t)gridDim.x * blockDim.x)
    dst[b * dst_bstride16 + pos * row16 + c] = src[b * src_bstride16 + c];
}

extern "C" int dsv2_copy_token_rows(const void* src, int64_t src_batch_stride, void* dst, int64_t dst_batch_stride,
                                    int64_t row_bytes, const int64_t* cache_position, int64_t max_tokens, int batch,
                                    int32_t* status, void* stream) {
  DSV2_REQUIRE(src && dst && cache_position, DSV2_E_NULL, "copy_token_rows: null pointer");
  DSV2_REQUIRE(batch >= 0 && batch <= 65535 && row_bytes > 0 && row_bytes % 16 == 0 && max_tokens > 0, DSV2_E_SHAPE,
               "copy_token_rows: bad shape");
  DSV2_REQUIRE(dsv2_aligned16(src) && dsv2_aligned16(dst) && src_batch_stride % 16 == 0 &&
                   dst_batch_stride % 16 == 0,
               DSV2_E_ALIGN, "copy_token_rows: 16-byte alignment required");
  if (batch == 0) return DSV2_OK;
  const int64_t row16 = row_bytes / 16;
  const unsigned gx = (unsigned)((row16 + 255) / 256 < 64 ? (row16 + 255) / 256 : 64);
  hipLaunchKernelGGL(copy_token_rows_kernel, dim3(gx, batch), dim3(256), 0, (hipStream_t)stream, (const uint4*)src,
                     src_batch_stride / 16, (uint4*)dst, dst_batch_stride / 16, row16, cache_position, max_tokens,
                     status);
  return dsv2_launch_status("copy_token_rows");
}

// ---------------------------------------------------------------------------
__global__ void fill_positions_kernel(const int64_t* __restrict__ cache_position, int32_t* __restrict__ pos,
                                      int64_t* __restrict__ base, int32_t* __restrict__ capv, int64_t cap, int batch) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  // positions outside int32 saturate; the capacity check downstream then rejects them
  const int64_t p = cache_position[0];
  pos[b] = static_cast<int32_t>(p < 0 ? -1 : (p > 0x7fffffff ? 0x7fffffff : p));
  if (base) base[b] = (int64_t)b * cap;
  if (capv) capv[b] = static_cast<int32_t>(cap);
}

extern "C" int dsv2_fill_positions(const int64_t* cache_position, int32_t* pos, int64_t* base, int32_t* cap,
                                   int64_t per_row_capacity, int batch, void* stream) {
  DSV2_REQUIRE(cache_position && pos, DSV2_E_NULL, "fill_positions: null pointer");
  DSV2_REQUIRE(batch >= 0 && batch <= (1 << 24) && per_row_capacity > 0 && per_row_capacity <= 0x7fffffff,
               DSV2_E_SHAPE, "fill_positions: bad batch or capacity");
  if (batch == 0) return DSV2_OK;
  hipLaunchKernelGGL(fill_positions_kernel, dim3((batch + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                     cache_position, pos, base, cap, per_row_capacity, batch);
  return dsv2_launch_status("fill_positions");
}

// ---------------------------------------------------------------------------
__global__ void embed_gather_kernel(const int64_t* __restrict__ ids, const bf16_t* __restrict__ table, int hidden,
                                    bf16_t* __restrict__ out) {
  const int r = blockIdx.x;
  const int64_t id = ids[r];
  const int nch = hidden >> 3;
  for (int c = threadIdx.x; c < nch; c += blockDim.x)
    *reinterpret_cast<uint4*>(out + (int64_t)r * hidden + c * 8) = ldg16(table + id * hidden + c * 8);
}

extern "C" int dsv2_embed_gather_bf16(const int64_t* ids, const void* table, int hidden, void* out, int rows,
                                      void* stream) {
  DSV2_REQUIRE(ids && table && out, DSV2_E_NULL, "embed_gather: null pointer");
  DSV2_REQUIRE(rows >= 0 && hidden > 0 && hidden % 8 == 0, DSV2_E_SHAPE, "embed_gather: bad shape");
  if (rows == 0) return DSV2_OK;
  hipLaunchKernelGGL(embed_gather_kernel, dim3(rows), dim3(256), 0, (hipStream_t)stream, ids, (const bf16_t*)table,
                     hidden, (bf16_t*)out);
  return dsv2_launch_status("embed_gather");
}

// ---------------------------------------------------------------------------
// Greedy argmax (first index of the maximum, like torch.argmax) + position step.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void argmax_kernel(const float* __restrict__ logits, int vocab,
                                                      int64_t* __restrict__ next_ids, int32_t* __restrict__ pos) {
  __shared__ float sv[16];
  __shared__ int si[16];
  const int r = blockIdx.x;
  const float* lr = logits + (int64_t)r * vocab;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  const int nch = vocab >> 2;
  // kU of the thread's 16-byte chunks requested together (clamped, masked where compared),
  // then compared in index order: one load round trip per kU chunks instead of per chunk
  constexpr int kU = 16;
  for (int c0 = threadIdx.x; c0 < nch; c0 += 1024 * kU) {
    float4 v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) v[u] = reinterpret_cast<const float4*>(lr)[min(c0 + 1024 * u, nch - 1)];
#pragma unroll
    for (int u = 0; u < kU; ++u) pin(__float_as_uint(v[u].x));  // all issued before the first wait
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int c = c0 + 1024 * u;
      const float vv[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (c < nch && vv[i] > best) {
          best = vv[i];
          bi = c * 4 + i;
        }
    }
  }
  for (int j = nch * 4 + threadIdx.x; j < vocab; j += 1024)
    if (lr[j] > best) {
      best = lr[j];
      bi = j;
    }
  wave_argmax(best, bi);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) {
    sv[w] = best;
    si[w] = bi;
  }
  __syncthreads();
  if (w == 0) {
    best = lane < 16 ? sv[lane] : -INFINITY;
    bi = lane < 16 ? si[lane] : 0x7fffffff;
    wave_argmax(best, bi);
    if (lane == 0) {
      next_ids[r] = bi == 0x7fffffff ? 0 : bi;
      if (pos) pos[r] += 1;
    }
  }
}

extern "C" int dsv2_argmax_f32(const float* logits, int rows, int vocab, int64_t* next_ids, int32_t* pos,
                               void* stream) {
  DSV2_REQUIRE(logits && next_ids, DSV2_E_NULL, "argmax: null pointer");
  DSV2_REQUIRE(rows >= 0 && vocab > 0, DSV2_E_SHAPE, "argmax: bad shape");
  DSV2_REQUIRE(dsv2_aligned16(logits) && vocab % 4 == 0, DSV2_E_ALIGN, "argmax: logits rows must be 16B aligned");
  if (rows == 0) return DSV2_OK;
  hipLaunchKernelGGL(argmax_kernel, dim3(rows), dim3(1024), 0, (hipStream_t)stream, logits, vocab, next_ids, pos);
  return dsv2_launch_status("argmax");
}

// ---------------------------------------------------------------------------
// Device copy (a measurement reference, not a step kernel): every thread moves 4 x 16 B per
// pass, all four loads in flight before the stores, a grid of a few resident waves per SIMD
// striding over the buffer; non-temporal loads and stores (the bytes are touched once).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void stream_copy_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                                          int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * 256 * 4;
  for (int64_t i = (int64_t)blockIdx.x * 256 * 4 + threadIdx.x; i < n16; i += stride) {
    u32x4_t v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int64_t j = min(i + k * 256, n16 - 1);  // past the end: the last unit (not stored)
      v[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(src + j));
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (i + k * 256 < n16) __builtin_nontemporal_store(v[k], reinterpret_cast<u32x4_t*>(dst + i + k * 256));
  }
}

extern "C" int dsv2_stream_copy(const void* src, void* dst, int64_t nbytes, void* stream) {
  DSV2_REQUIRE(src && dst, DSV2_E_NULL, "stream_copy: null pointer");
  DSV2_REQUIRE(nbytes >= 0 && nbytes % 16 == 0, DSV2_E_SHAPE, "stream_copy: nbytes %% 16 required");
  DSV2_REQUIRE(dsv2_aligned16(src) && dsv2_aligned16(dst), DSV2_E_ALIGN, "stream_copy: alignment");
  if (nbytes == 0) return DSV2_OK;
  const int64_t n16 = nbytes / 16;
  const int64_t wgs = min((int64_t)256 * 8, (n16 + 1023) / 1024);
  hipLaunchKernelGGL(stream_copy_kernel, dim3((unsigned)wgs), dim3(256), 0, (hipStream_t)stream, (const uint4*)src,
                     (uint4*)dst, n16);
  return dsv2_launch_status("stream_copy");
}

extern "C" int dsv2_abi_version(void) { return DSV2_ABI_VERSION; }
extern "C" const char* dsv2_last_error_message(void) { return g_err; }
