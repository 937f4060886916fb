// Element-wise and row-wise bf16 ops of the decode layer chain around the
// quantized projections (RMSNorm, SwiGLU gate, residual add, GQA head
// repeat), with MLX's bf16 rounding points:
//   rms_norm  (src/primitives/nn.rs:35-37 -> mlx fast::rms_norm):
//             y = bf16( w * bf16( x * 1/sqrt(mean(x^2) + eps) ) ), sums in f32
//   silu_mul  (src/models/llama.rs:1040-1045: silu(gate) * up, nn.rs:50-52):
//             s = bf16(1 / (1 + exp(-g))); a = bf16(g * s); y = bf16(a * u)
//   add       (src/models/llama.rs:725-733 residual adds): y = bf16(a + b)
//   repeat_kv (src/primitives/attention.rs:45-55): head h of the output is
//             KV head h / groups (groups adjacent)
// All are HBM-bound and tiny next to the projections; 16-byte vectors.
#include <hip/hip_runtime.h>

#include <string>

#include "common.hpp"

using namespace mlxq;

namespace {

constexpr int kNormThreads = 256;

__device__ __forceinline__ float lo_f(uint32_t w) { return bf16_bits_to_f32(w & 0xFFFFu); }
__device__ __forceinline__ float hi_f(uint32_t w) { return bf16_bits_to_f32(w >> 16); }
__device__ __forceinline__ uint32_t pack2(float a, float b) { return f32_to_bf16_bits(a) | (f32_to_bf16_bits(b) << 16); }

// one workgroup per row; D % 8 == 0
__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(const uint16_t* __restrict__ x,
                                                                const uint16_t* __restrict__ w, int D, float eps,
                                                                uint16_t* __restrict__ y) {
  __shared__ float part[kNormThreads / 64];
  const int row = blockIdx.x;
  const uint4* xr = reinterpret_cast<const uint4*>(x + static_cast<int64_t>(row) * D);
  uint4* yr = reinterpret_cast<uint4*>(y + static_cast<int64_t>(row) * D);
  const uint4* wv = reinterpret_cast<const uint4*>(w);
  const int pieces = D / 8;
  float ss = 0.f;
  for (int i = threadIdx.x; i < pieces; i += kNormThreads) {
    const uint4 v = xr[i];
    const uint32_t a[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float p = lo_f(a[j]), q = hi_f(a[j]);
      ss = fmaf(p, p, ss);
      ss = fmaf(q, q, ss);
    }
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; i++) tot += part[i];
  const float inv = 1.0f / sqrtf(tot / static_cast<float>(D) + eps);
  for (int i = threadIdx.x; i < pieces; i += kNormThreads) {
    const uint4 v = xr[i], g = wv[i];
    const uint32_t a[4] = {v.x, v.y, v.z, v.w}, b[4] = {g.x, g.y, g.z, g.w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float n0 = bf16_bits_to_f32(f32_to_bf16_bits(lo_f(a[j]) * inv));
      const float n1 = bf16_bits_to_f32(f32_to_bf16_bits(hi_f(a[j]) * inv));
      o[j] = pack2(lo_f(b[j]) * n0, hi_f(b[j]) * n1);
    }
    yr[i] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// The same computation with the row's pieces (i = t, t + 256, ...; at most
// PT per thread) loaded once, all before any arithmetic, and kept in
// registers for the second pass: one memory round trip instead of three.
template <int PT>
__global__ __launch_bounds__(kNormThreads) void rms_norm_reg_kernel(const uint16_t* __restrict__ x,
                                                                    const uint16_t* __restrict__ w, int D, float eps,
                                                                    uint16_t* __restrict__ y) {
  __shared__ float part[kNormThreads / 64];
  const int row = blockIdx.x;
  const uint4* xr = reinterpret_cast<const uint4*>(x + static_cast<int64_t>(row) * D);
  uint4* yr = reinterpret_cast<uint4*>(y + static_cast<int64_t>(row) * D);
  const uint4* wv = reinterpret_cast<const uint4*>(w);
  const int pieces = D / 8;
  uint4 v[PT], g[PT];
#pragma unroll
  for (int k = 0; k < PT; k++) {
    const int i = min(static_cast<int>(threadIdx.x) + kNormThreads * k, pieces - 1);  // clamped, no branch
    v[k] = xr[i];
    g[k] = wv[i];
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < PT; k++) {
    if (static_cast<int>(threadIdx.x) + kNormThreads * k >= pieces) break;
    const uint32_t a[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float p = lo_f(a[j]), q = hi_f(a[j]);
      ss = fmaf(p, p, ss);
      ss = fmaf(q, q, ss);
    }
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; i++) tot += part[i];
  const float inv = 1.0f / sqrtf(tot / static_cast<float>(D) + eps);
#pragma unroll
  for (int k = 0; k < PT; k++) {
    const int i = static_cast<int>(threadIdx.x) + kNormThreads * k;
    if (i >= pieces) break;
    const uint32_t a[4] = {v[k].x, v[k].y, v[k].z, v[k].w}, b[4] = {g[k].x, g[k].y, g[k].z, g[k].w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float n0 = bf16_bits_to_f32(f32_to_bf16_bits(lo_f(a[j]) * inv));
      const float n1 = bf16_bits_to_f32(f32_to_bf16_bits(hi_f(a[j]) * inv));
      o[j] = pack2(lo_f(b[j]) * n0, hi_f(b[j]) * n1);
    }
    yr[i] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

__device__ __forceinline__ float silu_bf16(float g) {
  const float s = bf16_bits_to_f32(f32_to_bf16_bits(1.0f / (1.0f + expf(-g))));
  return bf16_bits_to_f32(f32_to_bf16_bits(g * s));
}

// n8 = number of 8-element pieces
__global__ void silu_mul_kernel(const uint4* __restrict__ g, const uint4* __restrict__ u, int64_t n8,
                                uint4* __restrict__ y) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n8;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const uint4 a = g[i], b = u[i];
    const uint32_t ga[4] = {a.x, a.y, a.z, a.w}, ub[4] = {b.x, b.y, b.z, b.w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; j++) o[j] = pack2(silu_bf16(lo_f(ga[j])) * lo_f(ub[j]), silu_bf16(hi_f(ga[j])) * hi_f(ub[j]));
    y[i] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// The residual add of a layer's end and the RMSNorm that starts the next
// layer (or the final norm) in one pass: one workgroup per row writes
// s = bf16(a + b) and y = rms_norm(s), each rounded as add_kernel /
// rms_norm_kernel round it.  s may be a or b (the in-place residual update
// h = h + x): each element of a and b is read once, by the thread that then
// writes that element of s, and the second pass reads s back (the same
// thread's own writes), never a or b.
__global__ __launch_bounds__(kNormThreads) void add_rms_norm_kernel(const uint16_t* a, const uint16_t* b,
                                                                    const uint16_t* __restrict__ w, int D, float eps,
                                                                    uint16_t* s, uint16_t* __restrict__ y) {
  __shared__ float part[kNormThreads / 64];
  const int64_t off = static_cast<int64_t>(blockIdx.x) * D;
  const uint4* ar = reinterpret_cast<const uint4*>(a + off);
  const uint4* br = reinterpret_cast<const uint4*>(b + off);
  uint4* sr = reinterpret_cast<uint4*>(s + off);
  uint4* yr = reinterpret_cast<uint4*>(y + off);
  const uint4* wv = reinterpret_cast<const uint4*>(w);
  const int pieces = D / 8;
  float ss = 0.f;
  for (int i = threadIdx.x; i < pieces; i += kNormThreads) {
    const uint4 p = ar[i], q = br[i];
    const uint32_t pa[4] = {p.x, p.y, p.z, p.w}, qb[4] = {q.x, q.y, q.z, q.w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      o[j] = pack2(lo_f(pa[j]) + lo_f(qb[j]), hi_f(pa[j]) + hi_f(qb[j]));
      const float u = lo_f(o[j]), v = hi_f(o[j]);
      ss = fmaf(u, u, ss);
      ss = fmaf(v, v, ss);
    }
    sr[i] = make_uint4(o[0], o[1], o[2], o[3]);
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; i++) tot += part[i];
  const float inv = 1.0f / sqrtf(tot / static_cast<float>(D) + eps);
  for (int i = threadIdx.x; i < pieces; i += kNormThreads) {
    const uint4 p = sr[i], g = wv[i];  // the sums this thread wrote above
    const uint32_t sa[4] = {p.x, p.y, p.z, p.w}, gw[4] = {g.x, g.y, g.z, g.w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t sv = sa[j];
      const float n0 = bf16_bits_to_f32(f32_to_bf16_bits(lo_f(sv) * inv));
      const float n1 = bf16_bits_to_f32(f32_to_bf16_bits(hi_f(sv) * inv));
      o[j] = pack2(lo_f(gw[j]) * n0, hi_f(gw[j]) * n1);
    }
    yr[i] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

__global__ void add_kernel(const uint4* __restrict__ a, const uint4* __restrict__ b, int64_t n8,
                           uint4* __restrict__ y) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n8;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const uint4 p = a[i], q = b[i];
    const uint32_t pa[4] = {p.x, p.y, p.z, p.w}, qb[4] = {q.x, q.y, q.z, q.w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; j++) o[j] = pack2(lo_f(pa[j]) + lo_f(qb[j]), hi_f(pa[j]) + hi_f(qb[j]));
    y[i] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// x: [rows, kv_heads, hd]; y: [rows, kv_heads * groups, hd]; hd % 8 == 0
__global__ void repeat_kv_kernel(const uint4* __restrict__ x, int64_t rows, int kv_heads, int groups, int hd8,
                                 uint4* __restrict__ y) {
  const int64_t out_row = static_cast<int64_t>(kv_heads) * groups * hd8;
  const int64_t total = rows * out_row;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = i / out_row, c = i % out_row;
    const int64_t h = c / hd8, d = c % hd8;
    y[i] = x[(r * kv_heads + h / groups) * hd8 + d];
  }
}

bool misaligned(const void* p) { return reinterpret_cast<uintptr_t>(p) & 15u; }

unsigned grid_for(int64_t n8) { return static_cast<unsigned>(std::min<int64_t>(ceil_div(n8, 256), 4096)); }

}  // namespace

extern "C" int mlxq_rms_norm(const void* x, const void* weight, int64_t rows, int64_t dim, float eps, void* y,
                             void* stream) {
  clear_error();
  if (rows < 0 || dim <= 0 || dim > (1 << 24)) return fail(MLXQ_ERR_INVALID, "rms_norm: bad shape");
  if (dim % 8) return fail(MLXQ_ERR_SHAPE, "rms_norm: dim must be a multiple of 8");
  if (!(eps >= 0.f)) return fail(MLXQ_ERR_INVALID, "rms_norm: eps must be >= 0");
  if (rows == 0) return MLXQ_OK;
  if (!x || !weight || !y) return fail(MLXQ_ERR_INVALID, "rms_norm: null pointer");
  if (misaligned(x) || misaligned(weight) || misaligned(y))
    return fail(MLXQ_ERR_INVALID, "rms_norm: pointers must be 16-byte aligned");
  if (rows > INT32_MAX) return fail(MLXQ_ERR_INVALID, "rms_norm: too many rows");
  // rows of up to 16384: the register-resident form (same results)
  const int64_t pt = ceil_div(dim / 8, int64_t(kNormThreads));
  auto kern = pt <= 1 ? rms_norm_reg_kernel<1>
              : pt <= 2 ? rms_norm_reg_kernel<2>
              : pt <= 4 ? rms_norm_reg_kernel<4>
              : pt <= 8 ? rms_norm_reg_kernel<8>
                        : rms_norm_kernel;
  MLXQ_LAUNCH(kern, dim3(static_cast<unsigned>(rows)), dim3(kNormThreads), 0, as_stream(stream),
                     static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(weight), static_cast<int>(dim),
                     eps, static_cast<uint16_t*>(y));
  return check_launch("rms_norm");
}

extern "C" int mlxq_add_rms_norm(const void* a, const void* b, const void* weight, int64_t rows, int64_t dim,
                                 float eps, void* sum, void* y, void* stream) {
  clear_error();
  if (rows < 0 || dim <= 0) return fail(MLXQ_ERR_INVALID, "add_rms_norm: bad shape");
  if (dim % 8) return fail(MLXQ_ERR_SHAPE, "add_rms_norm: dim must be a multiple of 8");
  if (!(eps >= 0.f)) return fail(MLXQ_ERR_INVALID, "add_rms_norm: eps must be >= 0");
  if (rows == 0) return MLXQ_OK;
  if (!a || !b || !weight || !sum || !y) return fail(MLXQ_ERR_INVALID, "add_rms_norm: null pointer");
  if (misaligned(a) || misaligned(b) || misaligned(weight) || misaligned(sum) || misaligned(y))
    return fail(MLXQ_ERR_INVALID, "add_rms_norm: pointers must be 16-byte aligned");
  if (rows > INT32_MAX || dim > INT32_MAX) return fail(MLXQ_ERR_INVALID, "add_rms_norm: too large");
  MLXQ_LAUNCH(add_rms_norm_kernel, dim3(static_cast<unsigned>(rows)), dim3(kNormThreads), 0,
                     as_stream(stream), static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b),
                     static_cast<const uint16_t*>(weight), static_cast<int>(dim), eps, static_cast<uint16_t*>(sum),
                     static_cast<uint16_t*>(y));
  return check_launch("add_rms_norm");
}

extern "C" int mlxq_silu_mul(const void* gate, const void* up, int64_t n, void* y, void* stream) {
  clear_error();
  if (n < 0) return fail(MLXQ_ERR_INVALID, "silu_mul: bad size");
  if (n % 8) return fail(MLXQ_ERR_SHAPE, "silu_mul: n must be a multiple of 8");
  if (n == 0) return MLXQ_OK;
  if (!gate || !up || !y) return fail(MLXQ_ERR_INVALID, "silu_mul: null pointer");
  if (misaligned(gate) || misaligned(up) || misaligned(y))
    return fail(MLXQ_ERR_INVALID, "silu_mul: pointers must be 16-byte aligned");
  const int64_t n8 = n / 8;
  MLXQ_LAUNCH(silu_mul_kernel, dim3(grid_for(n8)), dim3(256), 0, as_stream(stream),
                     static_cast<const uint4*>(gate), static_cast<const uint4*>(up), n8, static_cast<uint4*>(y));
  return check_launch("silu_mul");
}

extern "C" int mlxq_add(const void* a, const void* b, int64_t n, void* y, void* stream) {
  clear_error();
  if (n < 0) return fail(MLXQ_ERR_INVALID, "add: bad size");
  if (n % 8) return fail(MLXQ_ERR_SHAPE, "add: n must be a multiple of 8");
  if (n == 0) return MLXQ_OK;
  if (!a || !b || !y) return fail(MLXQ_ERR_INVALID, "add: null pointer");
  if (misaligned(a) || misaligned(b) || misaligned(y))
    return fail(MLXQ_ERR_INVALID, "add: pointers must be 16-byte aligned");
  const int64_t n8 = n / 8;
  MLXQ_LAUNCH(add_kernel, dim3(grid_for(n8)), dim3(256), 0, as_stream(stream), static_cast<const uint4*>(a),
                     static_cast<const uint4*>(b), n8, static_cast<uint4*>(y));
  return check_launch("add");
}

extern "C" int mlxq_repeat_kv(const void* x, int64_t rows, int kv_heads, int head_dim, int groups, void* y,
                              void* stream) {
  clear_error();
  if (rows < 0 || kv_heads <= 0 || head_dim <= 0 || groups <= 0) return fail(MLXQ_ERR_INVALID, "repeat_kv: bad shape");
  if (head_dim % 8) return fail(MLXQ_ERR_SHAPE, "repeat_kv: head_dim must be a multiple of 8");
  if (rows == 0) return MLXQ_OK;
  if (!x || !y) return fail(MLXQ_ERR_INVALID, "repeat_kv: null pointer");
  if (misaligned(x) || misaligned(y)) return fail(MLXQ_ERR_INVALID, "repeat_kv: pointers must be 16-byte aligned");
  const int64_t total = rows * kv_heads * groups * (head_dim / 8);
  MLXQ_LAUNCH(repeat_kv_kernel, dim3(grid_for(total)), dim3(256), 0, as_stream(stream),
                     static_cast<const uint4*>(x), rows, kv_heads, groups, head_dim / 8, static_cast<uint4*>(y));
  return check_launch("repeat_kv");
}
