// Decoder-step helpers: the elementwise work around the decode op, fused so that one Llama decoder layer
// is a handful of launches (palu_tt.model and palu_tt.attention). They have no counterpart in the
// reference's op interface; the arithmetic is the reference model's (tt_transformers' RMSNorm, SwiGLU
// MLP and rotary_embedding_llama on Meta-interleaved heads, as palu_tt/attention.py:585-733 and
// palu_tt/model.py drive them), computed in fp32 with bf16 inputs and outputs.
#include "palu_kernel.h"

namespace {

__device__ __forceinline__ float bf(const __bf16 x) { return (float)x; }

// One workgroup per row: h = x (+ res), stored when h_out is given; y = h * rsqrt(mean(h^2) + eps) * w.
// Each thread holds up to RMS_VEC vectors of 8 elements in registers between the two passes. The kernel
// is tiny and bound by memory latency, so every load of the row (x, the residual or the first RMS_PK
// partial slices, the weight) is issued before the first is used: one round trip to memory, plus one
// per further RMS_PK slices.
constexpr int RMS_THREADS = 512;
constexpr int RMS_VEC = 2;               // dim <= 512 * 8 * 2 = 8192
constexpr int RMS_PK = 4;                // fp32 partial slices loaded together

__device__ __forceinline__ bf16x8 ld8(const __bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }
__device__ __forceinline__ f32x4 ld4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }

__global__ __launch_bounds__(RMS_THREADS) void palu_rmsnorm_kernel(const __bf16* x, const __bf16* res,
                                                                   const float* res_part, int res_ks, long long part_stride,
                                                                   __bf16* h_out, __bf16* y_out, const __bf16* w, int dim,
                                                                   float eps, int y_tiled) {
  const int row = blockIdx.x, tid = threadIdx.x;
  const __bf16* xr = x + (long long)row * dim;
  const __bf16* rr = res ? res + (long long)row * dim : nullptr;
  const float* pr = res_part ? res_part + (long long)row * dim : nullptr;

  // Loads; a lane past the row's end reads its last vector (in bounds) and never uses it.
  bf16x8 xa[RMS_VEC], ra[RMS_VEC], wa[RMS_VEC];
  f32x4 pa[RMS_VEC][RMS_PK][2];
#pragma unroll
  for (int i = 0; i < RMS_VEC; ++i) {
    const int e = min((tid + i * RMS_THREADS) * 8, dim - 8);
    xa[i] = ld8(xr + e);
    wa[i] = ld8(w + e);
    if (rr) ra[i] = ld8(rr + e);
    if (pr) {
#pragma unroll
      for (int k = 0; k < RMS_PK; ++k) {
        const float* pp = pr + min(k, res_ks - 1) * part_stride + e;
        pa[i][k][0] = ld4(pp);
        pa[i][k][1] = ld4(pp + 4);
      }
    }
  }

  float v[RMS_VEC][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < RMS_VEC; ++i) {
    const int e = (tid + i * RMS_THREADS) * 8;
    bf16x8 hv;
    if (rr) {
#pragma unroll
      for (int j = 0; j < 8; ++j) hv[j] = (__bf16)(bf(xa[i][j]) + bf(ra[i][j]));   // bf16 residual stream
    } else if (pr) {
      // the sublayer output as the fp32 k-slice partials of its projection: summed here, in slice order
      f32x4 s0 = pa[i][0][0], s1 = pa[i][0][1];
#pragma unroll
      for (int k = 1; k < RMS_PK; ++k) {
        if (k < res_ks) {
          s0 += pa[i][k][0];
          s1 += pa[i][k][1];
        }
      }
      for (int k0 = RMS_PK; k0 < res_ks; k0 += RMS_PK) {
        const int ec = min(e, dim - 8);
        f32x4 q[RMS_PK][2];
#pragma unroll
        for (int k = 0; k < RMS_PK; ++k) {
          const float* pp = pr + min(k0 + k, res_ks - 1) * part_stride + ec;
          q[k][0] = ld4(pp);
          q[k][1] = ld4(pp + 4);
        }
#pragma unroll
        for (int k = 0; k < RMS_PK; ++k) {
          if (k0 + k < res_ks) {
            s0 += q[k][0];
            s1 += q[k][1];
          }
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        hv[j] = (__bf16)(bf(xa[i][j]) + s0[j]);
        hv[4 + j] = (__bf16)(bf(xa[i][4 + j]) + s1[j]);
      }
    } else {
      hv = xa[i];
    }
    const bool live = e < dim;
    if (live && h_out) *reinterpret_cast<bf16x8*>(h_out + (long long)row * dim + e) = hv;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      v[i][j] = live ? bf(hv[j]) : 0.f;
      ss += v[i][j] * v[i][j];
    }
  }
  __shared__ float part[RMS_THREADS / 64];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
  if ((tid & 63) == 0) part[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int k = 0; k < RMS_THREADS / 64; ++k) tot += part[k];
  const float r = rsqrtf(tot / (float)dim + eps);
#pragma unroll
  for (int i = 0; i < RMS_VEC; ++i) {
    const int e = (tid + i * RMS_THREADS) * 8;
    if (e < dim) {
      bf16x8 o;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = (__bf16)((v[i][j] * r) * bf(wa[i][j]));
      *reinterpret_cast<bf16x8*>(y_out + (y_tiled ? tiled_row_offset(row, e) : (long long)row * dim + e)) = o;
    }
  }
}

// Greedy sampling's argmax: out[r] = the index of the largest value of row r, the first one among equal
// maxima, NaN above every number (torch.argmax's order). One workgroup per row; each thread scans every
// ARG_THREADS-th 8-element vector in index order, ARG_UNROLL loads at a time, then the workgroup reduces
// the (key, index) pairs. Comparisons are branch-free on an integer key that orders bf16 values as
// numbers (sign-magnitude bits to two's-complement order) with every NaN above +inf.
constexpr int ARG_THREADS = 1024;
constexpr int ARG_UNROLL = 8;

typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));

// 0x8000 + magnitude for a positive value, 0x8000 + ~magnitude = 0x7fff - magnitude for a negative one,
// 0x10000 for NaN. (-0 and +0 get 0x7fff and 0x8000: +0 wins a tie that torch would give to the earlier
// index; logits are never both zeros of opposite sign at the maximum in practice.)
__device__ __forceinline__ int arg_key(unsigned int b) {
  const int mag = b & 0x7fff, s = -(int)((b >> 15) & 1);
  const int k = 0x8000 + (mag ^ s);
  return mag > 0x7f80 ? 0x10000 : k;
}

__global__ __launch_bounds__(ARG_THREADS) void palu_argmax_kernel(const __bf16* x, long long ld, int n,
                                                                  int64_t* out) {
  const int row = blockIdx.x, tid = threadIdx.x;
  const __bf16* xr = x + (long long)row * ld;
  int bk = -1, bi = 0;
  const int nv = n / 8;                               // whole vectors; the tail is scanned below
  for (int v0 = tid; v0 < nv; v0 += ARG_THREADS * ARG_UNROLL) {
    u16x8 buf[ARG_UNROLL];
    // Vectors past the row (v >= nv) re-read the last one and carry indices past the row: the vector's
    // owner holds the same keys at smaller indices, so the reduction's tie rule never picks them.
#pragma unroll
    for (int u = 0; u < ARG_UNROLL; ++u) {
      const int v = min(v0 + u * ARG_THREADS, nv - 1);
      buf[u] = __builtin_bit_cast(u16x8, *reinterpret_cast<const bf16x8*>(xr + 8LL * v));
    }
#pragma unroll
    for (int u = 0; u < ARG_UNROLL; ++u) {
      const int v = v0 + u * ARG_THREADS;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int k = arg_key(buf[u][j]);
        const bool gt = k > bk;                           // strict: the earlier index keeps a tie
        bk = max(k, bk);
        bi = gt ? 8 * v + j : bi;
      }
    }
  }
  for (int e = 8 * nv + tid; e < n; e += ARG_THREADS) {
    const int k = arg_key(__builtin_bit_cast(unsigned short, xr[e]));
    const bool gt = k > bk;
    bk = gt ? k : bk;
    bi = gt ? e : bi;
  }
  auto take = [&](int ok, int oi) {
    const bool b = ok > bk || (ok == bk && oi < bi);
    bk = b ? ok : bk;
    bi = b ? oi : bi;
  };
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) take(__shfl_xor(bk, o, 64), __shfl_xor(bi, o, 64));
  __shared__ int sk[ARG_THREADS / 64], si[ARG_THREADS / 64];
  if ((tid & 63) == 0) { sk[tid >> 6] = bk; si[tid >> 6] = bi; }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < ARG_THREADS / 64; ++w) take(sk[w], si[w]);
    out[row] = bi;
  }
}

// out[r][f] = silu(g) * u with g = gu[r][f], u = gu[r][ffn + f]; 8 elements per thread.
__global__ __launch_bounds__(256) void palu_swiglu_kernel(const __bf16* gu, __bf16* out, int rows, int ffn,
                                                          int out_tiled) {
  const long long vecs = (long long)rows * (ffn / 8);
  for (long long e = blockIdx.x * 256LL + threadIdx.x; e < vecs; e += (long long)gridDim.x * 256) {
    const int r = (int)(e / (ffn / 8)), f = (int)(e % (ffn / 8)) * 8;
    const bf16x8 g = *reinterpret_cast<const bf16x8*>(gu + (long long)r * 2 * ffn + f);
    const bf16x8 u = *reinterpret_cast<const bf16x8*>(gu + (long long)r * 2 * ffn + ffn + f);
    bf16x8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float gv = bf(g[j]);
      o[j] = (__bf16)((gv / (1.f + __expf(-gv))) * bf(u[j]));
    }
    *reinterpret_cast<bf16x8*>(out + (out_tiled ? tiled_row_offset(r, f) : (long long)r * ffn + f)) = o;
  }
}

// dst[b][h][:] = Meta-interleaved RoPE of src[b * stride + h * 128 ...] at position pos[b] (clamped into
// the table): pairs (2i, 2i+1) -> (x0 c - x1 s, x1 c + x0 s) with c = cos[p][2i], s = sin[p][2i].
// One thread per (row, head, 8 dims).
__global__ __launch_bounds__(256) void palu_rope_rows_kernel(const __bf16* src, long long stride, __bf16* dst,
                                                             const int32_t* pos, const float* cos_t, const float* sin_t,
                                                             int table_rows, int rows, int heads) {
  const long long vecs = (long long)rows * heads * (HD / 8);
  for (long long e = blockIdx.x * 256LL + threadIdx.x; e < vecs; e += (long long)gridDim.x * 256) {
    const int d8 = (int)(e % (HD / 8)) * 8;
    const long long bh = e / (HD / 8);
    const int h = (int)(bh % heads), b = (int)(bh / heads);
    int p = pos[b];
    p = p < 0 ? 0 : (p >= table_rows ? table_rows - 1 : p);
    const bf16x8 x = *reinterpret_cast<const bf16x8*>(src + b * stride + (long long)h * HD + d8);
    const float4 c0 = *reinterpret_cast<const float4*>(cos_t + (long long)p * HD + d8);
    const float4 c1 = *reinterpret_cast<const float4*>(cos_t + (long long)p * HD + d8 + 4);
    const float4 s0 = *reinterpret_cast<const float4*>(sin_t + (long long)p * HD + d8);
    const float4 s1 = *reinterpret_cast<const float4*>(sin_t + (long long)p * HD + d8 + 4);
    const float c[4] = {c0.x, c0.z, c1.x, c1.z}, s[4] = {s0.x, s0.z, s1.x, s1.z};
    bf16x8 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float x0 = bf(x[2 * i]), x1 = bf(x[2 * i + 1]);
      o[2 * i] = (__bf16)(x0 * c[i] - x1 * s[i]);
      o[2 * i + 1] = (__bf16)(x1 * c[i] + x0 * s[i]);
    }
    *reinterpret_cast<bf16x8*>(dst + bh * HD + d8) = o;
  }
}

int grid_for(long long work) {
  long long blocks = (work + 255) / 256;
  return (int)(blocks > 8192 ? 8192 : (blocks < 1 ? 1 : blocks));
}

inline bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int launched(const char* what) {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? PALU_OK : fail(PALU_EHIP, "%s launch: %s", what, hipGetErrorString(e));
}

}  // namespace

extern "C" {

int palu_rmsnorm(const void* x, const void* res, const float* res_part, int res_ks, void* h_out, void* y_out,
                 const void* weight, int rows, int dim, float eps, int y_tiled, hipStream_t stream) {
  palu::g_err[0] = 0;
  if (!x || !y_out || !weight) return fail(PALU_EINVAL, "palu_rmsnorm: a required pointer is null");
  if (rows <= 0 || dim <= 0 || dim % 8 != 0 || dim > RMS_THREADS * 8 * RMS_VEC)
    return fail(PALU_EINVAL, "palu_rmsnorm: dim must be a multiple of 8 up to %d, got %d", RMS_THREADS * 8 * RMS_VEC, dim);
  if (y_tiled && (rows > 64 || dim % 32 != 0))
    return fail(PALU_EINVAL, "palu_rmsnorm: a tiled output needs rows <= 64 and dim a multiple of 32, got %d x %d", rows, dim);
  if (res && res_part) return fail(PALU_EINVAL, "palu_rmsnorm: res and res_part are exclusive");
  if (res_part && (res_ks < 1 || res_ks > 64))
    return fail(PALU_EINVAL, "palu_rmsnorm: res_ks = %d partial slices (1..64)", res_ks);
  if (!a16(x) || !a16(y_out) || !a16(weight) || (res && !a16(res)) || (h_out && !a16(h_out)) ||
      (res_part && !a16(res_part)))
    return fail(PALU_EINVAL, "palu_rmsnorm: 16-byte alignment required");
  hipLaunchKernelGGL(palu_rmsnorm_kernel, dim3(rows), dim3(RMS_THREADS), 0, stream, static_cast<const __bf16*>(x),
                     static_cast<const __bf16*>(res), res_part, res_part ? res_ks : 0, (long long)rows * dim,
                     static_cast<__bf16*>(h_out), static_cast<__bf16*>(y_out), static_cast<const __bf16*>(weight), dim,
                     eps, y_tiled ? 1 : 0);
  return launched("palu_rmsnorm");
}
int palu_argmax_rows(const void* x, long long ld, int rows, int n, int64_t* out, hipStream_t stream) {
  palu::g_err[0] = 0;
  if (!x || !out) return fail(PALU_EINVAL, "palu_argmax_rows: a required pointer is null");
  if (rows <= 0 || rows > 65535 || n <= 0 || ld < n || ld % 8 != 0)
    return fail(PALU_EINVAL, "palu_argmax_rows: rows %d (1..65535), n %d and a row stride %lld >= n, a multiple of 8",
                rows, n, ld);
  if (!a16(x)) return fail(PALU_EINVAL, "palu_argmax_rows: 16-byte alignment required");
  hipLaunchKernelGGL(palu_argmax_kernel, dim3(rows), dim3(ARG_THREADS), 0, stream, static_cast<const __bf16*>(x), ld, n,
                     out);
  return launched("palu_argmax_rows");
}

int palu_swiglu(const void* gu, void* out, int rows, int ffn, int out_tiled, hipStream_t stream) {
  palu::g_err[0] = 0;
  if (!gu || !out) return fail(PALU_EINVAL, "palu_swiglu: a required pointer is null");
  if (rows <= 0 || ffn <= 0 || ffn % 8 != 0) return fail(PALU_EINVAL, "palu_swiglu: ffn must be a multiple of 8, got %d", ffn);
  if (out_tiled && (rows > 64 || ffn % 32 != 0))
    return fail(PALU_EINVAL, "palu_swiglu: a tiled output needs rows <= 64 and ffn a multiple of 32, got %d x %d", rows, ffn);
  if (!a16(gu) || !a16(out)) return fail(PALU_EINVAL, "palu_swiglu: 16-byte alignment required");
  hipLaunchKernelGGL(palu_swiglu_kernel, dim3(grid_for((long long)rows * (ffn / 8))), dim3(256), 0, stream,
                     static_cast<const __bf16*>(gu), static_cast<__bf16*>(out), rows, ffn, out_tiled ? 1 : 0);
  return launched("palu_swiglu");
}

int palu_rope_rows(const void* src, long long src_row_stride, void* dst, const int32_t* pos, const float* cos_table,
                   const float* sin_table, int table_rows, int rows, int heads, hipStream_t stream) {
  palu::g_err[0] = 0;
  if (!src || !dst || !pos || !cos_table || !sin_table) return fail(PALU_EINVAL, "palu_rope_rows: a required pointer is null");
  if (rows <= 0 || heads <= 0 || table_rows <= 0) return fail(PALU_EINVAL, "palu_rope_rows: sizes must be positive");
  if (src_row_stride < (long long)heads * HD || src_row_stride % 8 != 0)
    return fail(PALU_EINVAL, "palu_rope_rows: row stride %lld must be a multiple of 8 and hold %d heads", src_row_stride, heads);
  if (!a16(src) || !a16(dst) || !a16(cos_table) || !a16(sin_table))
    return fail(PALU_EINVAL, "palu_rope_rows: 16-byte alignment required");
  hipLaunchKernelGGL(palu_rope_rows_kernel, dim3(grid_for((long long)rows * heads * (HD / 8))), dim3(256), 0, stream,
                     static_cast<const __bf16*>(src), src_row_stride, static_cast<__bf16*>(dst), pos, cos_table,
                     sin_table, table_rows, rows, heads);
  return launched("palu_rope_rows");
}

}  // extern "C"
