// Device-resident steps of the dense transformer block around the quantized projections
// (src/forward.rs:100-586, src/infer.rs:72-223, src/runner.rs:105-282): RMS-norm, NeoX RoPE,
// K/V cache append, causal GQA attention, residual/bias add, SwiGLU, argmax, embedding gather.
// Positions come from a device integer so that one captured graph serves every decode step.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "kernels.hpp"

namespace rehip {

// block-wide reductions for 256-thread workgroups (fixed tree: deterministic)
__device__ __forceinline__ float block_sum256(float v, float* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}
__device__ __forceinline__ float block_max256(float v, float* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// out = x * (1 / sqrt(mean(x^2) + eps)) * w, one workgroup per row (infer.rs:72-82)
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                      int d, float eps, float* __restrict__ out) {
  __shared__ float red[4];
  const float* xr = x + (size_t)blockIdx.x * d;
  float s = 0.0f;
  for (int i = threadIdx.x; i < d; i += 256) s = __builtin_fmaf(xr[i], xr[i], s);
  s = block_sum256(s, red);
  const float inv = 1.0f / sqrtf(s / (float)d + eps);
  float* o = out + (size_t)blockIdx.x * d;
  for (int i = threadIdx.x; i < d; i += 256) o[i] = xr[i] * inv * w[i];
}

// NeoX rotate-half of head h of row r at position *pos + off + r (infer.rs:90-139):
// angle = p * base^(-2i/d); (x0, x1) -> (x0 c - x1 s, x1 c + x0 s)
__global__ __launch_bounds__(64) void rope_kernel(float* __restrict__ x, int heads, int hd, float base,
                                                  const int* __restrict__ pos, int off) {
  const int r = blockIdx.y, h = blockIdx.x, i = threadIdx.x;
  const int half = hd >> 1;
  if (i >= half) return;
  const float p = (float)(*pos + off + r);
  const float f = 1.0f / powf(base, (float)(2 * i) / (float)hd);
  const float a = p * f;
  const float c = cosf(a), s = sinf(a);
  float* v = x + ((size_t)r * heads + h) * hd;
  const float x0 = v[i], x1 = v[i + half];
  v[i] = x0 * c - x1 * s;
  v[i + half] = x1 * c + x0 * s;
}

__global__ __launch_bounds__(256) void kv_append_kernel(const float* __restrict__ k, const float* __restrict__ v,
                                                        int kv_dim, float* __restrict__ kc, float* __restrict__ vc,
                                                        int max_seq, const int* __restrict__ pos) {
  const int r = blockIdx.x;
  const int row = *pos + r;
  if (row < 0 || row >= max_seq) return;
  const size_t dst = (size_t)row * kv_dim;
  for (int i = threadIdx.x; i < kv_dim; i += 256) {
    kc[dst + i] = k[(size_t)r * kv_dim + i];
    vc[dst + i] = v[(size_t)r * kv_dim + i];
  }
}

// Causal GQA attention (forward.rs:232-277, 437-470): query row r at position p = *pos + r
// attends to cache rows 0..p with scores q.k * (1/sqrt(hd)), softmax as moe.rs:61-72 (exp of
// x - max, divided by the sum when it is non-zero), then the probability-weighted values.
// Cache rows past the last visible one are never read (loads clamp to it), so rows of the cache
// that were never written do not enter the result.

// v of lane (lane ^ OFF) without the LDS pipe: v_permlane32_swap / v_permlane16_swap exchange
// 32- / 16-lane halves (each returns both halves; the lane keeps the one that came from its
// partner), DPP row moves do the rest (row_ror:8 = xor 8 within a 16-lane row, quad_perm
// [3,2,1,0] then row_half_mirror = xor 4, quad_perm [2,3,0,1] / [1,0,3,2] = xor 2 / xor 1).
// The pairs are those of __shfl_xor(v, OFF, 64), so a butterfly over them keeps its bits.
template <int OFF>
__device__ __forceinline__ float lane_xor(float v) {
  const int u = __float_as_int(v);
  if constexpr (OFF == 32) {
    const auto s = __builtin_amdgcn_permlane32_swap((unsigned)u, (unsigned)u, false, false);
    return __uint_as_float((threadIdx.x & 32) ? s[0] : s[1]);
  } else if constexpr (OFF == 16) {
    const auto s = __builtin_amdgcn_permlane16_swap((unsigned)u, (unsigned)u, false, false);
    return __uint_as_float((threadIdx.x & 16) ? s[0] : s[1]);
  } else if constexpr (OFF == 8) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, u, 0x128, 0xF, 0xF, false));
  } else if constexpr (OFF == 4) {
    const int r = __builtin_amdgcn_update_dpp(0, u, 0x1B, 0xF, 0xF, false);
    return __int_as_float(__builtin_amdgcn_update_dpp(0, r, 0x141, 0xF, 0xF, false));
  } else if constexpr (OFF == 2) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, u, 0x4E, 0xF, 0xF, false));
  } else {
    static_assert(OFF == 1, "lane_xor: OFF is a power of two up to 32");
    return __int_as_float(__builtin_amdgcn_update_dpp(0, u, 0xB1, 0xF, 0xF, false));
  }
}
// butterfly max / sum over the wave (every lane ends with the result), pairs xor 32, 16, .., 1
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, lane_xor<32>(v));
  v = fmaxf(v, lane_xor<16>(v));
  v = fmaxf(v, lane_xor<8>(v));
  v = fmaxf(v, lane_xor<4>(v));
  v = fmaxf(v, lane_xor<2>(v));
  return fmaxf(v, lane_xor<1>(v));
}
__device__ __forceinline__ float wave_sum(float v) {
  v += lane_xor<32>(v);
  v += lane_xor<16>(v);
  v += lane_xor<8>(v);
  v += lane_xor<4>(v);
  v += lane_xor<2>(v);
  return v + lane_xor<1>(v);
}

// Few rows (decode), or head sizes other than 64: one 1024-thread workgroup per (query head,
// row). A team of 16 lanes owns one key (a float4 of dimensions per lane and 64-dimension slot,
// NC slots); the 64 teams cover 64 * U keys per pass with all U * NC loads of a lane in flight.
// Scores go to LDS (max_seq floats); the p * v pass uses the same teams, and the 16 waves'
// partials are folded in a fixed order.
constexpr int kAttnRowsThreads = 1024;

template <int NC>
__global__ __launch_bounds__(kAttnRowsThreads) void attention_rows_kernel(
    const float* __restrict__ q, const float* __restrict__ kc, const float* __restrict__ vc, int heads, int kv_heads,
    int hd, int max_seq, const int* __restrict__ pos, float* __restrict__ ctx) {
  constexpr int U = 16 / NC;             // keys per team per pass
  extern __shared__ __attribute__((aligned(16))) float sc[];   // scores[(max_seq + 3) & ~3], 16 x hd partials
  __shared__ float red[16];
  const int h = blockIdx.x, r = blockIdx.y;
  const int kvh = h / (heads / kv_heads);
  const int kv_dim = kv_heads * hd;
  const int L = min(max(*pos + r + 1, 1), max_seq);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int team = 4 * w + (lane >> 4), tl = lane & 15;
  const float* qh = q + ((size_t)r * heads + h) * hd;
  float4 qv[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int d = 4 * tl + 64 * c;
    qv[c] = d < hd ? *reinterpret_cast<const float4*>(qh + d) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const float scale = 1.0f / sqrtf((float)hd);
  const float* kbase = kc + (size_t)kvh * hd;
  const float* vbase = vc + (size_t)kvh * hd;
  float mx = -INFINITY;
  for (int base = 0; base < L; base += 64 * U) {
    float4 kv[U][NC];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float* kr = kbase + (size_t)min(base + 64 * u + team, L - 1) * kv_dim;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int d = 4 * tl + 64 * c;
        kv[u][c] = d < hd ? *reinterpret_cast<const float4*>(kr + d) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float a = 0.0f;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        a = __builtin_fmaf(qv[c].x, kv[u][c].x, a);
        a = __builtin_fmaf(qv[c].y, kv[u][c].y, a);
        a = __builtin_fmaf(qv[c].z, kv[u][c].z, a);
        a = __builtin_fmaf(qv[c].w, kv[u][c].w, a);
      }
#pragma unroll
      for (int off = 8; off > 0; off >>= 1) a += __shfl_xor(a, off, 64);
      const int j = base + 64 * u + team;
      if (tl == 0 && j < L) {
        const float v = a * scale;
        sc[j] = v;
        mx = fmaxf(mx, v);
      }
    }
  }
  mx = wave_max(mx);
  __syncthreads();
  if (lane == 0) red[w] = mx;
  __syncthreads();
  mx = red[0];
#pragma unroll
  for (int i = 1; i < 16; ++i) mx = fmaxf(mx, red[i]);
  float sum = 0.0f;
  for (int j = threadIdx.x; j < L; j += kAttnRowsThreads) {
    const float e = expf(sc[j] - mx);
    sc[j] = e;
    sum += e;
  }
  sum = wave_sum(sum);
  __syncthreads();
  if (lane == 0) red[w] = sum;
  __syncthreads();
  sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) sum += red[i];
  const float inv = sum != 0.0f ? 1.0f / sum : 1.0f;
  float4 acc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) acc[c] = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int base = 0; base < L; base += 64 * U) {
    float4 vv[U][NC];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float* vr = vbase + (size_t)min(base + 64 * u + team, L - 1) * kv_dim;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int d = 4 * tl + 64 * c;
        vv[u][c] = d < hd ? *reinterpret_cast<const float4*>(vr + d) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = base + 64 * u + team;
      const float p = j < L ? sc[j] * inv : 0.0f;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        acc[c].x = __builtin_fmaf(p, vv[u][c].x, acc[c].x);
        acc[c].y = __builtin_fmaf(p, vv[u][c].y, acc[c].y);
        acc[c].z = __builtin_fmaf(p, vv[u][c].z, acc[c].z);
        acc[c].w = __builtin_fmaf(p, vv[u][c].w, acc[c].w);
      }
    }
  }
  // fold the four teams of the wave (fixed xor tree), then the 16 waves in order
#pragma unroll
  for (int c = 0; c < NC; ++c) {
#pragma unroll
    for (int off = 16; off < 64; off <<= 1) {
      acc[c].x += __shfl_xor(acc[c].x, off, 64);
      acc[c].y += __shfl_xor(acc[c].y, off, 64);
      acc[c].z += __shfl_xor(acc[c].z, off, 64);
      acc[c].w += __shfl_xor(acc[c].w, off, 64);
    }
  }
  float* part = sc + ((max_seq + 3) & ~3);
  if ((lane >> 4) == 0) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d = 4 * tl + 64 * c;
      if (d < hd) *reinterpret_cast<float4*>(part + w * hd + d) = acc[c];
    }
  }
  __syncthreads();
  float* out = ctx + ((size_t)r * heads + h) * hd;
  for (int d = threadIdx.x; d < hd; d += kAttnRowsThreads) {
    float o = part[d];
#pragma unroll
    for (int i = 1; i < 16; ++i) o += part[i * hd + d];
    out[d] = o;
  }
}

// Few rows with a workspace: the cache is cut into kAttnSplitKeys-key splits, one 256-thread
// workgroup per (query head, row, split) -- so a decode step spreads over heads * splits CUs
// instead of heads -- each writing (max m, sum l of exp(s - m), sum of exp(s - m) * v) for its
// keys; a second kernel combines the splits in split order:
//   M = max m_s, L = sum l_s exp(m_s - M), out = sum acc_s exp(m_s - M) / L.
// Splits past the visible keys write m = -inf and are skipped.
constexpr int kAttnSplitKeys = 128;      // 16 teams x 8 keys
constexpr int kAttnMaxSplits = 256;      // 32768 cache rows

// One decode row's q|k|v epilogue folded into the key-split attention (attention_decode): the
// projection outputs are raw (no bias, not rotated); each workgroup rotates its q head itself,
// and the split holding the new key position rotates k and biases v for its kv head, uses them
// for that key, and (the first q head of the kv group only) appends them to the caches. No other
// split reads that cache row in this launch, so there is no ordering between workgroups.
struct DecodeQkv {
  const float* ks;      // raw k of the row (kv_heads x hd), ks/vs strided like q
  const float* vs;
  const float* bq;      // biases or null
  const float* bk;
  const float* bv;
  float base;           // RoPE theta
  float* kc_out;        // caches, written at row *pos
  float* vc_out;
  const float2* rope;   // null, or (cos, sin) of every pair at positions 0 .. rope_rows - 1
  int rope_rows;
};

// NeoX rotation of the pair (x0, x1) = (x[i], x[i + hd/2]) at position p (infer.rs:90-139): the
// angle's cosine and sine, and the rotation. Shared by qkv_rope_append_kernel, the folded decode
// epilogue and rope_table_kernel, so every path gives the same bits.
__device__ __forceinline__ void rope_cs(int i, int hd, int p, float base, float& c, float& sn) {
  const float f = 1.0f / powf(base, (float)(2 * i) / (float)hd);
  const float a = (float)p * f;
  c = cosf(a);
  sn = sinf(a);
}
__device__ __forceinline__ void rope_rot(float x0, float x1, float c, float sn, float& o0, float& o1) {
  o0 = x0 * c - x1 * sn;
  o1 = x1 * c + x0 * sn;
}
__device__ __forceinline__ void rope_pair(float x0, float x1, int i, int hd, int p, float base, float& o0, float& o1) {
  float c, sn;
  rope_cs(i, hd, p, base, c, sn);
  rope_rot(x0, x1, c, sn, o0, o1);
}

// tab[p * hd/2 + i] = (cos, sin) of pair i's angle at position p, for p < rows
__global__ __launch_bounds__(256) void rope_table_kernel(float base, int hd, int rows, float2* __restrict__ tab) {
  const int half = hd >> 1;
  const size_t n = (size_t)rows * (size_t)half;
  for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (size_t)gridDim.x * 256) {
    const int p = (int)(e / (size_t)half), i = (int)(e - (size_t)p * (size_t)half);
    float c, sn;
    rope_cs(i, hd, p, base, c, sn);
    tab[e] = make_float2(c, sn);
  }
}

// Dims d .. d + 3 of a rotated head vector from the raw ones (own), their rotation partners
// (par, at d + hd/2 when lo, else d - hd/2) and the (cos, sin) of pairs i .. i + 3
// (cs0 = pairs i, i + 1; cs1 = i + 2, i + 3): the x0 side of each pair when lo, else the x1 side.
__device__ __forceinline__ float4 rope4(float4 own, float4 par, float4 cs0, float4 cs1, bool lo) {
  const float o[4] = {own.x, own.y, own.z, own.w}, q[4] = {par.x, par.y, par.z, par.w};
  const float c[4] = {cs0.x, cs0.z, cs1.x, cs1.z}, sn[4] = {cs0.y, cs0.w, cs1.y, cs1.w};
  float r[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float o0, o1;
    if (lo) {
      rope_rot(o[j], q[j], c[j], sn[j], o0, o1);
      r[j] = o0;
    } else {
      rope_rot(q[j], o[j], c[j], sn[j], o0, o1);
      r[j] = o1;
    }
  }
  return make_float4(r[0], r[1], r[2], r[3]);
}
__device__ __forceinline__ float4 add4(float4 a, float4 b) { return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w); }

// TAB (with QKV, hd % 8 == 0, dq.rope given): each lane rotates its own dims of q, and the team
// holding the new key those of k, in registers with the table's (cos, sin); no LDS pass or barrier
// comes before the scores.
// FULL: hd == 64 NC, so every lane's dims are inside the head and the K/V loads need no guard (a
// guarded load is a branch, and the compiler then waited for every K load before issuing the V
// loads: two memory round trips instead of one)
template <int NC, bool QKV, bool TAB = false, bool FULL = false>   // kc / vc are not __restrict__: with QKV the new row is stored through dq
__global__ __launch_bounds__(256) void attention_split_kernel(const float* __restrict__ q, const float* kc,
                                                              const float* vc, int heads, int kv_heads,
                                                              int hd, int max_seq, const int* __restrict__ pos,
                                                              float* __restrict__ work, DecodeQkv dq) {
  constexpr int U = 8;
  __shared__ float sc[kAttnSplitKeys];
  __shared__ float red[4];
  __shared__ __attribute__((aligned(16))) float part[4 * 256];
  const int h = blockIdx.x, r = blockIdx.y, sp = blockIdx.z, nsp = gridDim.z;
  const int kvh = h / (heads / kv_heads);
  const int kv_dim = kv_heads * hd;
  const int p0 = *pos;
  const int L = min(max(p0 + r + 1, 1), max_seq);
  const int j0 = sp * kAttnSplitKeys;
  float* wp = work + (((size_t)r * heads + h) * nsp + sp) * (hd + 2);
  if (j0 >= L) {                         // nothing visible in this split
    if (threadIdx.x == 0) { wp[0] = -INFINITY; wp[1] = 0.0f; }
    return;
  }
  const int jn = min(kAttnSplitKeys, L - j0);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int team = 4 * w + (lane >> 4), tl = lane & 15;
  const float scale = 1.0f / sqrtf((float)hd);
  const float* kbase = kc + (size_t)kvh * hd;
  const float* vbase = vc + (size_t)kvh * hd;
  // QKV: the split holding key p0 (< max_seq) also builds the new key and value. Thread t < hd/2
  // takes rotation pair t of q (and of k), thread t < hd element t of v; their inputs are loaded
  // before the K/V rows so that the epilogue waits for them alone.
  const bool has_new = QKV && p0 >= 0 && p0 < max_seq && p0 >= j0 && p0 < j0 + jn;
  const int half = hd >> 1, t = threadIdx.x;
  float qx0 = 0.0f, qx1 = 0.0f, kx0 = 0.0f, kx1 = 0.0f, vx = 0.0f;
  // keys j0 + 16 u + team, u < U: all loads of K and V issued first, ahead of the epilogue's
  // (whose bias and table loads sit under branches, after which the compiler waits for every
  // load issued so far: issued later, K and V took a second memory round trip). With QKV the new
  // key's row, not yet written, is replaced after the epilogue.
  float4 kv[U][NC], vv[U][NC];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const size_t row = (size_t)(j0 + min(16 * u + team, jn - 1)) * kv_dim;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d = 4 * tl + 64 * c;
      kv[u][c] = FULL || d < hd ? *reinterpret_cast<const float4*>(kbase + row + d) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const size_t row = (size_t)(j0 + min(16 * u + team, jn - 1)) * kv_dim;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d = 4 * tl + 64 * c;
      vv[u][c] = FULL || d < hd ? *reinterpret_cast<const float4*>(vbase + row + d) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  // TAB: raw q of this lane's dims and their partners (biased), the new key's and value's (every
  // team of the split holding key p0: teams past the split's last key, jn - 1, read that row too),
  // and the (cos, sin) of their pairs
  float4 tq[NC], tqp[NC], tk[NC], tkp[NC], tv[NC], tc0[NC], tc1[NC];
  const bool newteam = TAB && has_new;
  if constexpr (TAB) {
    const bool from_tab = p0 >= 0 && p0 < dq.rope_rows;
    const int prow = from_tab ? p0 : 0;  // a position past the table reads row 0 (not used)
    const float* qr = q + (size_t)h * hd;
    const float* kr = dq.ks + (size_t)kvh * hd;
    const float* vr = dq.vs + (size_t)kvh * hd;
    // an absent bias reads its row instead (readable; the values are not used)
    const float* bqr = dq.bq ? dq.bq + (size_t)h * hd : qr;
    const float* bkr = dq.bk ? dq.bk + (size_t)kvh * hd : kr;
    const float* bvr = dq.bv ? dq.bv + (size_t)kvh * hd : vr;
    float4 bq0[NC], bq1[NC], bk0[NC], bk1[NC], bv0[NC];
    // every load first and none under a branch: after a branch the compiler waited for all the
    // loads issued so far, one memory round trip per branch
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d = 4 * tl + 64 * c;
      const int dd = d < hd ? d : 0;
      const bool lo = dd < half;
      const int dp = lo ? dd + half : dd - half, i0 = lo ? dd : dd - half;
      tq[c] = *reinterpret_cast<const float4*>(qr + dd);
      tqp[c] = *reinterpret_cast<const float4*>(qr + dp);
      bq0[c] = *reinterpret_cast<const float4*>(bqr + dd);
      bq1[c] = *reinterpret_cast<const float4*>(bqr + dp);
      const float2* cs = dq.rope + (size_t)prow * half + i0;
      tc0[c] = *reinterpret_cast<const float4*>(cs);
      tc1[c] = *reinterpret_cast<const float4*>(cs + 2);
      tk[c] = *reinterpret_cast<const float4*>(kr + dd);
      tkp[c] = *reinterpret_cast<const float4*>(kr + dp);
      tv[c] = *reinterpret_cast<const float4*>(vr + dd);
      bk0[c] = *reinterpret_cast<const float4*>(bkr + dd);
      bk1[c] = *reinterpret_cast<const float4*>(bkr + dp);
      bv0[c] = *reinterpret_cast<const float4*>(bvr + dd);
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if (dq.bq) {
        tq[c] = add4(tq[c], bq0[c]);
        tqp[c] = add4(tqp[c], bq1[c]);
      }
      if (!from_tab) {                   // a position past the table: computed here
        const int d = 4 * tl + 64 * c;
        const int dd = d < hd ? d : 0;
        const int i0 = dd < half ? dd : dd - half;
        float cv[4], sv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) rope_cs(i0 + j, hd, p0, dq.base, cv[j], sv[j]);
        tc0[c] = make_float4(cv[0], sv[0], cv[1], sv[1]);
        tc1[c] = make_float4(cv[2], sv[2], cv[3], sv[3]);
      }
      if (dq.bk) {                       // (the new key and value are used by the new team only)
        tk[c] = add4(tk[c], bk0[c]);
        tkp[c] = add4(tkp[c], bk1[c]);
      }
      if (dq.bv) tv[c] = add4(tv[c], bv0[c]);
    }
  } else if constexpr (QKV) {
    if (t < half) {
      const float* qr = q + (size_t)h * hd;
      qx0 = qr[t];
      qx1 = qr[t + half];
      if (dq.bq) {
        qx0 += dq.bq[(size_t)h * hd + t];
        qx1 += dq.bq[(size_t)h * hd + t + half];
      }
      if (has_new) {
        const float* kr = dq.ks + (size_t)kvh * hd;
        kx0 = kr[t];
        kx1 = kr[t + half];
        if (dq.bk) {
          kx0 += dq.bk[(size_t)kvh * hd + t];
          kx1 += dq.bk[(size_t)kvh * hd + t + half];
        }
      }
    }
    if (has_new && t < hd) vx = dq.bv ? dq.vs[(size_t)kvh * hd + t] + dq.bv[(size_t)kvh * hd + t] : dq.vs[(size_t)kvh * hd + t];
  }
  float4 qv[NC];
  if constexpr (TAB) {
    // the kv group's first q head appends, from the team whose own key is p0
    const bool app = newteam && team == ((jn - 1) & 15) && h % (heads / kv_heads) == 0;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d = 4 * tl + 64 * c;
      const bool lo = d < half;
      qv[c] = d < hd ? rope4(tq[c], tqp[c], tc0[c], tc1[c], lo) : make_float4(0.f, 0.f, 0.f, 0.f);
      if (newteam && d < hd) {
        const float4 kn = rope4(tk[c], tkp[c], tc0[c], tc1[c], lo);
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if (j0 + min(16 * u + team, jn - 1) == p0) {   // the row read for key p0 (or past it)
            kv[u][c] = kn;
            vv[u][c] = tv[c];
          }
        }
        if (app) {
          *reinterpret_cast<float4*>(dq.kc_out + (size_t)p0 * kv_dim + (size_t)kvh * hd + d) = kn;
          *reinterpret_cast<float4*>(dq.vc_out + (size_t)p0 * kv_dim + (size_t)kvh * hd + d) = tv[c];
        }
      }
    }
  }
  // QKV: rotated q in part[0..hd), the new key and value in part[256..256+hd), part[512..512+hd)
  if constexpr (QKV && !TAB) {
    if (t < half) {
      rope_pair(qx0, qx1, t, hd, p0, dq.base, part[t], part[t + half]);
      if (has_new) rope_pair(kx0, kx1, t, hd, p0, dq.base, part[256 + t], part[256 + t + half]);
    }
    if (has_new && t < hd) part[512 + t] = vx;
    __syncthreads();
    if (has_new && h % (heads / kv_heads) == 0) {
      for (int i = threadIdx.x; i < hd; i += 256) {
        dq.kc_out[(size_t)p0 * kv_dim + (size_t)kvh * hd + i] = part[256 + i];
        dq.vc_out[(size_t)p0 * kv_dim + (size_t)kvh * hd + i] = part[512 + i];
      }
    }
  }
  if constexpr (!TAB) {
    const float* qh = QKV ? part : q + ((size_t)r * heads + h) * hd;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d = 4 * tl + 64 * c;
      qv[c] = d < hd ? *reinterpret_cast<const float4*>(qh + d) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  if (!TAB && has_new) {                 // the new key is the split's last: from LDS, not the cache
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (j0 + min(16 * u + team, jn - 1) == p0) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const int d = 4 * tl + 64 * c;
          if (d < hd) {
            kv[u][c] = *reinterpret_cast<const float4*>(part + 256 + d);
            vv[u][c] = *reinterpret_cast<const float4*>(part + 512 + d);
          }
        }
      }
    }
  }
  // the U keys' dots, then their team reductions interleaved (no key's shuffle rounds wait on
  // another's); each key's terms add in the same order either way
  float a[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    a[u] = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      a[u] = __builtin_fmaf(qv[c].x, kv[u][c].x, a[u]);
      a[u] = __builtin_fmaf(qv[c].y, kv[u][c].y, a[u]);
      a[u] = __builtin_fmaf(qv[c].z, kv[u][c].z, a[u]);
      a[u] = __builtin_fmaf(qv[c].w, kv[u][c].w, a[u]);
    }
  }
#pragma unroll
  for (int off = 8; off > 0; off >>= 1)
#pragma unroll
    for (int u = 0; u < U; ++u) a[u] += __shfl_xor(a[u], off, 64);
  float mx = -INFINITY;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int jj = 16 * u + team;
    if (tl == 0 && jj < jn) {
      const float v = a[u] * scale;
      sc[jj] = v;
      mx = fmaxf(mx, v);
    }
  }
  mx = wave_max(mx);
  if (lane == 0) red[w] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float4 acc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) acc[c] = make_float4(0.f, 0.f, 0.f, 0.f);
  float lsum = 0.0f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int jj = 16 * u + team;
    const float e = jj < jn ? expf(sc[jj] - mx) : 0.0f;
    lsum += e;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      acc[c].x = __builtin_fmaf(e, vv[u][c].x, acc[c].x);
      acc[c].y = __builtin_fmaf(e, vv[u][c].y, acc[c].y);
      acc[c].z = __builtin_fmaf(e, vv[u][c].z, acc[c].z);
      acc[c].w = __builtin_fmaf(e, vv[u][c].w, acc[c].w);
    }
  }
  // lsum: every lane of a team holds its team's sum; fold teams of the wave, then the waves
#pragma unroll
  for (int off = 16; off < 64; off <<= 1) lsum += __shfl_xor(lsum, off, 64);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
#pragma unroll
    for (int off = 16; off < 64; off <<= 1) {
      acc[c].x += __shfl_xor(acc[c].x, off, 64);
      acc[c].y += __shfl_xor(acc[c].y, off, 64);
      acc[c].z += __shfl_xor(acc[c].z, off, 64);
      acc[c].w += __shfl_xor(acc[c].w, off, 64);
    }
  }
  __syncthreads();                       // red[] reused
  if (lane == 0) red[w] = lsum;
  if ((lane >> 4) == 0) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d = 4 * tl + 64 * c;
      if (d < hd) *reinterpret_cast<float4*>(part + w * 256 + d) = acc[c];
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    wp[0] = mx;
    wp[1] = ((red[0] + red[1]) + red[2]) + red[3];
  }
  for (int d = threadIdx.x; d < hd; d += 256)
    wp[2 + d] = ((part[d] + part[256 + d]) + part[512 + d]) + part[768 + d];
}

__global__ __launch_bounds__(64) void attention_combine_kernel(const float* __restrict__ work, int heads, int hd,
                                                               int nsp, float* __restrict__ ctx) {
  __shared__ float f[kAttnMaxSplits];
  const int h = blockIdx.x, r = blockIdx.y, t = threadIdx.x;
  const size_t st = (size_t)hd + 2;
  const float* wp = work + ((size_t)r * heads + h) * nsp * st;
  // every split's (m, l) loaded in parallel (lane t: splits t, t + 64, ..)
  float mv[kAttnMaxSplits / 64], lv[kAttnMaxSplits / 64];
  float M = -INFINITY;
  int nvis = 0;                          // splits with visible keys: a prefix (the others wrote
#pragma unroll                           // only m = -inf and l = 0, no values)
  for (int k = 0; k < kAttnMaxSplits / 64; ++k) {
    const int sp = t + 64 * k;
    mv[k] = sp < nsp ? wp[sp * st] : -INFINITY;
    lv[k] = sp < nsp ? wp[sp * st + 1] : 0.0f;
    M = fmaxf(M, mv[k]);
    if (mv[k] != -INFINITY) nvis = sp + 1;
  }
  M = wave_max(M);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) nvis = max(nvis, __shfl_xor(nvis, off, 64));
  float tot = 0.0f;
#pragma unroll
  for (int k = 0; k < kAttnMaxSplits / 64; ++k) {
    const int sp = t + 64 * k;
    const float fk = mv[k] == -INFINITY ? 0.0f : expf(mv[k] - M);
    if (sp < nsp) f[sp] = fk;
    tot = __builtin_fmaf(lv[k], fk, tot);
  }
  tot = wave_sum(tot);
  __syncthreads();
  const float inv = tot != 0.0f ? 1.0f / tot : 1.0f;
  float* out = ctx + ((size_t)r * heads + h) * hd;
  for (int d = t; d < hd; d += 64) {
    const float* a = wp + 2 + d;
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;    // four independent chains, folded in order
    int sp = 0;
    for (; sp + 4 <= nvis; sp += 4) {
      s0 = __builtin_fmaf(a[sp * st], f[sp], s0);
      s1 = __builtin_fmaf(a[(sp + 1) * st], f[sp + 1], s1);
      s2 = __builtin_fmaf(a[(sp + 2) * st], f[sp + 2], s2);
      s3 = __builtin_fmaf(a[(sp + 3) * st], f[sp + 3], s3);
    }
    for (; sp < nvis; ++sp) s0 = __builtin_fmaf(a[sp * st], f[sp], s0);
    out[d] = (((s0 + s1) + s2) + s3) * inv;
  }
}

size_t attention_work_floats(int rows, int heads, int hd, int max_seq) {
  const size_t nsp = ((size_t)max_seq + kAttnSplitKeys - 1) / kAttnSplitKeys;
  return (size_t)rows * heads * nsp * (hd + 2);
}

// Many rows, head size 64 (prefill): f32 MFMA flash attention. A workgroup owns 32 query
// vectors of one kv head (vector g = row * grp + head-in-group, so a block may cut across
// rows) and its four waves split the cache into 32-key blocks (wave w takes blocks w, w+4, ..).
// Per key block, in v_mfma_f32_32x32x2_f32 layout with lane l = (half h = l/32, column l%32):
//   S^T[key][vec] = K Q^T: A = K[key l%32][dim 32h + s], B = Q[vec l%32][dim 32h + s],
//     s = 0..31; register i of the result is key 8(i/4) + 4h + i%4 of vector l%32;
//   online softmax per vector (running max m, rescale of earlier terms by exp(m_old - m_new));
//   O^T[dim][vec] += V^T P^T: step s takes the key held in result register s, so the B operand
//     is that register and A = V[that key][dim l%32 + 32 nb].
// The four waves' (m, sum, O) are combined in LDS in wave order. K and V of the next key block
// are loaded while the current one is in the MFMAs. Row blocks run longest-first.
constexpr int kAttnMfmaVecs = 32;

__device__ __forceinline__ int attn_key_of(int i, int h) { return 8 * (i >> 2) + 4 * h + (i & 3); }

__global__ __launch_bounds__(256) void attention_mfma_kernel(const float* __restrict__ q, const float* __restrict__ kc,
                                                             const float* __restrict__ vc, int rows, int heads,
                                                             int kv_heads, int max_seq, const int* __restrict__ pos,
                                                             float* __restrict__ ctx) {
  constexpr int HD = 64;
  typedef float f32x16 __attribute__((ext_vector_type(16)));
  __shared__ __attribute__((aligned(16))) float Os[4][kAttnMfmaVecs][HD + 4];
  __shared__ float Ms[4][kAttnMfmaVecs], Ls[4][kAttnMfmaVecs];
  const int grp = heads / kv_heads;
  const int blk = gridDim.x - 1 - blockIdx.x, kvh = blockIdx.y;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int vl = lane & 31, h = lane >> 5;
  const int kv_dim = kv_heads * HD;
  const int p0 = *pos;
  const int g0 = blk * kAttnMfmaVecs;
  const int r_last = min((g0 + kAttnMfmaVecs - 1) / grp, rows - 1);
  const int jmax = min(p0 + r_last, max_seq - 1);
  const int nkb = jmax / 32 + 1;
  // this lane's query vector
  const int g = g0 + vl, r = g / grp, head = kvh * grp + g % grp;
  const bool valid = r < rows;
  const int limit = valid ? min(p0 + r, max_seq - 1) : -1;
  float qb[32];
  {
    const float* qr = q + ((size_t)(valid ? r : 0) * heads + (valid ? head : 0)) * HD + 32 * h;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const float4 x = valid ? *reinterpret_cast<const float4*>(qr + 4 * t) : make_float4(0.f, 0.f, 0.f, 0.f);
      qb[4 * t] = x.x;
      qb[4 * t + 1] = x.y;
      qb[4 * t + 2] = x.z;
      qb[4 * t + 3] = x.w;
    }
  }
  const float scale = 1.0f / sqrtf((float)HD);
  const float* kb = kc + (size_t)kvh * HD;
  const float* vb = vc + (size_t)kvh * HD;
  auto load = [&](int kbi, float (&kd)[32], float (&vd)[2][16]) {
    const float* kr = kb + (size_t)min(32 * kbi + vl, jmax) * kv_dim + 32 * h;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const float4 x = *reinterpret_cast<const float4*>(kr + 4 * t);
      kd[4 * t] = x.x;
      kd[4 * t + 1] = x.y;
      kd[4 * t + 2] = x.z;
      kd[4 * t + 3] = x.w;
    }
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const float* vr = vb + (size_t)min(32 * kbi + attn_key_of(s, h), jmax) * kv_dim + vl;
      vd[0][s] = vr[0];
      vd[1][s] = vr[32];
    }
  };
  float m = -INFINITY, l = 0.0f;
  f32x16 o0 = {}, o1 = {};
  auto step = [&](int kbi, const float (&kd)[32], const float (&vd)[2][16]) {
    f32x16 st = {};
#pragma unroll
    for (int s = 0; s < 32; ++s) st = __builtin_amdgcn_mfma_f32_32x32x2f32(kd[s], qb[s], st, 0, 0, 0);
    float sv[16], mloc = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int j = 32 * kbi + attn_key_of(i, h);
      sv[i] = j <= limit ? st[i] * scale : -INFINITY;
      mloc = fmaxf(mloc, sv[i]);
    }
    const float mn = fmaxf(m, fmaxf(mloc, __shfl_xor(mloc, 32, 64)));
    float pv[16];
    if (mn == -INFINITY) {               // nothing visible yet for this vector
#pragma unroll
      for (int i = 0; i < 16; ++i) pv[i] = 0.0f;
    } else {
      const float alpha = expf(m - mn);  // m = -inf gives 0
      float ps = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        pv[i] = expf(sv[i] - mn);
        ps += pv[i];
      }
      l = __builtin_fmaf(l, alpha, ps);
      o0 *= alpha;
      o1 *= alpha;
      m = mn;
    }
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(vd[0][s], pv[s], o0, 0, 0, 0);
      o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(vd[1][s], pv[s], o1, 0, 0, 0);
    }
  };
  // two register sets, alternating by hand (a runtime index into them would go to scratch)
  float kA[32], vA[2][16], kB[32], vB[2][16];
  if (w < nkb) load(w, kA, vA);
  for (int kbi = w; kbi < nkb; kbi += 8) {
    if (kbi + 4 < nkb) load(kbi + 4, kB, vB);
    step(kbi, kA, vA);
    if (kbi + 4 >= nkb) break;
    if (kbi + 8 < nkb) load(kbi + 8, kA, vA);
    step(kbi + 4, kB, vB);
  }
  // wave partials: O^T register i of block nb is dim 32 nb + 8(i/4) + 4h + i%4 of vector vl
  l += __shfl_xor(l, 32, 64);
#pragma unroll
  for (int i = 0; i < 16; i += 4) {
    const int d = attn_key_of(i, h);
    *reinterpret_cast<float4*>(&Os[w][vl][d]) = make_float4(o0[i], o0[i + 1], o0[i + 2], o0[i + 3]);
    *reinterpret_cast<float4*>(&Os[w][vl][32 + d]) = make_float4(o1[i], o1[i + 1], o1[i + 2], o1[i + 3]);
  }
  if (h == 0) {
    Ms[w][vl] = m;
    Ls[w][vl] = l;
  }
  __syncthreads();
  // combine: thread t -> vector t / 8, dims 8 (t % 8) .. + 7
  const int v = threadIdx.x >> 3, d0 = 8 * (threadIdx.x & 7);
  const int gv = g0 + v, rv = gv / grp;
  if (rv >= rows) return;
  float M = Ms[0][v];
#pragma unroll
  for (int k = 1; k < 4; ++k) M = fmaxf(M, Ms[k][v]);
  if (M == -INFINITY) return;            // unreachable for a valid vector (key 0 is visible)
  float f[4], tot = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    f[k] = Ms[k][v] == -INFINITY ? 0.0f : expf(Ms[k][v] - M);
    tot = __builtin_fmaf(Ls[k][v], f[k], tot);
  }
  const float inv = tot != 0.0f ? 1.0f / tot : 1.0f;
  float outv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float a = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) a = __builtin_fmaf(Os[k][v][d0 + e], f[k], a);
    outv[e] = a * inv;
  }
  float* out = ctx + ((size_t)rv * heads + kvh * grp + gv % grp) * HD + d0;
  *reinterpret_cast<float4*>(out) = make_float4(outv[0], outv[1], outv[2], outv[3]);
  *reinterpret_cast<float4*>(out + 4) = make_float4(outv[4], outv[5], outv[6], outv[7]);
}

// q/k/v projection rows (strided; q|k|v may be one fused projection) plus their biases ->
// rotated q rows (rows x heads x hd, contiguous), rotated k and v appended at cache rows
// *pos + r (forward.rs:347-363, 437-449). One workgroup per (head of q then k, row); the k
// workgroups also copy v. Rows landing at or past max_seq are not stored.
__global__ __launch_bounds__(64) void qkv_rope_append_kernel(const float* __restrict__ qs, int ldq,
                                                             const float* __restrict__ ks, int ldk,
                                                             const float* __restrict__ vs, int ldv,
                                                             const float* __restrict__ bq, const float* __restrict__ bk,
                                                             const float* __restrict__ bv, int heads, int kv_heads,
                                                             int hd, float base, const int* __restrict__ pos,
                                                             float* __restrict__ qout, float* __restrict__ kc,
                                                             float* __restrict__ vc, int max_seq) {
  const int hh = blockIdx.x, r = blockIdx.y;
  const int half = hd >> 1;
  const int p = *pos + r;
  const bool is_q = hh < heads;
  const int kh = hh - heads;
  if (!is_q && (p < 0 || p >= max_seq)) return;
  const float* src = is_q ? qs + (size_t)r * ldq + (size_t)hh * hd : ks + (size_t)r * ldk + (size_t)kh * hd;
  const float* bias = is_q ? (bq ? bq + (size_t)hh * hd : nullptr) : (bk ? bk + (size_t)kh * hd : nullptr);
  float* dst = is_q ? qout + ((size_t)r * heads + hh) * hd : kc + (size_t)p * kv_heads * hd + (size_t)kh * hd;
  for (int i = threadIdx.x; i < half; i += 64) {
    float x0 = src[i], x1 = src[i + half];
    if (bias) {
      x0 += bias[i];
      x1 += bias[i + half];
    }
    rope_pair(x0, x1, i, hd, p, base, dst[i], dst[i + half]);
  }
  if (!is_q) {
    const float* vsrc = vs + (size_t)r * ldv + (size_t)kh * hd;
    float* vdst = vc + (size_t)p * kv_heads * hd + (size_t)kh * hd;
    for (int i = threadIdx.x; i < hd; i += 64) vdst[i] = bv ? vsrc[i] + bv[kh * hd + i] : vsrc[i];
  }
}

// End of a decode step: the token is the index in the largest of the argmax slots (see
// argmax_key), the position advances, the token is recorded at its position in hist (when
// given) and the slots are cleared.
__global__ void decode_advance_kernel(unsigned long long* best, int* tok, int* pos, int delta, int* hist,
                                      int hist_len) {
  if (threadIdx.x != 0) return;
  unsigned long long k = best[0];
#pragma unroll
  for (int i = 1; i < kArgmaxSlots; ++i) k = best[i] > k ? best[i] : k;
  const int t = (int)(unsigned)(k & 0xffffffffull);
  const int np = *pos + delta;
  *tok = t;
  *pos = np;
  if (hist && np >= 0 && np < hist_len) hist[np] = t;
#pragma unroll
  for (int i = 0; i < kArgmaxSlots; ++i) best[i] = 0ull;
}

// out[i] = a[i] + b[i % nb]
__global__ __launch_bounds__(256) void add_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                  size_t n, size_t nb, float* __restrict__ out) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = a[i] + b[i % nb];
}

// index of the largest value; among equal maxima the last (Iterator::max_by, infer.rs:217-223)
__global__ __launch_bounds__(1024) void argmax_kernel(const float* __restrict__ x, int n, int* __restrict__ idx) {
  __shared__ float bv[16];
  __shared__ int bi[16];
  float best = -INFINITY;
  int besti = -1;
  for (int i = threadIdx.x; i < n; i += 1024) {
    const float v = x[i];
    if (v > best || (v == best && i > besti)) { best = v; besti = i; }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off, 64);
    const int oi = __shfl_xor(besti, off, 64);
    if (ov > best || (ov == best && oi > besti)) { best = ov; besti = oi; }
  }
  if ((threadIdx.x & 63) == 0) { bv[threadIdx.x >> 6] = best; bi[threadIdx.x >> 6] = besti; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 16; ++w)
      if (bv[w] > best || (bv[w] == best && bi[w] > besti)) { best = bv[w]; besti = bi[w]; }
    *idx = besti < 0 ? 0 : besti;
  }
}

__global__ __launch_bounds__(256) void embed_kernel(const float* __restrict__ table, int n_vocab, int d,
                                                    const int* __restrict__ tok, float* __restrict__ out) {
  const int t = tok[blockIdx.x];
  float* o = out + (size_t)blockIdx.x * d;
  if (t < 0 || t >= n_vocab) {
    for (int i = threadIdx.x; i < d; i += 256) o[i] = 0.0f;
    return;
  }
  const float* src = table + (size_t)t * d;
  for (int i = threadIdx.x; i < d; i += 256) o[i] = src[i];
}

__global__ void pos_add_kernel(int* pos, int delta) {
  if (threadIdx.x == 0) *pos += delta;
}

hipError_t launch_rmsnorm(const float* x, const float* w, int rows, int d, float eps, float* out, hipStream_t s) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)rows), dim3(256), 0, s, x, w, d, eps, out);
  return hipGetLastError();
}
hipError_t launch_rope(float* x, int rows, int heads, int hd, float base, const int* pos, int off, hipStream_t s) {
  hipLaunchKernelGGL(rope_kernel, dim3((unsigned)heads, (unsigned)rows), dim3(64), 0, s, x, heads, hd, base, pos, off);
  return hipGetLastError();
}
hipError_t launch_kv_append(const float* k, const float* v, int rows, int kv_dim, float* kc, float* vc,
                            int max_seq, const int* pos, hipStream_t s) {
  hipLaunchKernelGGL(kv_append_kernel, dim3((unsigned)rows), dim3(256), 0, s, k, v, kv_dim, kc, vc, max_seq, pos);
  return hipGetLastError();
}
hipError_t launch_attention(const float* q, const float* kc, const float* vc, int rows, int heads, int kv_heads,
                            int hd, int max_seq, const int* pos, float* work, float* ctx, hipStream_t s) {
  if (rows >= 8 && hd == 64) {
    const int grp = heads / kv_heads;
    const dim3 grid((unsigned)(((size_t)rows * grp + kAttnMfmaVecs - 1) / kAttnMfmaVecs), (unsigned)kv_heads);
    hipLaunchKernelGGL(attention_mfma_kernel, grid, dim3(256), 0, s, q, kc, vc, rows, heads, kv_heads, max_seq, pos,
                       ctx);
    return hipGetLastError();
  }
  if (work) {
    const int nsp = (max_seq + kAttnSplitKeys - 1) / kAttnSplitKeys;
    const dim3 grid((unsigned)heads, (unsigned)rows, (unsigned)nsp);
    const DecodeQkv none{};
    if (hd <= 64)
      hipLaunchKernelGGL((attention_split_kernel<1, false>), grid, dim3(256), 0, s, q, kc, vc, heads, kv_heads, hd,
                         max_seq, pos, work, none);
    else if (hd <= 128)
      hipLaunchKernelGGL((attention_split_kernel<2, false>), grid, dim3(256), 0, s, q, kc, vc, heads, kv_heads, hd,
                         max_seq, pos, work, none);
    else
      hipLaunchKernelGGL((attention_split_kernel<4, false>), grid, dim3(256), 0, s, q, kc, vc, heads, kv_heads, hd,
                         max_seq, pos, work, none);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(attention_combine_kernel, dim3((unsigned)heads, (unsigned)rows), dim3(64), 0, s, work, heads,
                       hd, nsp, ctx);
    return hipGetLastError();
  }
  const size_t lds = ((size_t)((max_seq + 3) & ~3) + 16 * (size_t)hd) * sizeof(float);
  const dim3 grid((unsigned)heads, (unsigned)rows);
  if (hd <= 64)
    hipLaunchKernelGGL(attention_rows_kernel<1>, grid, dim3(kAttnRowsThreads), lds, s, q, kc, vc, heads, kv_heads, hd,
                       max_seq, pos, ctx);
  else if (hd <= 128)
    hipLaunchKernelGGL(attention_rows_kernel<2>, grid, dim3(kAttnRowsThreads), lds, s, q, kc, vc, heads, kv_heads, hd,
                       max_seq, pos, ctx);
  else
    hipLaunchKernelGGL(attention_rows_kernel<4>, grid, dim3(kAttnRowsThreads), lds, s, q, kc, vc, heads, kv_heads, hd,
                       max_seq, pos, ctx);
  return hipGetLastError();
}
hipError_t launch_rope_table(float base, int hd, int rows, float* tab, hipStream_t s) {
  const size_t n = (size_t)rows * (size_t)(hd / 2);
  const unsigned grid = (unsigned)std::min<size_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(rope_table_kernel, dim3(grid), dim3(256), 0, s, base, hd, rows, reinterpret_cast<float2*>(tab));
  return hipGetLastError();
}
hipError_t launch_attention_decode(const float* q, const float* k, const float* v, const float* bq, const float* bk,
                                   const float* bv, int heads, int kv_heads, int hd, float base, const float* rope,
                                   const int* pos, float* kc, float* vc, int max_seq, float* work, float* ctx,
                                   hipStream_t s) {
  const int nsp = (max_seq + kAttnSplitKeys - 1) / kAttnSplitKeys;
  const dim3 grid((unsigned)heads, 1u, (unsigned)nsp);
  const DecodeQkv dq{k, v, bq, bk, bv, base, kc, vc, reinterpret_cast<const float2*>(rope), max_seq};
  auto a16 = [](const void* x) { return ((uintptr_t)x & 15) == 0; };   // null passes
  if (rope && hd % 8 == 0 && a16(rope) && a16(q) && a16(k) && a16(v) && a16(bq) && a16(bk) && a16(bv)) {
    if (hd == 64)
      hipLaunchKernelGGL((attention_split_kernel<1, true, true, true>), grid, dim3(256), 0, s, q, kc, vc, heads,
                         kv_heads, hd, max_seq, pos, work, dq);
    else if (hd <= 64)
      hipLaunchKernelGGL((attention_split_kernel<1, true, true>), grid, dim3(256), 0, s, q, kc, vc, heads, kv_heads,
                         hd, max_seq, pos, work, dq);
    else if (hd <= 128)
      hipLaunchKernelGGL((attention_split_kernel<2, true, true>), grid, dim3(256), 0, s, q, kc, vc, heads, kv_heads,
                         hd, max_seq, pos, work, dq);
    else
      hipLaunchKernelGGL((attention_split_kernel<4, true, true>), grid, dim3(256), 0, s, q, kc, vc, heads, kv_heads,
                         hd, max_seq, pos, work, dq);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(attention_combine_kernel, dim3((unsigned)heads, 1u), dim3(64), 0, s, work, heads, hd, nsp, ctx);
    return hipGetLastError();
  }
  if (hd <= 64)
    hipLaunchKernelGGL((attention_split_kernel<1, true>), grid, dim3(256), 0, s, q, kc, vc, heads, kv_heads, hd,
                       max_seq, pos, work, dq);
  else if (hd <= 128)
    hipLaunchKernelGGL((attention_split_kernel<2, true>), grid, dim3(256), 0, s, q, kc, vc, heads, kv_heads, hd,
                       max_seq, pos, work, dq);
  else
    hipLaunchKernelGGL((attention_split_kernel<4, true>), grid, dim3(256), 0, s, q, kc, vc, heads, kv_heads, hd,
                       max_seq, pos, work, dq);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(attention_combine_kernel, dim3((unsigned)heads, 1u), dim3(64), 0, s, work, heads, hd, nsp, ctx);
  return hipGetLastError();
}

hipError_t launch_add(const float* a, const float* b, size_t n, size_t nb, float* out, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(add_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a, b, n, nb, out);
  return hipGetLastError();
}
hipError_t launch_argmax(const float* x, int n, int* idx, hipStream_t s) {
  hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, s, x, n, idx);
  return hipGetLastError();
}
hipError_t launch_embed(const float* table, int n_vocab, int d, const int* tok, int rows, float* out,
                        hipStream_t s) {
  hipLaunchKernelGGL(embed_kernel, dim3((unsigned)rows), dim3(256), 0, s, table, n_vocab, d, tok, out);
  return hipGetLastError();
}
hipError_t launch_qkv_rope_append(const float* qs, int ldq, const float* ks, int ldk, const float* vs, int ldv,
                                  const float* bq, const float* bk, const float* bv, int rows, int heads,
                                  int kv_heads, int hd, float base, const int* pos, float* qout, float* kc,
                                  float* vc, int max_seq, hipStream_t s) {
  hipLaunchKernelGGL(qkv_rope_append_kernel, dim3((unsigned)(heads + kv_heads), (unsigned)rows), dim3(64), 0, s, qs,
                     ldq, ks, ldk, vs, ldv, bq, bk, bv, heads, kv_heads, hd, base, pos, qout, kc, vc, max_seq);
  return hipGetLastError();
}
hipError_t launch_decode_advance(unsigned long long* best, int* tok, int* pos, int delta, int* hist, int hist_len,
                                 hipStream_t s) {
  hipLaunchKernelGGL(decode_advance_kernel, dim3(1), dim3(64), 0, s, best, tok, pos, delta, hist, hist_len);
  return hipGetLastError();
}
hipError_t launch_pos_add(int* pos, int delta, hipStream_t s) {
  hipLaunchKernelGGL(pos_add_kernel, dim3(1), dim3(64), 0, s, pos, delta);
  return hipGetLastError();
}

}  // namespace rehip
