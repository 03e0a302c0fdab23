// MoE kernels: SwiGLU between the gate/up and down projections, the weighted combine of the
// routed expert outputs (src/moe.rs:280-283, 376-383), and the grouped expert GEMV used when
// the experts receive few rows each.
#include <hip/hip_runtime.h>

#include <cfloat>

#include "deq.hpp"
#include "kernels.hpp"

#include <algorithm>

namespace rehip {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;


// h = silu(g) * u, silu(x) = x * (1 / (1 + exp(-x)))  (moe.rs:44-51, 280-283)
__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                     float* __restrict__ h, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  h[i] = silu_mul(g[i], u[i]);
}

// out[t][c] = sum over j = 0..k-1, in order, of w[t*k+j] * yp[pos[t*k+j]][c]; the sum starts
// from 0 and every step is a rounded multiply then a rounded add (moe.rs:376-383). A thread
// takes V consecutive columns; the rows of eight pairs are loaded before any is added, so a
// token's k row reads overlap instead of following one another.
template <int V>
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ yp, const int* __restrict__ pos,
                                                      const float* __restrict__ w, float* __restrict__ out,
                                                      int k, int hidden) {
  typedef __attribute__((__vector_size__(V * sizeof(float)))) float fv;
  const int t = blockIdx.y;
  const int c = (blockIdx.x * 256 + threadIdx.x) * V;
  if (c >= hidden) return;
  fv o;
#pragma unroll
  for (int v = 0; v < V; ++v) o[v] = 0.0f;
  for (int j0 = 0; j0 < k; j0 += 8) {
    int pj[8];
    float wj[8];
    fv y[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      pj[j] = j0 + j < k ? pos[t * k + j0 + j] : -1;   // -1: past k, or an expert id out of range
      wj[j] = j0 + j < k ? w[t * k + j0 + j] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (pj[j] >= 0) y[j] = *reinterpret_cast<const fv*>(yp + (size_t)pj[j] * hidden + c);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (pj[j] >= 0) {
#pragma unroll
        for (int v = 0; v < V; ++v) o[v] = __fadd_rn(o[v], __fmul_rn(wj[j], y[j][v]));
      }
  }
  *reinterpret_cast<fv*>(out + (size_t)t * hidden + c) = o;
}

// ---- device-side routing and grouping (no host round trip) --------------------------------

// Router scores of one token: one wave per token; lane l holds experts l, l + 64, ...
// Selection repeats a wave-wide argmax k times, ties to the lower expert index, which is the
// order the reference's stable descending sort gives (moe.rs:75-93, 98-118). NaN scores are
// treated as -inf (the reference's partial_cmp leaves their order unspecified).
constexpr int kRouteMaxExperts = 1024;

// One wave routes one token (`row` holds its n_experts scores): up to EPL experts per lane, of
// which the first ceil(n_experts / 64) are used. Lane 0 writes the k ids and weights to ids[] /
// weights[] (global memory or LDS); topv / topi: k entries of scratch that lane 0 alone touches.
template <int EPL>
__device__ __forceinline__ void route_token(const float* row, int n_experts, int k, int gate, int lane,
                                            float* topv, int* topi, int* ids, float* weights) {
  const int epl = (n_experts + 63) / 64;
  float v[EPL];
  bool taken[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    float x = -INFINITY;
    if (j < epl && e < n_experts) {
      x = row[e];
      if (gate == 1) x = 1.0f / (1.0f + expf(-x));     // sigmoid (moe.rs:43-46)
      if (x != x) x = -INFINITY;
    }
    v[j] = x;
    taken[j] = e >= n_experts;
  }
  for (int r = 0; r < k; ++r) {
    float bv = -INFINITY;
    int be = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      if (j >= epl) break;                             // uniform
      const int e = lane + 64 * j;
      if (!taken[j] && (v[j] > bv || (v[j] == bv && e < be))) { bv = v[j]; be = e; }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = __shfl_xor(bv, off, 64);
      const int oe = __shfl_xor(be, off, 64);
      if (ov > bv || (ov == bv && oe < be)) { bv = ov; be = oe; }
    }
#pragma unroll
    for (int j = 0; j < EPL; ++j)
      if (lane + 64 * j == be) taken[j] = true;
    if (lane == 0) { topv[r] = bv; topi[r] = be; }
  }
  if (lane != 0) return;
  if (gate == 1) {
    // weights = sig / sum of the chosen sigs, summed in order (moe.rs:108-117)
    float ws = 0.0f;
    for (int r = 0; r < k; ++r) ws += topv[r];
    for (int r = 0; r < k; ++r) {
      ids[r] = topi[r];
      weights[r] = ws == 0.0f ? 0.0f : topv[r] / ws;
    }
  } else {
    // softmax over the chosen logits (moe.rs:53-72): max, exp(v - max), sequential sum, divide
    float mx = -INFINITY;
    for (int r = 0; r < k; ++r) mx = fmaxf(mx, topv[r]);
    float sum = 0.0f;
    for (int r = 0; r < k; ++r) {
      topv[r] = expf(topv[r] - mx);
      sum += topv[r];
    }
    for (int r = 0; r < k; ++r) {
      ids[r] = topi[r];
      weights[r] = sum != 0.0f ? topv[r] / sum : topv[r];
    }
  }
}

// EPL = experts per lane (n_experts <= 64 EPL).
template <int EPL>
__global__ __launch_bounds__(64) void moe_route_kernel(const float* __restrict__ logits, int n_experts, int k,
                                                       int gate, int* __restrict__ ids,
                                                       float* __restrict__ weights) {
  __shared__ float topv[kRouteMaxExperts];
  __shared__ int topi[kRouteMaxExperts];
  const int t = blockIdx.x;
  route_token<EPL>(logits + (size_t)t * n_experts, n_experts, k, gate, threadIdx.x, topv, topi, ids + (size_t)t * k,
                   weights + (size_t)t * k);
}

// Bias-corrected group routing of one token per wave (route_group / route_noaux_tc,
// moe.rs:126-268). Scores sigmoid(logit + bias[e]) (bias entries past bias_len are 0) go to
// LDS; lane g then scores group g, the experts e with e * ng / n == g, walking them in index order
// as the reference does: their sum from 0.0 (top2 = 0), or the sum of the two best with the
// reference's update rule (top2 = 1). The top_k_group best groups (ties to the lower group, the
// stable descending sort; 0 = every group) are picked by repeated wave argmax, experts outside them
// are excluded, and the top k of the rest are picked the same way and renormalised over their
// scores, summed in rank order. When the eligible groups hold fewer than k experts the remaining
// slots get id -1 and weight 0 (the reference returns the shorter list; an id out of range
// contributes nothing downstream). NaN scores rank as -inf.
template <int EPL>
__global__ __launch_bounds__(64) void moe_route_group_kernel(const float* __restrict__ logits, int n_experts, int k,
                                                             int top2, const float* __restrict__ bias, int bias_len,
                                                             int ng, int tkg, int* __restrict__ ids,
                                                             float* __restrict__ weights) {
  __shared__ float sc[kRouteMaxExperts];
  __shared__ float gs[kRouteMaxExperts];
  __shared__ int allowed[kRouteMaxExperts];
  __shared__ float topv[kRouteMaxExperts];
  __shared__ int topi[kRouteMaxExperts];
  const int t = blockIdx.x, lane = threadIdx.x;
  const float* row = logits + (size_t)t * n_experts;
  for (int e = lane; e < n_experts; e += 64) {
    const float x = row[e] + (bias && e < bias_len ? bias[e] : 0.0f);
    float s = 1.0f / (1.0f + expf(-x));                // sigmoid (moe.rs:43-46)
    if (s != s) s = -INFINITY;
    sc[e] = s;
  }
  __syncthreads();
  for (int g = lane; g < ng; g += 64) {
    const int lo = (int)(((long long)g * n_experts + ng - 1) / ng);
    const int hi = (int)(((long long)(g + 1) * n_experts + ng - 1) / ng);
    float sum = 0.0f, t1 = -FLT_MAX, t2 = -FLT_MAX;
    for (int i = lo; i < hi; ++i) {
      const float v = sc[i];
      if (!top2) {
        sum += v;
      } else if (v >= t1) {
        t2 = t1;
        t1 = v;
      } else if (v > t2) {
        t2 = v;
      }
    }
    gs[g] = top2 ? t1 + (t2 == -FLT_MAX ? 0.0f : t2) : sum;
    allowed[g] = tkg == 0;
  }
  __syncthreads();
  const int take = tkg < ng ? tkg : ng;
  for (int r = 0; r < take; ++r) {
    float bv = -INFINITY;
    int bg = 0x7fffffff;
    for (int g = lane; g < ng; g += 64)
      if (!allowed[g] && (gs[g] > bv || (gs[g] == bv && g < bg))) { bv = gs[g]; bg = g; }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = __shfl_xor(bv, off, 64);
      const int og = __shfl_xor(bg, off, 64);
      if (ov > bv || (ov == bv && og < bg)) { bv = ov; bg = og; }
    }
    if (lane == 0 && bg < ng) allowed[bg] = 1;
    __syncthreads();
  }
  const int epl = (n_experts + 63) / 64;
  float v[EPL];
  bool taken[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    const bool in = j < epl && e < n_experts;
    v[j] = in ? sc[e] : -INFINITY;
    taken[j] = !in || !allowed[(int)((long long)e * ng / n_experts)];
  }
  for (int r = 0; r < k; ++r) {
    float bv = -INFINITY;
    int be = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      if (j >= epl) break;                             // uniform
      const int e = lane + 64 * j;
      if (!taken[j] && (v[j] > bv || (v[j] == bv && e < be))) { bv = v[j]; be = e; }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = __shfl_xor(bv, off, 64);
      const int oe = __shfl_xor(be, off, 64);
      if (ov > bv || (ov == bv && oe < be)) { bv = ov; be = oe; }
    }
#pragma unroll
    for (int j = 0; j < EPL; ++j)
      if (lane + 64 * j == be) taken[j] = true;
    if (lane == 0) { topv[r] = bv; topi[r] = be; }
  }
  if (lane != 0) return;
  int kk = 0;                                          // eligible experts found (a prefix of the ranks)
  while (kk < k && topi[kk] < n_experts) ++kk;
  float ws = 0.0f;
  for (int r = 0; r < kk; ++r) ws += topv[r];
  for (int r = 0; r < k; ++r) {
    ids[(size_t)t * k + r] = r < kk ? topi[r] : -1;
    weights[(size_t)t * k + r] = r < kk && ws != 0.0f ? topv[r] / ws : 0.0f;
  }
}

// logits[t][e] = router_w[e] . x[t] (the f32 matvec of moe.rs:367): x[t] staged in LDS, one wave
// per expert; lanes take every 64th element, then a fixed xor tree.
__global__ __launch_bounds__(256) void moe_router_logits_kernel(const float* __restrict__ x,
                                                                const float* __restrict__ w, int hidden,
                                                                int n_experts, float* __restrict__ logits) {
  extern __shared__ float xs[];
  const int t = blockIdx.y;
  const float* xr = x + (size_t)t * hidden;
  for (int i = threadIdx.x; i < hidden; i += 256) xs[i] = xr[i];
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (e >= n_experts) return;
  const float* wr = w + (size_t)e * hidden;
  float a = 0.0f;
  for (int i = lane; i < hidden; i += 64) a = __builtin_fmaf(wr[i], xs[i], a);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) a += __shfl_xor(a, off, 64);
  if (lane == 0) logits[(size_t)t * n_experts + e] = a;
}

// Grouping on the device, one 1024-thread workgroup, as a stable counting sort by expert (pair
// order inside an expert: the host grouping's order). Wave w ranks the pairs of its own segment
// (16 contiguous segments, a multiple of 64 pairs each) 64 at a time: the lanes holding the same
// expert are found by one ballot per bit of the expert id (each lane keeps the ballots that agree
// with its bits), a lane's rank is the count of those lanes below it plus the wave's running
// count of that expert, kept in LDS. Per-expert prefix sums over the waves and over the experts
// then give slot = start[e] + earlier waves' count + rank, xrow[slot] = pair / k and
// pos[pair] = slot; per-expert counts and starts give the chunks (runs of `chunk` gathered rows)
// and the task lists, laid out exactly as the host planner lays them out (expert, then chunk,
// then weight-row task). Pairs with an expert id out of range get pos = -1 and no task (the
// combine skips them).
constexpr int kPlanWaves = 16;

__device__ __forceinline__ void moe_plan_body(const int* __restrict__ ids, const MoePlanShape& sh,
                                              int* __restrict__ meta) {
  __shared__ uint32_t key[kMoeMaxDevicePairs];              // (expert << 16) | rank in the segment
  __shared__ int hist[kPlanWaves * kRouteMaxExperts];       // per wave and expert
  __shared__ int cnt[kRouteMaxExperts], start[kRouteMaxExperts], cstart[kRouteMaxExperts + 1];
  const int P = sh.pairs, E = sh.n_experts, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  int* xrow = meta;
  int* pos = meta + P;
  int* ntasks = meta + 2 * P;
  uint8_t* tasks = (uint8_t*)(meta + 2 * P + 4);
  const int seg = (P + 64 * kPlanWaves - 1) / (64 * kPlanWaves) * 64;   // pairs per wave (<= 512)
  const int nb = 32 - __builtin_clz((unsigned)max(E - 1, 1));            // bits of an expert id
  int* wh = hist + w * kRouteMaxExperts;   // this wave's counts: only this wave touches them before the barrier
  for (int e = lane; e < E; e += 64) wh[e] = 0;
  const uint64_t below = (1ull << lane) - 1, above = ~((2ull << lane) - 1);
  // the wave's ids, all loads in flight at once (seg <= 512: at most 8 per lane)
  constexpr int kSub = kMoeMaxDevicePairs / (64 * kPlanWaves);
  int ev[kSub];
#pragma unroll
  for (int i = 0; i < kSub; ++i) {
    const int p = w * seg + 64 * i + lane;
    ev[i] = 64 * i < seg && p < P ? ids[p] : -1;
  }
#pragma unroll
  for (int i = 0; i < kSub; ++i) {
    const int p = w * seg + 64 * i + lane;
    if (64 * i >= seg || w * seg + 64 * i >= P) break;   // uniform
    int e = ev[i];
    if (p < P && (e < 0 || e >= E)) {
      pos[p] = -1;
      key[p] = 0xffffffffu;
    }
    if (e >= E) e = -1;
    const bool valid = e >= 0;
    uint64_t same = __ballot(valid);
    for (int b = 0; b < nb; ++b) {
      const bool bit = valid && ((e >> b) & 1);
      const uint64_t bal = __ballot(bit);
      same &= bit ? bal : ~bal;
    }
    if (valid) {
      const int prev = wh[e];
      key[p] = ((uint32_t)e << 16) | (uint32_t)(prev + __popcll(same & below));
      if ((same & above) == 0) wh[e] = prev + __popcll(same);   // the highest lane of the expert
    }
  }
  __syncthreads();
  // per expert: the waves' counts become exclusive offsets, their sum the expert's count
  if (tid < E) {
    int c[kPlanWaves];
#pragma unroll
    for (int v = 0; v < kPlanWaves; ++v) c[v] = hist[v * kRouteMaxExperts + tid];
    int run = 0;
#pragma unroll
    for (int v = 0; v < kPlanWaves; ++v) {
      hist[v * kRouteMaxExperts + tid] = run;
      run += c[v];
    }
    cnt[tid] = run;
  }
  __syncthreads();
  // row starts and chunk starts per expert: an exclusive scan over the block, one expert per
  // thread (E <= 1024): wave scans, then the wave totals in order
  __shared__ int wsum[2][kPlanWaves];
  {
    const int c = tid < E ? cnt[tid] : 0;
    const int ch = tid < E ? (c + sh.chunk - 1) / sh.chunk : 0;
    int sc = c, sch = ch;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int a = __shfl_up(sc, off, 64), b = __shfl_up(sch, off, 64);
      if (lane >= off) { sc += a; sch += b; }
    }
    if (lane == 63) { wsum[0][w] = sc; wsum[1][w] = sch; }
    __syncthreads();
    int base = 0, cbase = 0, ctot = 0;
    for (int j = 0; j < kPlanWaves; ++j) {
      if (j < w) { base += wsum[0][j]; cbase += wsum[1][j]; }
      ctot += wsum[1][j];
    }
    if (tid < E) {
      start[tid] = base + sc - c;
      cstart[tid] = cbase + sch - ch;
    }
    if (tid == 0) {
      cstart[E] = ctot;
      ntasks[0] = min(ctot * sh.tiles_gu, sh.max_gu);   // the capacities bound every count
      ntasks[1] = min(ctot * sh.tiles_d, sh.max_d);
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kSub; ++i) {
    const int p = tid + 64 * kPlanWaves * i;
    if (p >= P) break;
    const uint32_t kk = key[p];
    if (kk == 0xffffffffu) continue;
    const int e = (int)(kk >> 16);
    const int slot = start[e] + hist[(p / seg) * kRouteMaxExperts + e] + (int)(kk & 0xffffu);
    xrow[slot] = p / sh.k;
    pos[p] = slot;
  }
  const int nch = cstart[E];
  const int n_gu = min(nch * sh.tiles_gu, sh.max_gu), n_d = min(nch * sh.tiles_d, sh.max_d);
  auto chunk_of = [&](int c, int& e, int& r0, int& rn) {
    int lo = 0, hi = E - 1;                  // last expert with cstart <= c
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (cstart[mid] <= c) lo = mid; else hi = mid - 1;
    }
    e = lo;
    const int r = (c - cstart[e]) * sh.chunk;
    r0 = start[e] + r;
    rn = min(sh.chunk, cnt[e] - r);
  };
  // one thread per chunk finds its expert, then the tasks are written with consecutive threads on
  // consecutive records (task t = chunk * tiles + tile). The chunk table reuses the sort keys:
  // expert << 20 | first row << 7 | rows (rows <= 64, first row < 8192, expert < 1024).
  __syncthreads();                                   // every key has been read above
  for (int c = tid; c < nch; c += 1024) {
    int e, r0, rn;
    chunk_of(c, e, r0, rn);
    key[c] = ((uint32_t)e << 20) | ((uint32_t)r0 << 7) | (uint32_t)rn;
  }
  __syncthreads();
  auto write_tasks = [&](uint8_t* list, int n, int tiles, int rows) {
    for (int t0 = 0; t0 < n; t0 += 4096) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int t = t0 + 1024 * u + tid;
        if (t >= n) break;
        const int c = t / tiles, j = t - c * tiles;
        const uint32_t kc = key[c];
        const int e = (int)(kc >> 20), r0 = (int)((kc >> 7) & 0x1fffu), rn = (int)(kc & 0x7fu);
        if (sh.gemv) reinterpret_cast<MoeGemvTask*>(list)[t] = {e, j * rows, r0, rn};
        else reinterpret_cast<GemmTask*>(list)[t] = {e, j, r0, rn};
      }
    }
  };
  const size_t rec = sh.gemv ? sizeof(MoeGemvTask) : sizeof(GemmTask);
  write_tasks(tasks, n_gu, sh.tiles_gu, sh.rows_gu);
  write_tasks(tasks + (size_t)sh.max_gu * rec, n_d, sh.tiles_d, sh.rows_d);
}

// The bf16 copy of X for the grouped GEMMs rides along with the plan: workgroups 1.. convert
// (round to nearest even, as x_to_bf16_kernel), workgroup 0 plans.
__global__ __launch_bounds__(64 * kPlanWaves) void moe_plan_convert_kernel(const int* __restrict__ ids,
                                                                           MoePlanShape sh, int* __restrict__ meta,
                                                                           const float4* __restrict__ x,
                                                                           bf16x8_t* __restrict__ xb, size_t n8,
                                                                           int split) {
  if (blockIdx.x == 0) {
    moe_plan_body(ids, sh, meta);
    return;
  }
  for (size_t i = (size_t)(blockIdx.x - 1) * 1024 + threadIdx.x; i < n8; i += (size_t)(gridDim.x - 1) * 1024) {
    const float4 a = x[2 * i], b = x[2 * i + 1];
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    bf16x8_t o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = (__bf16)v[j];
    xb[i] = o;
    if (split) {                          // the lo halves, as x_to_bf16_split_kernel
      bf16x8_t l;
#pragma unroll
      for (int j = 0; j < 8; ++j) l[j] = (__bf16)(v[j] - (float)o[j]);
      xb[n8 + i] = l;
    }
  }
}

size_t moe_meta_bytes(const MoePlanShape& sh) {
  const size_t rec = sh.gemv ? sizeof(MoeGemvTask) : sizeof(GemmTask);
  return (size_t)(2 * sh.pairs + 4) * sizeof(int) + (size_t)(sh.max_gu + sh.max_d) * rec;
}

hipError_t launch_moe_route(const float* logits, int tokens, int n_experts, int k, int gate, int* ids,
                            float* weights, hipStream_t s) {
  const int epl = (n_experts + 63) / 64;
  if (epl <= 1)
    hipLaunchKernelGGL(moe_route_kernel<1>, dim3((unsigned)tokens), dim3(64), 0, s, logits, n_experts, k, gate, ids, weights);
  else if (epl <= 2)
    hipLaunchKernelGGL(moe_route_kernel<2>, dim3((unsigned)tokens), dim3(64), 0, s, logits, n_experts, k, gate, ids, weights);
  else if (epl <= 4)
    hipLaunchKernelGGL(moe_route_kernel<4>, dim3((unsigned)tokens), dim3(64), 0, s, logits, n_experts, k, gate, ids, weights);
  else if (epl <= 8)
    hipLaunchKernelGGL(moe_route_kernel<8>, dim3((unsigned)tokens), dim3(64), 0, s, logits, n_experts, k, gate, ids, weights);
  else
    hipLaunchKernelGGL(moe_route_kernel<kRouteMaxExperts / 64>, dim3((unsigned)tokens), dim3(64), 0, s, logits, n_experts, k,
                       gate, ids, weights);
  return hipGetLastError();
}

hipError_t launch_moe_route_group(const float* logits, int tokens, int n_experts, int k, int top2, const float* bias,
                                  int bias_len, int n_groups, int top_k_group, int* ids, float* weights,
                                  hipStream_t s) {
  const int epl = (n_experts + 63) / 64;
#define RE_ROUTE_GROUP(E)                                                                                        \
  hipLaunchKernelGGL(moe_route_group_kernel<E>, dim3((unsigned)tokens), dim3(64), 0, s, logits, n_experts, k, top2, \
                     bias, bias_len, n_groups, top_k_group, ids, weights)
  if (epl <= 1) RE_ROUTE_GROUP(1);
  else if (epl <= 2) RE_ROUTE_GROUP(2);
  else if (epl <= 4) RE_ROUTE_GROUP(4);
  else if (epl <= 8) RE_ROUTE_GROUP(8);
  else RE_ROUTE_GROUP(kRouteMaxExperts / 64);
#undef RE_ROUTE_GROUP
  return hipGetLastError();
}

// Tiled form for hidden % 4 == 0 and 16-byte aligned rows: a workgroup computes 8 experts x TT
// tokens (two experts per wave); lane l takes the float4 at k = 4 l + 256 i of every row, so the
// router rows are read once per token tile and the token rows once per 8 experts. Each of the
// 2 TT sums is folded over the wave by a fixed xor tree.
template <int TT>
__global__ __launch_bounds__(256) void moe_router_tile_kernel(const float* __restrict__ x,
                                                              const float* __restrict__ w, int hidden,
                                                              int n_experts, int tokens,
                                                              float* __restrict__ logits) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e0 = blockIdx.x * 8 + 2 * wave, t0 = blockIdx.y * TT;
  if (e0 >= n_experts) return;           // no workgroup barrier below
  const bool e1ok = e0 + 1 < n_experts;
  const float4* w0 = reinterpret_cast<const float4*>(w + (size_t)e0 * hidden);
  const float4* w1 = reinterpret_cast<const float4*>(w + (size_t)(e1ok ? e0 + 1 : e0) * hidden);
  const float4* xr[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t)
    xr[t] = reinterpret_cast<const float4*>(x + (size_t)min(t0 + t, tokens - 1) * hidden);
  float acc[2][TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) acc[0][t] = acc[1][t] = 0.0f;
  const int nv = hidden / 4;
  // U of the lane's float4 at a time: their loads go out together, then the FMAs in the same
  // order (one float4 at a time waited an L2 round trip per step); past the row a lane loads the
  // last float4 and skips its FMAs
  constexpr int U = TT == 1 ? 8 : 4;
  for (int v0 = lane; v0 < nv; v0 += 64 * U) {
    float4 a[U], b[U], q[U][TT];
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const int v = min(v0 + 64 * j, nv - 1);
      a[j] = w0[v];
      b[j] = w1[v];
#pragma unroll
      for (int t = 0; t < TT; ++t) q[j][t] = xr[t][v];
    }
#pragma unroll
    for (int j = 0; j < U; ++j) {
      if (v0 + 64 * j < nv) {
#pragma unroll
        for (int t = 0; t < TT; ++t) {
          acc[0][t] = __builtin_fmaf(a[j].w, q[j][t].w, __builtin_fmaf(a[j].z, q[j][t].z,
                      __builtin_fmaf(a[j].y, q[j][t].y, __builtin_fmaf(a[j].x, q[j][t].x, acc[0][t]))));
          acc[1][t] = __builtin_fmaf(b[j].w, q[j][t].w, __builtin_fmaf(b[j].z, q[j][t].z,
                      __builtin_fmaf(b[j].y, q[j][t].y, __builtin_fmaf(b[j].x, q[j][t].x, acc[1][t]))));
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      float v = acc[j][t];
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
      acc[j][t] = v;
    }
  if (lane == 0) {
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      if (t0 + t >= tokens) break;
      logits[(size_t)(t0 + t) * n_experts + e0] = acc[0][t];
      if (e1ok) logits[(size_t)(t0 + t) * n_experts + e0 + 1] = acc[1][t];
    }
  }
}

hipError_t launch_moe_router_logits(const float* x, const float* router_w, int tokens, int hidden, int n_experts,
                                    float* logits, hipStream_t s) {
  const bool tiled = hidden % 4 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)router_w & 15) == 0;
  if (tiled) {
    const unsigned ge = (unsigned)((n_experts + 7) / 8);
    if (tokens < 8)
      hipLaunchKernelGGL(moe_router_tile_kernel<1>, dim3(ge, (unsigned)tokens), dim3(256), 0, s, x, router_w, hidden,
                         n_experts, tokens, logits);
    else
      hipLaunchKernelGGL(moe_router_tile_kernel<8>, dim3(ge, (unsigned)((tokens + 7) / 8)), dim3(256), 0, s, x,
                         router_w, hidden, n_experts, tokens, logits);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(moe_router_logits_kernel, dim3((unsigned)((n_experts + 3) / 4), (unsigned)tokens), dim3(256),
                     (size_t)hidden * sizeof(float), s, x, router_w, hidden, n_experts, logits);
  return hipGetLastError();
}

hipError_t launch_moe_plan(const int* ids, const MoePlanShape& sh, void* meta, const float* x, void* xb, size_t n,
                           hipStream_t s, bool split) {
  if (xb && n % 8) return hipErrorInvalidValue;
  const size_t n8 = xb ? n / 8 : 0;
  const unsigned conv = (unsigned)std::min<size_t>((n8 + 1023) / 1024, 255);
  hipLaunchKernelGGL(moe_plan_convert_kernel, dim3(1 + conv), dim3(64 * kPlanWaves), 0, s, ids, sh, (int*)meta,
                     (const float4*)x, (bf16x8_t*)xb, n8, split ? 1 : 0);
  return hipGetLastError();
}

// the same h rounded to bf16 (RNE), for a bf16-mode GEMM that consumes it
__global__ __launch_bounds__(256) void swiglu_bf16_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                          __bf16* __restrict__ h, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  h[i] = (__bf16)silu_mul(g[i], u[i]);
}

hipError_t launch_swiglu_bf16(const float* g, const float* u, void* h, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(swiglu_bf16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, g, u, (__bf16*)h, n);
  return hipGetLastError();
}

hipError_t launch_swiglu(const float* g, const float* u, float* h, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, g, u, h, n);
  return hipGetLastError();
}

hipError_t launch_combine(const float* yp, const int* pos, const float* w, float* out, int tokens, int k,
                          int hidden, hipStream_t s) {
  if (tokens == 0) return hipSuccess;
  // four columns a thread where every row start is 16-byte aligned
  const bool v4 = hidden % 4 == 0 && ((uintptr_t)yp | (uintptr_t)out) % 16 == 0;
  if (v4)
    hipLaunchKernelGGL(combine_kernel<4>, dim3((unsigned)((hidden / 4 + 255) / 256), (unsigned)tokens), dim3(256), 0,
                       s, yp, pos, w, out, k, hidden);
  else
    hipLaunchKernelGGL(combine_kernel<1>, dim3((unsigned)((hidden + 255) / 256), (unsigned)tokens), dim3(256), 0, s,
                       yp, pos, w, out, k, hidden);
  return hipGetLastError();
}


// Grouped expert GEMV for experts that receive at most NB gathered rows per task (decode-sized
// batches). A task is (expert, R weight rows starting at row0, gathered rows p0..p0+np-1). The
// workgroup stages the np activation rows (and their per-16 sums) in LDS; lane l of a wave
// serves weight row l % R, and the 64/R lane groups of every wave take the row's 32-quant units
// in turn (the row-group GEMV mapping). Each decoded run is dotted with all np rows, so a weight
// is read once per task. DUAL: the gate and up matrices are read side by side and the task
// writes silu(gate) * up (SwiGLU, moe.rs:280-283) directly. Sums fold over lane groups by a
// fixed xor tree and over waves in wave order (deterministic).
template <int T, int R, int WAVES, int NB, bool DUAL, bool ONE>
__global__ __launch_bounds__(WAVES * 64) void moe_gemv_kernel(MoeGemvArgs a) {
  using B = Blk<T>;
  constexpr int NCH = B::NCH;
  constexpr int D = ONE ? 1 : 2;         // units in flight per slot (ONE: a slot has at most one)
  constexpr int G = 64 / R;
  constexpr int S = WAVES * G;
  constexpr int NM = DUAL ? 2 : 1;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  // tasks from the list, or (tasks == nullptr: one activation row, expert 0, the decoder's gate/up
  // pair) row block blockIdx.x, with no dependent load before the first weight loads
  MoeGemvTask task{0, (int)blockIdx.x * R, 0, 1};
  if (a.tasks) {
    if (a.ntasks && (int)blockIdx.x >= *a.ntasks) return;   // grid sized for the most tasks
    task = a.tasks[blockIdx.x];
  } else if (a.ids || a.id_inline) {
    const int j = (int)blockIdx.x / a.id_tiles;
    const int e = a.ids ? a.ids[j] : a.id_v[j];
    if (e < 0 || e >= a.n_experts) return;
    task = {e, ((int)blockIdx.x - j * a.id_tiles) * R, j, 1};
  }
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int KP = a.KB * B::QK;
  float* xl = smem;                      // [NB][KP]
  float* xs16 = smem + NB * KP;          // [NB][KP/16]
  float* red = xs16 + NB * (KP / 16);    // [WAVES][NM][NB][R]
  float* ssred = red + WAVES * NM * NB * R;   // [WAVES][NB]

  // the task's R rows lie in one 64-row tile (row0 is a multiple of R, R divides 64), so the
  // tile and the weight resources are uniform
  const int row0 = __builtin_amdgcn_readfirstlane(task.row0);
  const int expert = __builtin_amdgcn_readfirstlane(task.expert);
  const int tile = row0 >> 6, rr = (row0 & 63) + (lane % R);
  const size_t wofs = (size_t)expert * a.w_stride + (size_t)tile * a.KB * B::SLAB;
  const uint32_t tbytes = (uint32_t)a.KB * (uint32_t)B::SLAB;
  const __amdgpu_buffer_rsrc_t w0r = make_rsrc(a.W0 + wofs, tbytes);
  const __amdgpu_buffer_rsrc_t w1r = make_rsrc(DUAL ? a.W1 + wofs : a.W0 + wofs, tbytes);
  const int slot = wave * G + lane / R;
  const int u_end = a.KB * NCH;
  // a chunk past the end reads at an offset past the resource (zeros, no memory traffic): the
  // ring's first loads need no branch, which made the compiler wait for each load where the
  // branch joins (one memory round trip per entry)
  auto load = [&](int u, typename B::CR& r0, typename B::CR& r1) {
    const uint32_t off = u < u_end ? (uint32_t)(u / NCH) * (uint32_t)B::SLAB : 0x80000000u;
    B::bload_chunk(w0r, off, rr, u % NCH, r0);
    if constexpr (DUAL) B::bload_chunk(w1r, off, rr, u % NCH, r1);
  };

  // this thread's first activation (and norm weight) goes out before the weight loads: loads
  // retire in order, so the staging below then waits for it alone and overlaps the weights'
  // round trip
  const int nv = KP / 4;
  float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), w0 = x0;
  {
    const int i = threadIdx.x, nb = i / nv, k = 4 * (i - nb * nv);
    if (i < NB * nv && nb < task.np && k < a.K) {
      const int p = task.p0 + nb;
      const int xr = a.ids || a.id_inline ? 0 : (a.xrow ? a.xrow[p] : p);
      x0 = *reinterpret_cast<const float4*>(a.X + (size_t)xr * a.K + k);
      if (a.norm_w) w0 = *reinterpret_cast<const float4*>(a.norm_w + k);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  typename B::CR ring0[D], ring1[D];
#pragma unroll
  for (int i = 0; i < D; ++i) load(slot + i * S, ring0[i], ring1[i]);
  __builtin_amdgcn_sched_barrier(0);

  // stage the task's activation rows (zero past K and past np); with an RMS-norm, x * w is
  // staged, each thread keeps its rows' sums of squares, and 1/rms scales the finished dots
  float ss[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) ss[nb] = 0.0f;
  for (int i = threadIdx.x; i < NB * nv; i += WAVES * 64) {
    const int nb = i / nv, k = 4 * (i - nb * nv);
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (nb < task.np && k < a.K) {
      const bool first = i == (int)threadIdx.x;
      const int p = task.p0 + nb;
      const int xr = a.ids || a.id_inline ? 0 : (a.xrow ? a.xrow[p] : p);   // routed by ids: the one row
      v = first ? x0 : *reinterpret_cast<const float4*>(a.X + (size_t)xr * a.K + k);
      if (a.norm_w) {
        float t = __builtin_fmaf(v.x, v.x, __builtin_fmaf(v.y, v.y, __builtin_fmaf(v.z, v.z, v.w * v.w)));
#pragma unroll
        for (int q = 0; q < NB; ++q)
          if (q == nb) ss[q] += t;
        const float4 w = first ? w0 : *reinterpret_cast<const float4*>(a.norm_w + k);
        v = make_float4(v.x * w.x, v.y * w.y, v.z * w.z, v.w * w.w);
      }
    }
    reinterpret_cast<float4*>(xl)[i] = v;
  }
  __syncthreads();
  if constexpr (kNeedXs16<T>) {   // per-16 sums of x: only the dots that take out an offset use them
    for (int i = threadIdx.x; i < NB * (KP / 16); i += WAVES * 64) {
      const float4* q = reinterpret_cast<const float4*>(xl + 16 * i);
      float sum = 0.0f;
#pragma unroll
      for (int v = 0; v < 4; ++v) { const float4 t = q[v]; sum += t.x; sum += t.y; sum += t.z; sum += t.w; }
      xs16[i] = sum;
    }
    __syncthreads();
  }

  float acc[NM][NB];
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[m][nb] = 0.0f;
  for (int base = slot; base < u_end; base += D * S) {
#pragma unroll
    for (int i = 0; i < D; ++i) {
      const int u = base + i * S;
      if (u < u_end) {
        const int kb = u / NCH, c = u - kb * NCH;
        Run a0, b0, a1, b1;
        B::decode_chunk(ring0[i], c, a0, b0);
        if constexpr (DUAL) B::decode_chunk(ring1[i], c, a1, b1);
        const int un = u + D * S;
        if (!ONE && un < u_end) load(un, ring0[i], ring1[i]);
        const int valid = a.K - kb * B::QK;   // K is a multiple of 32: a run is wholly in or out
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          if (nb >= task.np) break;            // uniform: the task's row count
          const float* xb = xl + nb * KP + kb * B::QK;
          const float* xs = xs16 + nb * (KP / 16) + kb * (B::QK / 16);
          if (a0.e < valid) acc[0][nb] += run_dot<T>(a0, xb, xs);
          if (b0.e < valid) acc[0][nb] += run_dot<T>(b0, xb, xs);
          if constexpr (DUAL) {
            if (a1.e < valid) acc[NM - 1][nb] += run_dot<T>(a1, xb, xs);
            if (b1.e < valid) acc[NM - 1][nb] += run_dot<T>(b1, xb, xs);
          }
        }
      }
    }
  }

#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      float v = acc[m][nb];
#pragma unroll
      for (int off = R; off < 64; off *= 2) v += __shfl_xor(v, off, 64);
      if (lane < R) red[((wave * NM + m) * NB + nb) * R + lane] = v;
    }
  if (a.norm_w) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      float t = ss[nb];
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) t += __shfl_xor(t, off, 64);
      if (lane == 0) ssred[wave * NB + nb] = t;
    }
  }
  __syncthreads();
  if ((int)threadIdx.x < R * NB) {
    const int r = threadIdx.x % R, nb = threadIdx.x / R;
    float inv = 1.0f;
    if (a.norm_w) {
      float t = ssred[nb];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) t += ssred[w * NB + nb];
      inv = 1.0f / sqrtf(t / (float)a.K + a.norm_eps);
    }
    float v[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      float sum = red[((0 * NM + m) * NB + nb) * R + r];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) sum += red[((w * NM + m) * NB + nb) * R + r];
      v[m] = a.norm_w ? sum * inv : sum;
    }
    const int wrow = task.row0 + r;
    if (nb < task.np && wrow < a.m) {
      float* y = a.Y + (size_t)(task.p0 + nb) * a.ldy + wrow;
      *y = DUAL ? silu_mul(v[0], v[NM - 1]) : v[0];
    }
  }
}

// One token's down projection and weighted combine in one launch (moe.rs:376-383 after
// moe.rs:288-300): a workgroup owns R output rows and runs over the k routed experts' weight
// rows for them (lane l serves row l % R; the 64 / R lane groups of every wave take the chunks
// of expert after expert in turn, so one load reads R * 16 contiguous bytes), each dotted with
// that expert's SwiGLU row staged in LDS. The k sums of a row fold over lane groups by a fixed
// xor tree and over waves in wave order; then out[r] = sum over j in order of w[j] * y[j][r]
// (each a rounded multiply then a rounded add, from 0), skipping ids out of range, as the
// combine. Row blocks are given to XCDs in contiguous runs (workgroup b runs on XCD b % 8).
template <int T, int R, int WAVES, int D>
__global__ __launch_bounds__(WAVES * 64) void moe_down_combine_kernel(MoeDownCombineArgs a) {
  using B = Blk<T>;
  constexpr int NCH = B::NCH;
  constexpr int KM = kMoeOneTokenMaxK;
  constexpr int G = 64 / R;
  constexpr int S = WAVES * G;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const int nblk = (a.m + R - 1) / R;
  const int per = (nblk + 7) / 8;
  const int blk = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
  if (blk >= nblk) return;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int KP = a.KB * B::QK;
  float* hl = smem;                      // [k][KP]
  float* hs16 = smem + KM * KP;          // [k][KP/16]
  float* red = hs16 + KM * (KP / 16);    // [WAVES][KM][R]
  const int row = blk * R + (lane % R);
  const int tile = row >> 6, rr = row & 63;
  const int slot = wave * G + lane / R;
  const int u_pair = a.KB * NCH;         // units (chunks) per expert row
  const int k = a.k;
  int ex[KM];
  float wv[KM];
  bool ok[KM];
#pragma unroll
  for (int j = 0; j < KM; ++j) {
    ex[j] = j < k ? (a.ids ? a.ids[j] : a.id_v[j]) : -1;
    wv[j] = j < k ? (a.ids ? a.wts[j] : a.w_v[j]) : 0.0f;
    ok[j] = ex[j] >= 0 && ex[j] < a.n_experts;
  }
  // unit u: chunk u % u_pair of expert j = u / u_pair (an id out of range reads expert 0, unused)
  auto base_of = [&](int j) {
    int e = 0;
#pragma unroll
    for (int q = 0; q < KM; ++q)
      if (q == j && ok[q]) e = ex[q];
    return a.W + (size_t)e * a.w_stride + (size_t)tile * a.KB * B::SLAB;
  };
  const int u_end = k * u_pair;
  // this thread's first rows of h go out before the weight loads (loads retire in order, so
  // the staging then waits for them alone and overlaps the weights' round trip)
  constexpr int PRE = 4;
  const int nh = k * KP / 4;
  float4 hp[PRE];
#pragma unroll
  for (int r = 0; r < PRE; ++r) {
    const int i = (int)threadIdx.x + r * WAVES * 64;
    const int j = i / (KP / 4), q = 4 * (i - j * (KP / 4));
    hp[r] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (i < nh && q < a.K) hp[r] = *reinterpret_cast<const float4*>(a.H + (size_t)j * a.K + q);
  }
  __builtin_amdgcn_sched_barrier(0);
  typename B::CR ring[D];
#pragma unroll
  for (int i = 0; i < D; ++i) {
    // unconditional (a slot past the end reloads the last unit, never used): a load under a
    // branch made the compiler wait for it where the branch joins, one round trip per entry
    const int u = min(slot + i * S, u_end - 1);
    const int j = u / u_pair, c = u - j * u_pair;
    B::load_chunk(base_of(j) + (size_t)(c / NCH) * B::SLAB, rr, c % NCH, ring[i]);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int r = 0; r < PRE; ++r) {
    const int i = (int)threadIdx.x + r * WAVES * 64;
    if (i < nh) reinterpret_cast<float4*>(hl)[i] = hp[r];
  }
  for (int i = (int)threadIdx.x + PRE * WAVES * 64; i < nh; i += WAVES * 64) {
    const int j = i / (KP / 4), q = 4 * (i - j * (KP / 4));
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (q < a.K) v = *reinterpret_cast<const float4*>(a.H + (size_t)j * a.K + q);
    reinterpret_cast<float4*>(hl)[j * (KP / 4) + q / 4] = v;
  }
  __syncthreads();
  if constexpr (kNeedXs16<T>) {
    for (int i = threadIdx.x; i < k * (KP / 16); i += WAVES * 64) {
      const int j = i / (KP / 16), q = i - j * (KP / 16);
      const float4* hv = reinterpret_cast<const float4*>(hl + j * KP + 16 * q);
      float sum = 0.0f;
#pragma unroll
      for (int v = 0; v < 4; ++v) { const float4 t = hv[v]; sum += t.x; sum += t.y; sum += t.z; sum += t.w; }
      hs16[j * (KP / 16) + q] = sum;
    }
    __syncthreads();
  }
  float acc[KM];
#pragma unroll
  for (int j = 0; j < KM; ++j) acc[j] = 0.0f;
  for (int b0 = slot; b0 < u_end; b0 += D * S) {
#pragma unroll
    for (int i = 0; i < D; ++i) {
      const int u = b0 + i * S;
      if (u < u_end) {
        const int j = u / u_pair, c = u - j * u_pair;
        const int kb = c / NCH, cc = c - kb * NCH;
        Run ra, rb;
        B::decode_chunk(ring[i], cc, ra, rb);
        const int un = u + D * S;
        if (un < u_end) {
          const int jn = un / u_pair, cn = un - jn * u_pair;
          B::load_chunk(base_of(jn) + (size_t)(cn / NCH) * B::SLAB, rr, cn % NCH, ring[i]);
        }
        const float* hb = hl + j * KP + kb * B::QK;
        const float* hs = hs16 + j * (KP / 16) + kb * (B::QK / 16);
        const int valid = a.K - kb * B::QK;
        float d = 0.0f;
        if (ra.e < valid) d += run_dot<T>(ra, hb, hs);
        if (rb.e < valid) d += run_dot<T>(rb, hb, hs);
#pragma unroll
        for (int q = 0; q < KM; ++q)
          if (q == j) acc[q] += d;
      }
    }
  }
  // every expert slot's lane-group fold at once (slots past k hold zeros), so the shuffle rounds
  // of different slots overlap instead of running one slot after another
#pragma unroll
  for (int off = R; off < 64; off *= 2)
#pragma unroll
    for (int j = 0; j < KM; ++j) acc[j] += __shfl_xor(acc[j], off, 64);
  if (lane < R) {
#pragma unroll
    for (int j = 0; j < KM; ++j) red[(wave * KM + j) * R + lane] = acc[j];
  }
  __syncthreads();
  // wave 0: lane (j, r) = (lane / R, lane % R) adds slot j's wave sums for row r in wave order;
  // lane r then gathers the KM slot sums and combines them in slot order
  static_assert(R * KM == 64, "one lane per (slot, row)");
  if (wave == 0) {
    const int j = lane / R, r = lane % R;
    float y = red[(0 * KM + j) * R + r];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) y += red[(w * KM + j) * R + r];
    float ys[KM];
#pragma unroll
    for (int q = 0; q < KM; ++q) ys[q] = __shfl(y, q * R + r, 64);
    if (lane < R) {
      float o = 0.0f;
#pragma unroll
      for (int q = 0; q < KM; ++q)
        if (q < k && ok[q]) o = __fadd_rn(o, __fmul_rn(wv[q], ys[q]));
      const int orow = blk * R + r;
      if (orow < a.m) a.out[orow] = o;
    }
  }
}

// 8 rows a workgroup (256 workgroups at hidden 2048), 8 waves (measured 15.7 against 17.6 us for 4
// waves at the Qwen3-30B-A3B shape, and slower with 16 waves or 4 loads in flight per slot)
constexpr int kDownCombineRows = 8, kDownCombineWaves = 8;

template <int T>
static size_t down_combine_lds(int KB) {
  const size_t KP = (size_t)KB * Blk<T>::QK;
  return (kMoeOneTokenMaxK * KP * 17 / 16 + (size_t)kDownCombineWaves * kMoeOneTokenMaxK * kDownCombineRows) *
         sizeof(float);
}

template <int T>
static hipError_t launch_down_combine_t(const MoeDownCombineArgs& a, hipStream_t s) {
  const size_t lds = down_combine_lds<T>(a.KB);
  if (lds > kMaxLdsBytes || a.k < 1 || a.k > kMoeOneTokenMaxK) return hipErrorInvalidValue;
  const int nblk = (a.m + kDownCombineRows - 1) / kDownCombineRows;
  const unsigned grid = (unsigned)((nblk + 7) / 8 * 8);
  hipLaunchKernelGGL((moe_down_combine_kernel<T, kDownCombineRows, kDownCombineWaves, 2>), dim3(grid),
                     dim3(kDownCombineWaves * 64), lds, s, a);
  return hipGetLastError();
}

size_t moe_down_combine_lds(uint32_t type, int KB, int k) {
  (void)k;
  switch (type) {
    case T_Q4_0: return down_combine_lds<T_Q4_0>(KB);
    case T_Q5_0: return down_combine_lds<T_Q5_0>(KB);
    case T_Q8_0: return down_combine_lds<T_Q8_0>(KB);
    case T_Q4_K: return down_combine_lds<T_Q4_K>(KB);
    case T_Q5_K: return down_combine_lds<T_Q5_K>(KB);
    case T_Q6_K: return down_combine_lds<T_Q6_K>(KB);
    default: return ~(size_t)0;
  }
}

hipError_t launch_moe_down_combine(uint32_t type, const MoeDownCombineArgs& a, hipStream_t s) {
  switch (type) {
    case T_Q4_0: return launch_down_combine_t<T_Q4_0>(a, s);
    case T_Q5_0: return launch_down_combine_t<T_Q5_0>(a, s);
    case T_Q8_0: return launch_down_combine_t<T_Q8_0>(a, s);
    case T_Q4_K: return launch_down_combine_t<T_Q4_K>(a, s);
    case T_Q5_K: return launch_down_combine_t<T_Q5_K>(a, s);
    case T_Q6_K: return launch_down_combine_t<T_Q6_K>(a, s);
    default: return hipErrorInvalidValue;
  }
}

template <int T, bool DUAL, int NB, int R = kMoeGemvRows, int W = kMoeGemvWaves>
static hipError_t launch_moe_gemv_nb(const MoeGemvArgs& a, int ntasks, hipStream_t s) {
  const int KP = a.KB * Blk<T>::QK;
  const size_t lds = ((size_t)NB * KP * 17 / 16 + (size_t)W * (DUAL ? 2 : 1) * NB * R + (size_t)W * NB) * sizeof(float);
  if ((size_t)a.KB * Blk<T>::NCH <= (size_t)W * 64 / R)
    hipLaunchKernelGGL((moe_gemv_kernel<T, R, W, NB, DUAL, true>), dim3((unsigned)ntasks), dim3(W * 64), lds, s, a);
  else
    hipLaunchKernelGGL((moe_gemv_kernel<T, R, W, NB, DUAL, false>), dim3((unsigned)ntasks), dim3(W * 64), lds, s, a);
  return hipGetLastError();
}

// tasks of at most one gathered row use the single-row instance (no idle activation slots)
template <int T, bool DUAL>
static hipError_t launch_moe_gemv_t(const MoeGemvArgs& a, int ntasks, hipStream_t s) {
  if (a.rows_per_task == kFfnGemvRows) {
    if constexpr (DUAL) {
      // one row: eight waves, one chunk of each matrix per lane (the launch is latency-bound;
      // measured in the Qwen2.5-0.5B decode step: 787 -> 779 us per token)
      if (a.max_rows <= 1) return launch_moe_gemv_nb<T, true, 1, kFfnGemvRows, 8>(a, ntasks, s);
    }
    return hipErrorInvalidValue;
  }
  if (a.rows_per_task == 64) {
    if constexpr (!DUAL) {
      return a.max_rows <= 1 ? launch_moe_gemv_nb<T, false, 1, 64>(a, ntasks, s)
                             : launch_moe_gemv_nb<T, false, kMoeGemvBatch, 64>(a, ntasks, s);
    }
    return hipErrorInvalidValue;
  }
  if (a.rows_per_task != kMoeGemvRows) return hipErrorInvalidValue;
  return a.max_rows <= 1 ? launch_moe_gemv_nb<T, DUAL, 1>(a, ntasks, s)
                         : launch_moe_gemv_nb<T, DUAL, kMoeGemvBatch>(a, ntasks, s);
}

hipError_t launch_moe_gemv(uint32_t type, bool dual, const MoeGemvArgs& a, int ntasks, hipStream_t s) {
  if (ntasks == 0) return hipSuccess;
  switch (type) {
    case T_Q4_0: return dual ? launch_moe_gemv_t<T_Q4_0, true>(a, ntasks, s) : launch_moe_gemv_t<T_Q4_0, false>(a, ntasks, s);
    case T_Q5_0: return dual ? launch_moe_gemv_t<T_Q5_0, true>(a, ntasks, s) : launch_moe_gemv_t<T_Q5_0, false>(a, ntasks, s);
    case T_Q8_0: return dual ? launch_moe_gemv_t<T_Q8_0, true>(a, ntasks, s) : launch_moe_gemv_t<T_Q8_0, false>(a, ntasks, s);
    case T_Q4_K: return dual ? launch_moe_gemv_t<T_Q4_K, true>(a, ntasks, s) : launch_moe_gemv_t<T_Q4_K, false>(a, ntasks, s);
    case T_Q5_K: return dual ? launch_moe_gemv_t<T_Q5_K, true>(a, ntasks, s) : launch_moe_gemv_t<T_Q5_K, false>(a, ntasks, s);
    case T_Q6_K: return dual ? launch_moe_gemv_t<T_Q6_K, true>(a, ntasks, s) : launch_moe_gemv_t<T_Q6_K, false>(a, ntasks, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace rehip
