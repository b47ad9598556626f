// Qwen3.6 gated full-attention decode step for gfx950 (the mixer of one
// layer in four; the MoE layer follows it).
//
// Semantics (reference kernels/triton/qwen36_attention.py:448-577; oracle
// reference/qwen36_real.py:283-326):
//   xn = RMSNorm(x) * (1 + w)
//   per head h: [q_h | gate_h] = rows 2hd*h .. 2hd*h + 2hd - 1 of xn Wq^T
//   k = xn Wk^T, v = xn Wv^T                      (kv head j serves heads j*G .. j*G + G - 1)
//   q_h = RMSNorm(q_h) * (1 + w_q), k_j = RMSNorm(k_j) * (1 + w_k)   (over head_dim)
//   RoPE of the first rope_dim dims at position p = start + t:
//     interleaved pairs (2i, 2i+1) (the Triton entry point and its test) or
//     halves (i, i + rope_dim/2) (the torch oracle), angle p * theta^(-2i/rope_dim)
//   cache[start + t] = (k, v); o_h = softmax(q_h . K_j[0..p] / sqrt(hd)) V_j[0..p]
//   update = (o * sigmoid(gate)) Wo^T;  hidden_out = x + update
//
// Kernels: T <= 4 at the shapes attn_step_chunks accepts (the model's) run
// as one launch, attn_step_kernel (below); other steps as four launches:
//   attn_proj_kernel  RMSNorm folded into a GEMV over [Wq | Wk | Wv] (9216
//                     rows at the model shape); H > 2048 takes the shared
//                     normalized projection kernel of fk_deltanet.hip
//   attn_split_kernel grid (position chunks, kv heads, T), 256 threads: the
//                     G query heads of one kv head over one chunk of
//                     positions (each cached row read once per chunk), head
//                     norms and RoPE in LDS, the step's new keys recomputed
//                     from k (no dependence on another workgroup's cache
//                     write), online softmax; a single chunk writes the
//                     gated output, more chunks leave per-chunk partials
//   attn_merge_kernel grid (heads, T), one thread per dim: merges the chunk
//                     partials and applies the gate (returns at once when
//                     one chunk covered the positions)
//   attn_out_kernel   grid ceil(H/4): 4 rows of Wo per workgroup (1 per
//                     wavefront, loaded once) against every token; residual;
//                     advances a device-held position
#include "fk_common.h"
#include "fk_host.h"

#include <type_traits>

namespace fk {

constexpr int kAttnMaxHeadDim = 256;
constexpr int kAttnMaxTokens = 32;  // new keys of the step are kept in LDS (T * hd floats)
constexpr int kAttnOutRows = 4;  // Wo rows per out-projection workgroup (1 per wavefront)

struct AttnArgs {
  const float* qg;      // [T, heads * 2 * hd] projected query/gate pairs
  const float* k;       // [T, kv_heads * hd]
  const float* v;       // [T, kv_heads * hd]
  const void* qn_w;     // [hd]
  const void* kn_w;     // [hd]
  int qn_dt, kn_dt;
  void* kc;             // [max_pos, kv_heads, hd]
  void* vc;
  const int* start_dev; // when set: the start position, read at run time (graph replays)
  int start, max_pos;
  int T, heads, kvh, hd, rope_dim;
  float theta_log2, eps;
  int interleaved;
  float* gated;         // [T, heads * hd]  o * sigmoid(gate)
  float* part;          // [T, heads, max_chunks, hd + 2] per-chunk (max, sum, weighted values)
  int chunk, max_chunks;
  int hsplit;           // workgroups per kv head: each takes G / hsplit of its query heads
};

constexpr int kAttnMaxKvHeads = 64;
constexpr int kAttnMaxChunks = 64;  // position chunks per (token, kv head): the merge reads at most this many

template <bool BF>
__device__ __forceinline__ float4 load4(const void* p, size_t i) {
  if constexpr (BF) {
    const uint2 r = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(p) + i);
    return make_float4(__uint_as_float(r.x << 16), __uint_as_float(r.x & 0xffff0000u), __uint_as_float(r.y << 16),
                       __uint_as_float(r.y & 0xffff0000u));
  } else {
    return *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + i);
  }
}

// Four consecutive elements of a cache row, raw (bf16: 8 bytes, converted
// where used, so a pass of rows in flight takes half the registers).
template <bool BF>
struct Row4 {
  typename std::conditional<BF, uint2, float4>::type r;
  __device__ __forceinline__ float4 f4() const {
    if constexpr (BF)
      return make_float4(__uint_as_float(r.x << 16), __uint_as_float(r.x & 0xffff0000u), __uint_as_float(r.y << 16),
                         __uint_as_float(r.y & 0xffff0000u));
    else
      return r;
  }
};
template <bool BF>
__device__ __forceinline__ Row4<BF> load_row4(const void* p, size_t i) {
  Row4<BF> v;
  if constexpr (BF) v.r = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(p) + i);
  else v.r = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + i);
  return v;
}

template <bool BF>
__device__ __forceinline__ void store1(void* p, size_t i, float v) {
  if constexpr (BF) reinterpret_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v);
  else reinterpret_cast<float*>(p)[i] = v;
}

// Sum over the workgroup's 256 threads (one value each); every thread gets it.
__device__ __forceinline__ float block256_sum(float v, float* s_red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_sum(v);
  __syncthreads();  // s_red may still be read from a previous call
  if (lane == 0) s_red[wave] = v;
  __syncthreads();
  return (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
}

// RMSNorm(1 + w) and RoPE at `pos` of one head held one dim per thread
// (thread d < hd; wd: the norm weight of dim d); `s_vec` is the head's LDS
// row.  Returns dim d's value.
__device__ __forceinline__ float norm_rope(float x, float wd, const AttnArgs& a, int pos, float* s_vec, float* s_red) {
  const int d = threadIdx.x;
  const bool in = d < a.hd;
  const float ss = block256_sum(in ? x * x : 0.f, s_red);
  float y = in ? x * rsqrtf(ss / (float)a.hd + a.eps) * (1.f + wd) : 0.f;
  const int rd = a.rope_dim;
  if (in) s_vec[d] = y;
  __syncthreads();
  if (d < rd) {
    int i, partner;
    float sign;
    if (a.interleaved) {
      i = d >> 1;
      partner = d ^ 1;
      sign = (d & 1) ? 1.f : -1.f;
    } else {
      const int h = rd >> 1;
      i = d < h ? d : d - h;
      partner = d < h ? d + h : d - h;
      sign = d < h ? -1.f : 1.f;
    }
    // angle = pos * theta^(-2i / rd), as the reference (fp32)
    const float inv_freq = exp2f(-(float)(2 * i) / (float)rd * a.theta_log2);
    float sn, cs;
    sincosf((float)pos * inv_freq, &sn, &cs);
    y = y * cs + sign * s_vec[partner] * sn;
  }
  __syncthreads();  // s_vec is reused by the caller
  return y;
}

// Workgroup (chunk c, kv head j, token t): positions c*C .. c*C + C - 1 (of
// 0 .. p, p = start + t) for the G <= 8 query heads of kv head j, so each
// cached row is read once per chunk.  Wavefront w takes positions c*C + w,
// + 4, .., eight in flight; per position the G dot products are summed over
// the lanes at once (rows8_sum) and each head keeps an online softmax (max,
// sum, 4 dims of the weighted value sum per lane).  The wavefronts' states
// are combined through LDS; with one chunk the gated output is written
// here, otherwise the chunk's per-head partials go to the workspace and
// attn_merge_kernel combines the chunks (a separate launch: merging in the
// last workgroup to arrive costs a device-scope release/acquire per
// workgroup and a serial chain of partial loads in that workgroup).
template <bool CBF>
__global__ __launch_bounds__(256) void attn_split_kernel(AttnArgs a) {
  constexpr int MAXG = 8, NB = CBF ? 4 : 8;  // (a bf16 cache also holds its step's own values: fewer rows in flight)
  extern __shared__ float4 s_dyn[];  // [G][hd] scaled queries, then [T][hd] new keys
  __shared__ float s_tmp[kAttnMaxHeadDim];
  __shared__ float s_red[4];
  __shared__ float s_m[4][MAXG], s_l[4][MAXG];
  __shared__ __align__(16) float s_acc[4][MAXG][kAttnMaxHeadDim];
  __shared__ float s_ss[4][MAXG];
  const int c = blockIdx.x, j = blockIdx.y / a.hsplit, hs = blockIdx.y - j * a.hsplit, t = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hd = a.hd, G = a.heads / a.kvh / a.hsplit;  // query heads of this workgroup
  const int hb = j * (a.heads / a.kvh) + hs * G;          // the first of them
  const int qw = a.heads * hd, kvw = a.kvh * hd;
  const bool in = tid < hd;
  float* s_q = reinterpret_cast<float*>(s_dyn);
  float* s_knew = s_q + MAXG * hd;
  // The queries, gates and norm weights do not depend on the position: they
  // are loaded before it, so the position's round trip overlaps theirs.
  float xq[MAXG], sq[MAXG];
  float gate[MAXG];  // this thread's gate values (used at the end)
  const int dq = in ? tid : 0;
#pragma unroll
  for (int g = 0; g < MAXG; ++g) {
    const size_t qb = (size_t)t * 2 * qw + (size_t)(hb + min(g, G - 1)) * 2 * hd + dq;
    xq[g] = a.qg[qb];
    gate[g] = a.qg[qb + hd];
  }
  const uint32_t qnw = elem_word(a.qn_w, a.qn_dt, dq);
  const uint32_t knw = elem_word(a.kn_w, a.kn_dt, dq);
  const int start = a.start_dev ? *a.start_dev : a.start;
  if (start < 0 || start + a.T > a.max_pos) {
    // a run-time position past the cache: no cache access, NaN outputs
    if (c == 0 && in)
      for (int g = 0; g < G; ++g) a.gated[(size_t)t * qw + (size_t)(hb + g) * hd + tid] = __builtin_nanf("");
    return;
  }
  const int pos = start + t, C = a.chunk;
  const int nc = (pos + C) / C;  // chunks covering 0 .. pos
  if (c >= nc) return;
  const int p_lo = c * C, p_hi = min(p_lo + C, pos + 1);

  // Loads first, in the order their data is used: the queries (and gates,
  // above), then this wavefront's first pass of cached rows, which arrive
  // while the queries are normalised and rotated.  Every load is unconditional
  // (clamped in range, unused values dropped after): a load under a
  // condition makes the compiler wait for the loads before it.
  const int d0 = lane * 4;
  const bool lin = d0 < hd;
  const int dl = lin ? d0 : 0;  // (idle lanes read dim 0)
  float4 q4[MAXG], acc[MAXG];
  float m[MAXG], l[MAXG];
  // OWN: the chunk holds some of the step's own positions (start ..), whose
  // keys are recomputed here and whose values come from v; their cache rows
  // are stale and are read only to keep the loads unconditional.
  auto body = [&](auto own_tag) {
    constexpr bool OWN = decltype(own_tag)::value;
    // the first own position's k (OWN chunks)
    const int u_lo = max(p_lo, start) - start, u_hi = p_hi - 1 - start;
    const float k_first = a.k[(size_t)(OWN ? u_lo : 0) * kvw + (size_t)j * hd + dq];
    // (an fp32 cache takes the step's own values from v with the same load,
    // its address chosen arithmetically; a bf16 cache loads both)
    constexpr bool VN = OWN && CBF;
    Row4<CBF> kk[NB], vv[NB];
    float4 vn[VN ? NB : 1];
    auto load_pass = [&](int p0) {
#pragma unroll
      for (int bb = 0; bb < NB; ++bb) {
        const int p = min(p0 + 4 * bb, p_hi - 1);
        const size_t cr = ((size_t)p * a.kvh + j) * hd + dl;
        kk[bb] = load_row4<CBF>(a.kc, cr);
        if constexpr (OWN && !CBF) {
          const float* vsrc = p >= start ? a.v + (size_t)(p - start) * kvw + (size_t)j * hd + dl
                                         : reinterpret_cast<const float*>(a.vc) + cr;
          vv[bb] = load_row4<CBF>(vsrc, 0);  // (CBF false here)
        } else {
          vv[bb] = load_row4<CBF>(a.vc, cr);
        }
        if constexpr (VN)
          vn[bb] = *reinterpret_cast<const float4*>(a.v + (p >= start ? (size_t)(p - start) * kvw : 0) + (size_t)j * hd + dl);
      }
    };
    const int p_first = p_lo + wave;
    load_pass(p_first);

    // queries of the G heads at once (thread d: dim d of every head): norms
    // from one transposed lane reduction, RoPE at pos, 1/sqrt(hd)
#pragma unroll
    for (int g = 0; g < MAXG; ++g) {
      xq[g] = in && g < G ? xq[g] : 0.f;
      sq[g] = xq[g] * xq[g];
    }
    const float r = rows8_sum(sq);
    if ((lane & 7) == 0) s_ss[wave][lane >> 3] = r;
    __syncthreads();
    const float wq = in ? 1.f + elem_value(qnw, a.qn_w, a.qn_dt, dq) : 0.f;
#pragma unroll
    for (int g = 0; g < MAXG; ++g) {
      const float tot = (s_ss[0][g] + s_ss[1][g]) + (s_ss[2][g] + s_ss[3][g]);
      xq[g] = xq[g] * rsqrtf(tot / (float)hd + a.eps) * wq;
      if (in && g < G) s_q[g * hd + tid] = xq[g];
    }
    __syncthreads();
    const int rd = a.rope_dim;
    if (tid < rd) {
      int i, partner;
      float sign;
      if (a.interleaved) {
        i = tid >> 1;
        partner = tid ^ 1;
        sign = (tid & 1) ? 1.f : -1.f;
      } else {
        const int hh = rd >> 1;
        i = tid < hh ? tid : tid - hh;
        partner = tid < hh ? tid + hh : tid - hh;
        sign = tid < hh ? -1.f : 1.f;
      }
      const float inv_freq = exp2f(-(float)(2 * i) / (float)rd * a.theta_log2);
      float sn, cs;
      sincosf((float)pos * inv_freq, &sn, &cs);
#pragma unroll
      for (int g = 0; g < MAXG; ++g)
        if (g < G) xq[g] = xq[g] * cs + sign * s_q[g * hd + partner] * sn;
    }
    __syncthreads();
    const float scale = rsqrtf((float)hd);
#pragma unroll
    for (int g = 0; g < MAXG; ++g)
      if (in && g < G) s_q[g * hd + tid] = xq[g] * scale;
    if constexpr (OWN) {
      // new keys of this chunk's positions (start .. pos), from k
      const float wk = elem_value(knw, a.kn_w, a.kn_dt, dq);
      for (int u = u_lo; u <= u_hi; ++u) {
        const float kx = u == u_lo ? k_first : a.k[(size_t)u * kvw + (size_t)j * hd + dq];
        const float kr = norm_rope(in ? kx : 0.f, wk, a, start + u, s_tmp, s_red);
        if (in) s_knew[u * hd + tid] = kr;
      }
      // the chunk holding position pos writes token t's cache row of kv head j
      if (c == nc - 1 && in) {
        const size_t cr = ((size_t)pos * a.kvh + j) * hd + tid;
        store1<CBF>(a.kc, cr, s_knew[t * hd + tid]);
        store1<CBF>(a.vc, cr, a.v[(size_t)t * kvw + (size_t)j * hd + tid]);
      }
    }
    __syncthreads();

#pragma unroll
    for (int g = 0; g < MAXG; ++g) {
      q4[g] = lin && g < G ? *reinterpret_cast<const float4*>(s_q + g * hd + d0) : make_float4(0.f, 0.f, 0.f, 0.f);
      acc[g] = make_float4(0.f, 0.f, 0.f, 0.f);
      m[g] = -INFINITY;
      l[g] = 0.f;
    }
    // passes of NB positions per wavefront (c*C + w, + 4, ..), the first one
    // already loaded; the step's own keys and values are selected per
    // position after the loads
    for (int p0 = p_first; p0 < p_hi; p0 += 4 * NB) {
      if (p0 != p_first) load_pass(p0);
      // the pass's scores for every head (independent of each other), then
      // per head one softmax step over the pass: one max, NB independent
      // exponentials and one rescale of (m, l, acc), not a serial online
      // update per position.  Positions past the chunk score -inf.
      float sr[NB];  // lanes 8g ..: head g's score at position p0 + 4 bb
#pragma unroll
      for (int bb = 0; bb < NB; ++bb) {
        float4 k4 = kk[bb].f4();
        if constexpr (OWN) {
          if (p0 + 4 * bb >= start && p0 + 4 * bb < p_hi)  // (uniform per wavefront)
            k4 = *reinterpret_cast<const float4*>(s_knew + (p0 + 4 * bb - start) * hd + dl);
        }
        float d[MAXG];
#pragma unroll
        for (int g = 0; g < MAXG; ++g) d[g] = q4[g].x * k4.x + q4[g].y * k4.y + q4[g].z * k4.z + q4[g].w * k4.w;
        sr[bb] = rows8_sum(d);
      }
#pragma unroll
      for (int g = 0; g < MAXG; ++g) {
        if (g >= G) break;
        float sc[NB];
        float mx = m[g];
#pragma unroll
        for (int bb = 0; bb < NB; ++bb) {
          sc[bb] = p0 + 4 * bb < p_hi ? __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(sr[bb]), 8 * g)) : -INFINITY;
          mx = fmaxf(mx, sc[bb]);
        }
        const float f = __expf(m[g] - mx);  // (mx is finite: position p0 exists)
        float es = 0.f;
        float4 av = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int bb = 0; bb < NB; ++bb) {
          const float e = __expf(sc[bb] - mx);
          float4 v4 = vv[bb].f4();
          if constexpr (VN) {
            if (p0 + 4 * bb >= start) v4 = vn[bb];  // (uniform per wavefront)
          }
          es += e;
          av.x = fmaf(e, v4.x, av.x);
          av.y = fmaf(e, v4.y, av.y);
          av.z = fmaf(e, v4.z, av.z);
          av.w = fmaf(e, v4.w, av.w);
        }
        l[g] = l[g] * f + es;
        acc[g].x = acc[g].x * f + av.x;
        acc[g].y = acc[g].y * f + av.y;
        acc[g].z = acc[g].z * f + av.z;
        acc[g].w = acc[g].w * f + av.w;
        m[g] = mx;
      }
    }
  };
  if (p_hi - 1 >= start) body(std::true_type{});
  else body(std::false_type{});
  // merge the 4 wavefronts, every head in one pass (thread d: dim d): one
  // chunk (short contexts) writes the gated output directly; otherwise the
  // chunk partial (m, l, acc[hd]) goes to the workspace for attn_merge_kernel
#pragma unroll
  for (int g = 0; g < MAXG; ++g) {
    if (g < G) {
      if (lane == 0) {
        s_m[wave][g] = m[g];
        s_l[wave][g] = l[g];
      }
      if (lin) *reinterpret_cast<float4*>(&s_acc[wave][g][d0]) = acc[g];
    }
  }
  __syncthreads();
  const int maxc = a.max_chunks;
#pragma unroll
  for (int g = 0; g < MAXG; ++g) {
    if (g >= G) break;
    const float M = fmaxf(fmaxf(s_m[0][g], s_m[1][g]), fmaxf(s_m[2][g], s_m[3][g]));
    float L = 0.f, o = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float f = s_m[w][g] == -INFINITY ? 0.f : __expf(s_m[w][g] - M);
      L += s_l[w][g] * f;
      o += in ? s_acc[w][g][tid] * f : 0.f;
    }
    if (nc == 1) {
      if (in) a.gated[(size_t)t * qw + (size_t)(hb + g) * hd + tid] = (o / L) * sigmoid(gate[g]);
    } else {
      float* part = a.part + ((size_t)(t * a.heads + hb + g) * maxc + c) * (hd + 2);
      if (in) part[2 + tid] = o;
      if (tid == 0) {
        part[0] = M;
        part[1] = L;
      }
    }
  }
}

// Merge of the chunk partials of (query head h, token t): thread d holds
// dim d.  The partials' values are loaded at once (up to kAttnMaxChunks per
// thread, clamped in range), the chunk statistics by the first nc threads
// into LDS; the chunks are combined in chunk order against the largest
// chunk maximum (as the split kernel combines its wavefronts), then gated.
struct AttnMergeArgs {
  const float* qg;
  const float* part;
  float* gated;
  const int* start_dev;
  int start, max_pos, T, heads, hd, chunk, max_chunks;
};

__global__ __launch_bounds__(256) void attn_merge_kernel(AttnMergeArgs a) {
  __shared__ float s_mc[kAttnMaxChunks], s_lc[kAttnMaxChunks];
  const int h = blockIdx.x, t = blockIdx.y, d = threadIdx.x;
  const int hd = a.hd, dd = d < hd ? d : 0;
  // Every partial row exists (max_chunks per head), so all loads are issued
  // before the position is known; rows past the chunk count are dropped.
  const float* base = a.part + (size_t)(t * a.heads + h) * a.max_chunks * (hd + 2);
  float ov[kAttnMaxChunks];
#pragma unroll
  for (int c = 0; c < kAttnMaxChunks; ++c) ov[c] = base[(size_t)c * (hd + 2) + 2 + dd];
  const float gate = a.qg[(size_t)t * 2 * a.heads * hd + (size_t)h * 2 * hd + hd + dd];
  const int dc = min(d, kAttnMaxChunks - 1);
  const float mc = base[(size_t)dc * (hd + 2)], lc = base[(size_t)dc * (hd + 2) + 1];
  const int start = a.start_dev ? *a.start_dev : a.start;
  if (start < 0 || start + a.T > a.max_pos) return;  // the split kernel wrote NaN outputs
  const int pos = start + t, nc = (pos + a.chunk) / a.chunk;
  if (nc == 1) return;  // the split kernel wrote the gated output itself
  if (d < kAttnMaxChunks) {
    s_mc[d] = mc;
    s_lc[d] = lc;
  }
  __syncthreads();
  float M = -INFINITY;
  for (int c = 0; c < nc; ++c) M = fmaxf(M, s_mc[c]);
  float L = 0.f, o = 0.f;
#pragma unroll
  for (int c = 0; c < kAttnMaxChunks; ++c) {
    if (c < nc) {
      const float f = s_mc[c] == -INFINITY ? 0.f : __expf(s_mc[c] - M);
      L += s_lc[c] * f;
      o += ov[c] * f;
    }
  }
  if (d < hd) a.gated[(size_t)t * a.heads * hd + (size_t)h * hd + d] = (o / L) * sigmoid(gate);
}

// Normalised projection of the attention inputs: rows of [Wq | Wk | Wv]
// (16 per workgroup, 4 whole rows per wavefront in registers), every token.
// RMSNorm(x) * (1 + w) is folded in: acc = sum W[r,c] * x[c] * (1 + w[c]),
// out = acc * rsqrt(mean(x^2) + eps).  Token 0's x and the norm weight are
// loaded before the rows (the load queue retires in order); the four row
// sums leave through one transposed lane reduction.
struct AttnProjArgs {
  const void* x;
  const void* nw;
  int nw_dt;
  const void* w[3];
  float* out[3];
  int rows[3];
  int T, H;
  float eps, off;
};
constexpr int kAttnProjRows = 16;

template <bool BFW, bool BFX>
__global__ __launch_bounds__(256) void attn_proj_kernel(AttnProjArgs a) {
  constexpr int NJ = 4;  // H <= 2048: 4 chunks of 8 per lane
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nch = a.H >> 3;
  int row = blockIdx.x * kAttnProjRows + wave * 4;  // first of this wavefront's 4 rows (one matrix)
  const int R = a.rows[0] + a.rows[1] + a.rows[2];
  if (row >= R) return;
  int m = 0;
  if (row >= a.rows[0]) {
    row -= a.rows[0];
    m = 1;
    if (row >= a.rows[1]) {
      row -= a.rows[1];
      m = 2;
    }
  }
  const char* W = reinterpret_cast<const char*>(m == 0 ? a.w[0] : m == 1 ? a.w[1] : a.w[2]);
  float* out = m == 0 ? a.out[0] : m == 1 ? a.out[1] : a.out[2];
  const int ostride = m == 0 ? a.rows[0] : m == 1 ? a.rows[1] : a.rows[2];
  const size_t esz = BFW ? 2 : 4;
  Raw8<BFX> xr[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int cc = min(lane + kWave * j, nch - 1);
    xr[j] = load_raw8<BFX>(a.x, (size_t)cc * 8);
  }
  float nw8[NJ][8];
#pragma unroll
  for (int j = 0; j < NJ; ++j) load8_any(a.nw, a.nw_dt, (size_t)min(lane + kWave * j, nch - 1) * 8, nw8[j]);
  Raw8<BFW> wr[4][NJ];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int c = min(lane + kWave * j, nch - 1);
      wr[r][j] = load_raw8_stream<BFW>(W + (size_t)(row + r) * a.H * esz, (size_t)c * 8);
    }
  for (int t = 0; t < a.T; ++t) {
    if (t > 0) {
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        xr[j] = load_raw8<BFX>(a.x, (size_t)t * a.H + (size_t)min(lane + kWave * j, nch - 1) * 8);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        asm volatile("" : "+v"(wr[r][j].a));  // rows converted where used, once per token
        if constexpr (!BFW) asm volatile("" : "+v"(wr[r][j].b));
      }
    float acc[4] = {0.f, 0.f, 0.f, 0.f}, ss = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if (lane + kWave * j < nch) {
        float x8[8];
        raw8_to_f32<BFX>(xr[j], x8);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          ss = fmaf(x8[q], x8[q], ss);
          x8[q] *= a.off + nw8[j][q];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float w8[8];
          raw8_to_f32<BFW>(wr[r][j], w8);
#pragma unroll
          for (int q = 0; q < 8; ++q) acc[r] = fmaf(w8[q], x8[q], acc[r]);
        }
      }
    }
    ss = wave_sum(ss);
    const float v = rows4_sum(acc) * rsqrtf(ss / (float)a.H + a.eps);  // lanes 16r ..: row r
    if ((lane & 15) == 0) out[(size_t)t * ostride + row + (lane >> 4)] = v;
  }
}

struct AttnOutArgs {
  const float* gated;  // [T, K]
  const void* wo;      // [H, K]
  const void* x;       // [T, H] residual input (NULL: no residual output)
  int x_dt;
  int T, H, K;
  float* update;
  float* hidden_out;
  int* advance;  // nullable: *advance += T at the end of the step (device-held position)
  int max_pos;   // the cache length: a position whose step would pass it is not advanced
  uint32_t* err; // the workspace's error word (FK_DEVICE_ERR_POSITION)
};

// 4 rows of Wo per workgroup (1 per wavefront), K <= 4096, loaded once and
// applied to every token.
template <bool BFW>
__global__ __launch_bounds__(256) void attn_out_kernel(AttnOutArgs a) {
  constexpr int NJ = 8, RPW = kAttnOutRows / 4;  // rows per wavefront
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r0 = blockIdx.x * kAttnOutRows + wave * RPW;
  const int nch = a.K >> 3;
  Raw8<BFW> wr[RPW][NJ];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int q = 0; q < NJ; ++q) {
      const int c = lane + kWave * q;
      if (c < nch && r0 + r < a.H) wr[r][q] = load_raw8_stream<BFW>(a.wo, (size_t)(r0 + r) * a.K + (size_t)c * 8);
    }
  for (int t = 0; t < a.T; ++t) {
    float acc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) acc[r] = 0.f;
#pragma unroll
    for (int q = 0; q < NJ; ++q) {
      const int c = lane + kWave * q;
      if (c < nch) {
        float g8[8];
        load8_act(a.gated, (size_t)t * a.K + (size_t)c * 8, g8);
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
          float w8[8];
          raw8_to_f32<BFW>(wr[r][q], w8);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[r] = fmaf(w8[e], g8[e], acc[r]);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) acc[r] = wave_sum(acc[r]);
    if (lane < RPW && r0 + lane < a.H) {
      float u = acc[0];
#pragma unroll
      for (int r = 1; r < RPW; ++r) u = lane == r ? acc[r] : u;
      const size_t o = (size_t)t * a.H + r0 + lane;
      a.update[o] = u;
      if (a.hidden_out) a.hidden_out[o] = load_scalar(a.x, a.x_dt, o) + u;
    }
  }
  // the attention launch before this one has read the position; one whose
  // step would pass the cache (NaN update) stays, and the error word says so
  if (a.advance && blockIdx.x == 0 && threadIdx.x == 0) {
    const int s0 = *a.advance;
    if (s0 >= 0 && s0 + a.T <= a.max_pos) *a.advance = s0 + a.T;
    else __hip_atomic_fetch_or(a.err, FK_DEVICE_ERR_POSITION, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---------------------------------------------------------------------------
// Single-launch attention step (fk_attention_decode for T <= 4 at the shapes
// attn_step_eligible accepts; the model's: hidden 2048, 16 query and 2 kv
// heads of 256, bf16 weights).  One 512-thread workgroup per CU, grid capped
// at the co-resident capacity; phases joined by launch-tagged words (value +
// 32-bit launch tag per 8-byte word, polled by the consumers, as in the MoE
// layer and the DeltaNet step).  Every consumer polls its inputs directly
// (waiting on hint words of its producers first cost a memory round trip
// more; the attention units' first round is in flight while they compute
// the RoPE angles):
//   A   projections: the R rows of [Wq | Wk | Wv] split evenly over the grid
//       (36 per workgroup at the model shape, 4 or 5 per wavefront), each a
//       whole-row dot product with the tokens x * (1 + w) staged in LDS,
//       times the token's rsqrt(mean(x^2) + eps); outputs leave tagged.
//   B   attention unit (t, j, hs, c), one per workgroup at the model shape:
//       query heads hs * 4 .. + 4 of kv head j for token t over chunk c of
//       its positions 0 .. start + t (split evenly over nch chunks at run
//       time; the chunk's first cached rows are fetched with the unit's
//       inputs and staged in LDS after the norms).  RoPE angles are computed
//       once per position; wavefronts 0-3 normalise and rotate the queries,
//       4-7 the step's own keys, recomputed from k (its own values come from
//       v: no dependence on another workgroup's cache write); 8 wavefronts
//       each keep an online softmax over their positions, merged through
//       LDS.  The chunk's (max, sum, weighted values) per head leave tagged,
//       and the chunk holding position start + t writes that token's cache
//       rows of kv head j.
//   M   merge unit (t, h, ds) on the last workgroups: dims 64 ds .. + 64 of
//       head h over the nch chunks, times sigmoid(gate); leaves the gated
//       values tagged.
//   C1  unit (rb, ks) on the first workgroups: rows 128 rb .. + 128 of Wo
//       restricted to columns 512 ks .. + 512 (fetched into registers when
//       the unit's attention role is done) against the gated values of
//       every token; partial sums leave tagged.
//   C2  workgroup b < H / 16: rows 16 b .. + 16 = the sum of the K / 512
//       partials (update), hidden_out = x + update.
// The last workgroup keeps the epoch: once every workgroup has stored its
// started word (after reading the epoch and the position) it advances the
// epoch and, with a device-held position, the position by T.
// ---------------------------------------------------------------------------
constexpr int kAsWaves = 8;
constexpr int kAsThreads = 64 * kAsWaves;
constexpr int kAsMaxTokens = 4;
constexpr int kAsMaxGrid = 512;
constexpr int kAsMaxRows = 5;      // phase A rows per wavefront
constexpr int kAsMaxChunks = 64;   // attention units per (token, kv head)
constexpr int kAsMDims = 64;       // head dims per merge unit
constexpr int kAsKcu = 512;        // Wo columns per C1 unit
constexpr int kAsRb = 128;         // Wo rows per C1 unit (16 per wavefront)
constexpr int kAsTile = 24;        // cached positions per LDS tile of an attention unit
constexpr int kAsMaxH = 2048;
constexpr int kAsMaxG = 8;         // query heads per kv head
constexpr int kAsGu = 4;           // query heads per attention unit
// dynamic LDS: phase B's [4][hd] x 2 (queries), [4][hd] x 3 (own keys raw
// and final, own values) and the softmax states [8 wavefronts][4][hd] (the
// cached rows go straight to registers); phase A's [T][H] and C1's
// [T][512] are smaller
constexpr size_t kAsMaxLds = (size_t)(2 * kAsGu + 3 * kAsMaxTokens + kAsWaves * kAsGu) * kAttnMaxHeadDim * 4;
static_assert(kAsMaxTokens * kAsMaxH * 4 <= kAsMaxLds, "phase A's tokens must fit in the LDS");

struct AttnTagWs {
  uint32_t* tickets;  // [16] workspace header (epoch, poll bound, error word)
  uint64_t* started;  // [kAsMaxGrid]
  uint64_t* qkv;      // [T][R] projected (q_h | gate_h) pairs, k, v
  uint64_t* part;     // [T][heads][kAsMaxChunks][hd + 2] chunk (max, sum, weighted values)
  uint64_t* gated;    // [T][K]
  uint64_t* cpart;    // [K / 512][T][H] C1 partial sums
};

struct AttnStepArgs {
  const void* x;
  const void* nw;
  int nw_dt;
  const void* wq;  // bf16 [2K, H]: rows 2 hd h .. + hd = q_h, the next hd = gate_h
  const void* wk;  // bf16 [kvh hd, H]
  const void* wv;
  const void* wo;  // bf16 [H, K]
  const void* qn_w;
  const void* kn_w;
  int qn_dt, kn_dt;
  void* kc;  // [max_pos, kvh, hd]
  void* vc;
  int* start_dev;
  int start, max_pos;
  int T, H, heads, kvh, hd, rope_dim, interleaved, nch;
  float theta_log2, eps, qk_eps;
  float* update;
  float* hidden_out;
  AttnTagWs tw;
};

// Phase A row split: workgroup b holds rows b * base + min(b, rem) .. (base
// + 1 rows for b < rem, base after); returns the workgroup holding row r.
__device__ __forceinline__ int as_wg_of_row(int r, int R, int G) {
  const int base = R / G, rem = R % G, cut = rem * (base + 1);
  return r < cut ? r / (base + 1) : rem + (r - cut) / base;
}

// RoPE of the 4 dims d0 .. d0 + 3 of a normalised head row in LDS (dims >=
// rope_dim unchanged); cs[i] = (cos, sin) of pair i's angle at the row's
// position, p * theta^(-2i / rope_dim) as the split kernel computes it.
__device__ __forceinline__ float4 as_rope4(const float* row, int d0, const float2* cs, const AttnStepArgs& a) {
  float y[4] = {row[d0], row[d0 + 1], row[d0 + 2], row[d0 + 3]};
  const int rd = a.rope_dim;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int d = d0 + e;
    if (d < rd) {
      int i, partner;
      float sign;
      if (a.interleaved) {
        i = d >> 1;
        partner = d ^ 1;
        sign = (d & 1) ? 1.f : -1.f;
      } else {
        const int h2 = rd >> 1;
        i = d < h2 ? d : d - h2;
        partner = d < h2 ? d + h2 : d - h2;
        sign = d < h2 ? -1.f : 1.f;
      }
      y[e] = y[e] * cs[i].x + sign * row[partner] * cs[i].y;
    }
  }
  return make_float4(y[0], y[1], y[2], y[3]);
}

// RMSNorm(1 + w) over hd of one head row in LDS, held 4 dims per lane by one
// wavefront (w: the lane's 4 norm-weight words); written back in place.
__device__ __forceinline__ void as_norm_row(float* row, int d0, bool lin, int hd, float eps, const uint32_t (&w)[4],
                                            const void* wp, int wdt) {
  float4 x4 = lin ? *reinterpret_cast<const float4*>(row + d0) : make_float4(0.f, 0.f, 0.f, 0.f);
  const float ss = wave_sum(x4.x * x4.x + x4.y * x4.y + x4.z * x4.z + x4.w * x4.w);
  const float r = rsqrtf(ss / (float)hd + eps);
  if (lin) {
    x4.x *= r * (1.f + elem_value(w[0], wp, wdt, d0));
    x4.y *= r * (1.f + elem_value(w[1], wp, wdt, d0 + 1));
    x4.z *= r * (1.f + elem_value(w[2], wp, wdt, d0 + 2));
    x4.w *= r * (1.f + elem_value(w[3], wp, wdt, d0 + 3));
    *reinterpret_cast<float4*>(row + d0) = x4;
  }
}

// elem_word through a global-address-space pointer (a global load, not a
// flat one, which would also count against the LDS wait counter).
__device__ __forceinline__ uint32_t as_elem_word(const void* p, int dtype, size_t i) {
  const uintptr_t at = reinterpret_cast<uintptr_t>(p) + (dtype == FK_DTYPE_BF16 ? i * 2 : i * 4);
  return *reinterpret_cast<const __attribute__((address_space(1))) uint32_t*>(at & ~(uintptr_t)3);
}

FK_TIMELINE_BUFFER(attn_step)

template <bool BFX, bool CBF>
__global__ __launch_bounds__(kAsThreads) void attn_step_kernel(AttnStepArgs a) {
  FK_TIMELINE_DECL;
  FK_MARK(0);  // (timeline markers: diagnostic builds only)
  extern __shared__ float4 s_dyn_v[];
  float* s_dyn = reinterpret_cast<float*>(s_dyn_v);
  __shared__ float s_part[kAsWaves][kAsMaxTokens];
  __shared__ float s_rs[kAsMaxTokens];
  __shared__ float s_m[kAsWaves][kAsGu], s_l[kAsWaves][kAsGu], s_f[kAsWaves][kAsGu], s_ML[kAsGu][2];
  __shared__ float2 s_cs[1 + kAsMaxTokens][kAttnMaxHeadDim / 2];  // RoPE (cos, sin): the queries', the own keys'

  __shared__ float s_fc[kAsMaxChunks];
  __shared__ float s_L;
  __shared__ float s_mo[kAsWaves][kAsMDims];
  __shared__ int s_fail, s_kfail;
  __shared__ uint32_t s_hdr[4];  // header words and position, as wavefront 0 loaded them
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = gridDim.x, b = blockIdx.x;
  const int T = a.T, H = a.H, hd = a.hd, heads = a.heads, kvh = a.kvh, Gq = heads / kvh;
  const int K = heads * hd, Rq = 2 * K, Rk = kvh * hd, R = Rq + 2 * Rk;
  const int nch = a.nch, nds = hd / kAsMDims, nks = K / kAsKcu, nchk = H >> 3;
  const int hd_sh = 31 - __builtin_clz(hd);  // (hd is a power of two: the host checks)
  // The workspace header and the device-held position are loaded first, by
  // wavefront 0 alone, and shared through LDS at the staging barrier: the
  // words are read past the caches (coherent loads), and the same lines
  // read by every wavefront of the grid at once queue behind each other.
  WaitHeader hdr{0u, 0u, 0u};
  int start_ld = a.start;
  if (wave == 0) {
    hdr = load_wait_header(a.tw.tickets, kWorkspaceEpochWord);
    if (a.start_dev) start_ld = load_coherent(a.start_dev);
  }

  // Roles: attention units and merge units on the last workgroups (at the
  // model shape every workgroup is an attention unit), C1 units and C2 rows
  // on the first; a workgroup runs its roles in the order B, M, C1, C2.
  const int hsplit = Gq > kAsGu ? Gq / kAsGu : 1, Gu = Gq / hsplit;  // units per kv head and token, heads per unit
  const int n_att = T * kvh * hsplit * nch, att0 = G - n_att;
  const int n_m = T * heads * nds, m0 = G - n_m;
  const int n_c1 = (H / kAsRb) * nks;
  const bool is_att = b >= att0, is_m = b >= m0, is_c1 = b < n_c1, is_out = b < H / 16;
  const int au = is_att ? b - att0 : 0;
  const int ac = au % nch, ahs = (au / nch) % hsplit, aj = (au / (nch * hsplit)) % kvh, at = au / (nch * hsplit * kvh);
  const int hb = aj * Gq + ahs * Gu;  // the unit's first query head
  const int d0 = lane * 4;
  const bool lin = d0 < hd;
  const int dl = lin ? d0 : 0;

  // ---- loads, in the order their data is used ----------------------------
  // tokens (chunk q = tid + 512 i of the T * H / 8) and the norm weight
  constexpr int XCH = kAsMaxTokens * kAsMaxH / 8 / kAsThreads;
  Raw8<BFX> xr[XCH];
  uint32_t nwr[XCH][8];
#pragma unroll
  for (int i = 0; i < XCH; ++i) {
    const int q = tid + i * kAsThreads, qc = q < T * nchk ? q : 0;
    xr[i] = load_raw8<BFX>(a.x, (size_t)qc * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) nwr[i][e] = as_elem_word(a.nw, a.nw_dt, (size_t)(qc % nchk) * 8 + e);
  }
  // q/k norm weights of this lane's dims, residual inputs of the C2 rows
  uint32_t qnr[4], knr[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    qnr[e] = as_elem_word(a.qn_w, a.qn_dt, dl + e);
    knr[e] = as_elem_word(a.kn_w, a.kn_dt, dl + e);
  }
  uint32_t xres[1];
  gather_raw<BFX>(a.x, is_out && tid < 16 * T ? (size_t)(tid >> 4) * H + b * 16 + (tid & 15) : 0, 0, 1, xres);
  // phase A rows of this wavefront: rlo .. rlo + rn - 1 (rn >= 1; the
  // unused row slots repeat the last row)
  const int rbase = R / G, rrem = R % G;
  const int wlo = b * rbase + min(b, rrem), wn = rbase + (b < rrem ? 1 : 0);
  const int vb = wn / kAsWaves, vr = wn % kAsWaves;
  const int rlo = wlo + wave * vb + min(wave, vr), rn = vb + (wave < vr ? 1 : 0);
  Raw8<true> wt[kAsMaxRows][4];
#pragma unroll
  for (int i = 0; i < kAsMaxRows; ++i) {
    const int row = rlo + (i < rn ? i : rn - 1);
    const uint16_t* wp = row < Rq        ? reinterpret_cast<const uint16_t*>(a.wq) + (size_t)row * H
                         : row < Rq + Rk ? reinterpret_cast<const uint16_t*>(a.wk) + (size_t)(row - Rq) * H
                                         : reinterpret_cast<const uint16_t*>(a.wv) + (size_t)(row - Rq - Rk) * H;
#pragma unroll
    for (int j = 0; j < 4; ++j) wt[i][j] = load_raw8_stream<true>(wp, (size_t)min(lane + kWave * j, nchk - 1) * 8);
  }
  // the unit's chunk (set at the staging, once the position is shared; its
  // first tile of cached rows is issued in phase B)
  int start = 0, apos = 0, an = 0, p_lo = 0, p_hi = 0;  // positions 0 .. apos of the token
  bool bad_pos = false;
  // Cached rows of an attention unit, a tile of kAsTile positions from pt at
  // a time, read straight into the registers of the wavefront that scores
  // them: wavefront w the positions pt + w + 8 bb (bb < kAsTile / 8), lane
  // l dims 4 l .. 4 l + 3 of their k and v rows (no LDS staging, no
  // barrier); positions past the chunk repeat its last one (clamped in
  // range, never scored).  Staged through LDS by every thread instead, the
  // step took 0.5-0.6 us longer (the staging and its barrier sat between
  // the RoPE and the softmax).
  constexpr int PPW = kAsTile / kAsWaves;  // positions per wavefront per tile
  Row4<CBF> ckr[PPW], cvr[PPW];
  auto issue_tile = [&](int pt) {
#pragma unroll
    for (int bb = 0; bb < PPW; ++bb) {
      const int p = max(min(pt + wave + kAsWaves * bb, p_hi - 1), 0);
      const size_t cr = ((size_t)p * kvh + aj) * hd + dl;
      ckr[bb] = load_row4<CBF>(a.kc, cr);
      cvr[bb] = load_row4<CBF>(a.vc, cr);
    }
  };
  FK_MARK(1);

  // ---- stage the tokens: s_x[t][c] = x * (1 + w), s_rs[t] -----------------
  uint32_t tag = 0u, plim = 0u;
  float* s_x = s_dyn;
  {
    float ssp[kAsMaxTokens] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < XCH; ++i) {
      const int q = tid + i * kAsThreads;
      if (q < T * nchk) {  // (uniform per wavefront: nchk is a multiple of 64)
        const int t = q / nchk, c = q - t * nchk;
        float x8[8];
        raw8_to_f32<BFX>(xr[i], x8);
        float p = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          p = fmaf(x8[e], x8[e], p);
          x8[e] *= 1.f + elem_value(nwr[i][e], a.nw, a.nw_dt, (size_t)c * 8 + e);
        }
#pragma unroll
        for (int u = 0; u < kAsMaxTokens; ++u) ssp[u] += u == t ? p : 0.f;
        float4* dst = reinterpret_cast<float4*>(s_x + (size_t)t * H + c * 8);
        dst[0] = make_float4(x8[0], x8[1], x8[2], x8[3]);
        dst[1] = make_float4(x8[4], x8[5], x8[6], x8[7]);
      }
    }
#pragma unroll
    for (int u = 0; u < kAsMaxTokens; ++u) {
      if (u < T) {
        const float s = wave_sum(ssp[u]);
        if (lane == 0) s_part[wave][u] = s;
      }
    }
    if (tid == 0) {
      s_fail = 0;
      s_kfail = 0;
      s_hdr[0] = hdr.epoch;
      s_hdr[1] = hdr.set;
      s_hdr[2] = hdr.err;
      s_hdr[3] = (uint32_t)start_ld;
    }
    lds_barrier();
    {
      WaitHeader h{s_hdr[0], s_hdr[1], s_hdr[2]};
      const WaitLimits wl = h.limits();
      tag = wl.tag;
      plim = wl.poll;
      start = (int)s_hdr[3];
      bad_pos = start < 0 || start + T > a.max_pos;
      apos = start + at;
      an = bad_pos ? 0 : apos + 1;
      const int aC = (an + nch - 1) / nch;
      p_lo = min(ac * aC, an);
      p_hi = min(p_lo + aC, an);
    }
    if (tid < T) {
      float tot = 0.f;
#pragma unroll
      for (int w = 0; w < kAsWaves; ++w) tot += s_part[w][tid];
      s_rs[tid] = rsqrtf(tot / (float)H + a.eps);
    }
    lds_barrier();
  }

  // ---- phase A: row dot products, every token --------------------------
  for (int t = 0; t < T; ++t) {
#pragma unroll
    for (int i = 0; i < kAsMaxRows; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) asm volatile("" : "+v"(wt[i][j].a));  // rows converted where used, per token
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (kWave * j < nchk) {  // (uniform)
        const float4* xp = reinterpret_cast<const float4*>(s_x + (size_t)t * H + (lane + kWave * j) * 8);
        const float4 xa = xp[0], xb = xp[1];
        const float x8[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
        for (int i = 0; i < kAsMaxRows; ++i) {
          float w8[8];
          raw8_to_f32<true>(wt[i][j], w8);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[i] = fmaf(w8[e], x8[e], acc[i]);
        }
      }
    }
    const float v = rows8_sum(acc) * s_rs[t];  // lanes 8i ..: row i
    const int ri = lane >> 3;
    if ((lane & 7) == 0 && ri < rn) store_tagged(a.tw.qkv + (size_t)t * R + rlo + ri, v, tag);
  }
  lds_barrier();  // phase B reuses the LDS
  if (tid == 0) store_tagged(a.tw.started + b, (float)start, tag);  // (after the epoch and position loads)
  FK_MARK(2);


  // ---- phase B: attention unit (at, aj, ahs, ac) ---------------------------
  if (is_att) {
    float* s_q = s_dyn;                            // [Gu][hd] raw, then normalised
    float* s_qf = s_q + kAsGu * hd;                // [Gu][hd] rotated and scaled
    float* s_kr = s_qf + kAsGu * hd;               // [4][hd] own keys raw, then normalised
    float* s_kf = s_kr + kAsMaxTokens * hd;        // [4][hd] own keys rotated
    float* s_vn = s_kf + kAsMaxTokens * hd;        // [4][hd] own values
    float* s_acc = s_vn + kAsMaxTokens * hd;       // [waves][Gu][hd] wavefront states after the last tile
    // own positions of the chunk: o_lo .. p_hi - 1, tokens u_lo ..
    const int o_lo = max(p_lo, start), n_own = p_hi > o_lo ? p_hi - o_lo : 0, u_lo = o_lo - start;
    // token at's queries of heads hb .. (word e = g * hd + d), the own
    // tokens' k and v (word e = s * hd + d), polled directly (their first
    // round of loads in flight while the RoPE angles are computed)
    uint64_t w[6];
    const uint64_t* srcs[6];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e = tid + i * kAsThreads, s = e >> hd_sh, d = e & (hd - 1);
      srcs[i] = e < Gu * hd ? a.tw.qkv + (size_t)at * R + (size_t)(hb + s) * 2 * hd + d : nullptr;
      const uint64_t* kr = a.tw.qkv + (size_t)(u_lo + s) * R + Rq + (size_t)aj * hd + d;
      srcs[2 + i] = s < n_own ? kr : nullptr;
      srcs[4 + i] = s < n_own ? kr + Rk : nullptr;
    }
#pragma unroll
    for (int i = 0; i < 6; ++i) w[i] = srcs[i] ? load_tagged(srcs[i]) : 0ull;
    // The unit's first tile of cached rows, behind the first round of its
    // inputs and staged after the norms and RoPE.  (Issued behind the phase
    // A weight rows instead, it was waited for with them: the attention
    // units then ended phase A last, 1.4 us later at ctx 1024.)
    issue_tile(p_lo);
    // RoPE angles, once per position: slot 0 the queries' (apos), slot
    // 1 + s own key s's (o_lo + s); entry i of a slot is pair i's (cos, sin)
    {
      const int npair = a.rope_dim >> 1;  // (<= 128)
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int e = tid + k * kAsThreads, slot = e >> 7, i = e & 127;
        if (i < npair && slot <= n_own) {
          const float inv_freq = exp2f(-(float)(2 * i) / (float)a.rope_dim * a.theta_log2);
          float sn, cs;
          sincosf((float)(slot == 0 ? apos : o_lo + slot - 1) * inv_freq, &sn, &cs);
          s_cs[slot][i] = make_float2(cs, sn);
        }
      }
    }
    if (!poll_tagged<6>(w, srcs, tag, plim)) s_fail = 1;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e = tid + i * kAsThreads;
      if (srcs[i]) s_q[e] = value_of(w[i]);
      if (srcs[2 + i]) {
        s_kr[e] = value_of(w[2 + i]);
        s_vn[e] = value_of(w[4 + i]);
      }
    }
    lds_barrier();
    FK_MARK(3);
    const bool bad = s_fail || bad_pos;
    // head norms: wavefront g < 4 query head hb + g, wavefront 4 + s own key s
    if (wave < Gu) as_norm_row(s_q + wave * hd, dl, lin, hd, a.qk_eps, qnr, a.qn_w, a.qn_dt);
    if (wave >= kAsGu && wave - kAsGu < n_own)
      as_norm_row(s_kr + (wave - kAsGu) * hd, dl, lin, hd, a.qk_eps, knr, a.kn_w, a.kn_dt);
    lds_barrier();
    FK_MARK(10);
    // RoPE, and the queries' 1/sqrt(hd)
    if (wave < Gu && lin) {
      const float scale = rsqrtf((float)hd);
      float4 y = as_rope4(s_q + wave * hd, d0, s_cs[0], a);
      y.x *= scale;
      y.y *= scale;
      y.z *= scale;
      y.w *= scale;
      *reinterpret_cast<float4*>(s_qf + wave * hd + d0) = y;
    }
    if (wave >= kAsGu && wave - kAsGu < n_own && lin) {
      const int s = wave - kAsGu;
      *reinterpret_cast<float4*>(s_kf + s * hd + d0) = as_rope4(s_kr + s * hd, d0, s_cs[1 + s], a);
    }
    lds_barrier();
    FK_MARK(11);
    float4 q4[kAsGu], acc[kAsGu];
    float m[kAsGu], l[kAsGu];
#pragma unroll
    for (int g = 0; g < kAsGu; ++g) {
      q4[g] = lin && g < Gu ? *reinterpret_cast<const float4*>(s_qf + g * hd + d0) : make_float4(0.f, 0.f, 0.f, 0.f);
      acc[g] = make_float4(0.f, 0.f, 0.f, 0.f);
      m[g] = -INFINITY;
      l[g] = 0.f;
    }
    // tiles of kAsTile positions (the first issued with the inputs):
    // wavefront w takes positions pt + w, + 8, .. from its registers; per
    // head one softmax step over its positions of the tile.  The step's own
    // positions read the recomputed keys and the values from v.
    for (int pt = p_lo; pt < p_hi; pt += kAsTile) {
      if (pt != p_lo) issue_tile(pt);
      FK_MARK(12);
      const int pend = min(pt + kAsTile, p_hi);
      float sr[PPW];  // lanes 16g ..: head g's score at position pt + w + 8 bb
#pragma unroll
      for (int bb = 0; bb < PPW; ++bb) {
        const int p = min(pt + wave + kAsWaves * bb, pend - 1);  // (positions past the tile: scored -inf below)
        const float4 k4 = p >= o_lo ? *reinterpret_cast<const float4*>(s_kf + (p - o_lo) * hd + dl) : ckr[bb].f4();  // (uniform)
        float d[kAsGu];
#pragma unroll
        for (int g = 0; g < kAsGu; ++g) d[g] = q4[g].x * k4.x + q4[g].y * k4.y + q4[g].z * k4.z + q4[g].w * k4.w;
        sr[bb] = rows4_sum(d);
      }
#pragma unroll
      for (int g = 0; g < kAsGu; ++g) {
        if (g >= Gu) break;
        float sc[PPW];
        float mx = m[g];
#pragma unroll
        for (int bb = 0; bb < PPW; ++bb) {
          sc[bb] = pt + wave + kAsWaves * bb < pend
                       ? __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(sr[bb]), 16 * g))
                       : -INFINITY;
          mx = fmaxf(mx, sc[bb]);
        }
        if (mx == -INFINITY) continue;  // (uniform: no position of this wavefront in the tile)
        const float f = __expf(m[g] - mx);
        float es = 0.f;
        float4 av = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int bb = 0; bb < PPW; ++bb) {
          const int p = min(pt + wave + kAsWaves * bb, pend - 1);
          const float e = __expf(sc[bb] - mx);
          const float4 v4 = p >= o_lo ? *reinterpret_cast<const float4*>(s_vn + (p - o_lo) * hd + dl) : cvr[bb].f4();  // (uniform)
          es += e;
          av.x = fmaf(e, v4.x, av.x);
          av.y = fmaf(e, v4.y, av.y);
          av.z = fmaf(e, v4.z, av.z);
          av.w = fmaf(e, v4.w, av.w);
        }
        l[g] = l[g] * f + es;
        acc[g].x = acc[g].x * f + av.x;
        acc[g].y = acc[g].y * f + av.y;
        acc[g].z = acc[g].z * f + av.z;
        acc[g].w = acc[g].w * f + av.w;
        m[g] = mx;
      }
    }
    lds_barrier();  // the softmax states reuse the row tile
    FK_MARK(13);
    // the wavefronts' states merged per (head, dim): per-wavefront factors
    // exp(m_w - M) once, then the chunk partial (max, sum, weighted values)
    // leaves tagged
#pragma unroll
    for (int g = 0; g < kAsGu; ++g) {
      if (g < Gu) {
        if (lane == 0) {
          s_m[wave][g] = m[g];
          s_l[wave][g] = l[g];
        }
        if (lin) *reinterpret_cast<float4*>(s_acc + ((size_t)wave * Gu + g) * hd + d0) = acc[g];
      }
    }
    lds_barrier();
    if (tid < kAsWaves * kAsGu) {
      const int w = tid / kAsGu, g = tid - w * kAsGu;
      if (g < Gu) {
        float M = s_m[0][g];
#pragma unroll
        for (int v = 1; v < kAsWaves; ++v) M = fmaxf(M, s_m[v][g]);
        s_f[w][g] = s_m[w][g] == -INFINITY ? 0.f : __expf(s_m[w][g] - M);
        if (w == 0) {
          float L = 0.f;
#pragma unroll
          for (int v = 0; v < kAsWaves; ++v) L += s_m[v][g] == -INFINITY ? 0.f : s_l[v][g] * __expf(s_m[v][g] - M);
          s_ML[g][0] = M;
          s_ML[g][1] = L;
        }
      }
    }
    lds_barrier();
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e = tid + i * kAsThreads;
      if (e < Gu * hd) {
        const int g = e >> hd_sh, d = e & (hd - 1);
        float o = 0.f;
#pragma unroll
        for (int w = 0; w < kAsWaves; ++w) o = fmaf(s_acc[((size_t)w * Gu + g) * hd + d], s_f[w][g], o);
        uint64_t* pp = a.tw.part + (((size_t)at * heads + hb + g) * kAsMaxChunks + ac) * (hd + 2);
        store_tagged(pp + 2 + d, poison_if(bad, o), tag);
        if (d == 0) {
          store_tagged(pp, poison_if(bad, s_ML[g][0]), tag);
          store_tagged(pp + 1, poison_if(bad, s_ML[g][1]), tag);
        }
      }
    }
    // the first unit of the chunk holding position apos writes token at's
    // cache rows of kv head aj (after its partials: nothing waits for these)
    if (!bad_pos && ahs == 0 && apos >= p_lo && apos < p_hi && tid < hd) {
      const int s = apos - o_lo;
      const size_t cr = ((size_t)apos * kvh + aj) * hd + tid;
      store1<CBF>(a.kc, cr, poison_if(bad, s_kf[s * hd + tid]));
      store1<CBF>(a.vc, cr, poison_if(bad, s_vn[s * hd + tid]));
    }
    lds_barrier();  // (the LDS is reused by the next role)
    FK_MARK(14);
  }
  FK_MARK(4);

  // ---- phase M: merge unit (mt, mh, mds) -----------------------------------
  if (is_m) {
    const int mu = b - m0, mt = mu / (heads * nds), mh = (mu / nds) % heads, mds = mu % nds;
    // (the partials are polled directly, as every input of this kernel)
    // thread (wavefront cg, lane dd): dim 64 mds + dd of chunks cg, cg + 8, ..;
    // wavefront 0 also the chunk statistics (lane c) and the gate (lane dd)
    const uint64_t* pbase = a.tw.part + ((size_t)mt * heads + mh) * kAsMaxChunks * (hd + 2);
    uint64_t w[kAsMaxChunks / kAsWaves];
    const uint64_t* srcs[kAsMaxChunks / kAsWaves];
#pragma unroll
    for (int k = 0; k < kAsMaxChunks / kAsWaves; ++k) {
      const int c = wave + kAsWaves * k;
      srcs[k] = c < nch ? pbase + (size_t)c * (hd + 2) + 2 + mds * kAsMDims + lane : nullptr;
      w[k] = srcs[k] ? load_tagged(srcs[k]) : 0ull;
    }
    uint64_t st[3];
    const uint64_t* ss[3] = {nullptr, nullptr, nullptr};
    if (wave == 0) {
      ss[0] = lane < nch ? pbase + (size_t)lane * (hd + 2) : nullptr;
      ss[1] = lane < nch ? pbase + (size_t)lane * (hd + 2) + 1 : nullptr;
      ss[2] = a.tw.qkv + (size_t)mt * R + (size_t)mh * 2 * hd + hd + mds * kAsMDims + lane;
    }
#pragma unroll
    for (int i = 0; i < 3; ++i) st[i] = ss[i] ? load_tagged(ss[i]) : 0ull;
    bool ok = poll_tagged<kAsMaxChunks / kAsWaves>(w, srcs, tag, plim);
    ok = poll_tagged<3>(st, ss, tag, plim) && ok;
    if (!ok) s_fail = 1;
    if (wave == 0) {
      const float mc = lane < nch ? value_of(st[0]) : -INFINITY, lc = lane < nch ? value_of(st[1]) : 0.f;
      const float M = wave_max(mc);
      const float fc = mc == -INFINITY ? 0.f : __expf(mc - M);
      const float L = wave_sum(fc * lc);
      s_fc[lane] = fc;
      if (lane == 0) s_L = L;
    }
    lds_barrier();
    float o = 0.f;
#pragma unroll
    for (int k = 0; k < kAsMaxChunks / kAsWaves; ++k)
      if (srcs[k]) o = fmaf(s_fc[wave + kAsWaves * k], value_of(w[k]), o);
    s_mo[wave][lane] = o;
    lds_barrier();
    if (wave == 0) {
      float tot = 0.f;
#pragma unroll
      for (int cg = 0; cg < kAsWaves; ++cg) tot += s_mo[cg][lane];
      const float gv = tot / s_L * sigmoid(value_of(st[2]));
      store_tagged(a.tw.gated + (size_t)mt * K + (size_t)mh * hd + mds * kAsMDims + lane, poison_if(s_fail != 0, gv), tag);
    }
    lds_barrier();  // (the LDS is reused by the next role)
  }
  FK_MARK(5);

  // ---- phase C1: unit (urb, uks) -------------------------------------------
  if (is_c1) {
    // Wo block first: a unit without an attention or merge role gets here
    // right after phase A, so its rows arrive while it waits for the merges
    const int urb = b / nks, uks = b - urb * nks;
    u32x4 wo[16];
    {
      const uint16_t* wp = reinterpret_cast<const uint16_t*>(a.wo) + (size_t)(urb * kAsRb + wave * 16) * K +
                           (size_t)uks * kAsKcu + lane * 8;
#pragma unroll
      for (int r = 0; r < 16; ++r) wo[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wp + (size_t)r * K));
    }
    float* s_g = s_dyn;  // [T][512] gated values of the unit's columns (polled directly)
    {
      uint64_t w[kAsMaxTokens];
      const uint64_t* srcs[kAsMaxTokens];
#pragma unroll
      for (int t = 0; t < kAsMaxTokens; ++t) {
        srcs[t] = t < T ? a.tw.gated + (size_t)t * K + (size_t)uks * kAsKcu + tid : nullptr;
        w[t] = srcs[t] ? load_tagged(srcs[t]) : 0ull;
      }
      if (!poll_tagged<kAsMaxTokens>(w, srcs, tag, plim)) s_fail = 1;
#pragma unroll
      for (int t = 0; t < kAsMaxTokens; ++t)
        if (t < T) s_g[t * kAsKcu + tid] = value_of(w[t]);
    }
    lds_barrier();
    FK_MARK(6);
    const bool bad = s_fail != 0;
    for (int t = 0; t < T; ++t) {
      const float4* gp = reinterpret_cast<const float4*>(s_g + t * kAsKcu + lane * 8);
      const float4 ga = gp[0], gb = gp[1];
      const float g8[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
      float lo[8], hi[8];
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        Raw8<true> r0, r1;
        r0.a = wo[r];
        r1.a = wo[r + 8];
        float w0[8], w1[8];
        raw8_to_f32<true>(r0, w0);
        raw8_to_f32<true>(r1, w1);
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          s0 = fmaf(w0[e], g8[e], s0);
          s1 = fmaf(w1[e], g8[e], s1);
        }
        lo[r] = s0;
        hi[r] = s1;
      }
      const float vlo = rows8_sum(lo), vhi = rows8_sum(hi);  // lanes 8i ..: rows i and 8 + i
      if ((lane & 7) == 0) {
        const size_t o = ((size_t)uks * T + t) * H + (size_t)urb * kAsRb + wave * 16 + (lane >> 3);
        store_tagged(a.tw.cpart + o, poison_if(bad, vlo), tag);
        store_tagged(a.tw.cpart + o + 8, poison_if(bad, vhi), tag);
      }
    }
  }
  FK_MARK(7);

  // ---- phase C2: rows 16b .. 16b + 15 = sum of the nks unit partials -------
  if (is_out && tid < 16 * T) {
    // (nks <= 8 partials per thread, polled directly)
    const int r = tid & 15, t = tid >> 4;
    uint64_t w[8];
    const uint64_t* srcs[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      srcs[j] = j < nks ? a.tw.cpart + ((size_t)j * T + t) * H + b * 16 + r : nullptr;
      w[j] = srcs[j] ? load_tagged(srcs[j]) : 0ull;
    }
    const bool pok = poll_tagged<8>(w, srcs, tag, plim);
    if (!pok) s_fail = 1;
    float v = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (j < nks) v += value_of(w[j]);
    v = poison_if(!pok, v);
    const size_t o = (size_t)t * H + b * 16 + r;
    a.update[o] = v;
    if (a.hidden_out) a.hidden_out[o] = raw_value<BFX>(xres[0]) + v;
  }
  FK_MARK(8);

  // ---- epoch keeper ----------------------------------------------------------
  if (b == G - 1) {
    uint64_t w[1];
    const uint64_t* srcs[1] = {tid < G ? a.tw.started + tid : nullptr};
    w[0] = srcs[0] ? load_tagged(srcs[0]) : 0ull;
    if (!poll_tagged<1>(w, srcs, tag, plim)) s_kfail = 1;
    lds_barrier();
    // (not after a failed wait: a workgroup that has not read the epoch and
    // the position yet would take the next launch's; the error word poisons
    // later launches)
    if (tid == 0 && !s_kfail) {
      store_coherent(&a.tw.tickets[kWorkspaceEpochWord], tag);
      // (a position whose step would pass the cache stays where it is)
      if (a.start_dev && !bad_pos) store_coherent(a.start_dev, start + T);
    }
  }
  lds_barrier();
  if (tid == 0 && (s_fail || s_kfail))
    __hip_atomic_fetch_or(&a.tw.tickets[kWorkspaceErrorWord], FK_DEVICE_ERR_BARRIER, __ATOMIC_RELAXED,
                          __HIP_MEMORY_SCOPE_AGENT);
  if (b == 0 && tid == 0 && bad_pos)
    __hip_atomic_fetch_or(&a.tw.tickets[kWorkspaceErrorWord], FK_DEVICE_ERR_POSITION, __ATOMIC_RELAXED,
                          __HIP_MEMORY_SCOPE_AGENT);
  FK_MARK(9);
  FK_TIMELINE_COMMIT(attn_step, blockIdx.x);
}

// Attention workspace: the single-launch step's tagged region first (its
// 16-word header at offset 0 serves fk_workspace_status; the other words
// exist for T <= kAsMaxTokens only), then the staged launches' buffers.
struct AttnWs {
  AttnTagWs tw;
  float* qg;
  float* k;
  float* v;
  float* gated;
  float* part;
};

static size_t attn_ws_layout(int T, int heads, int kvh, int hd, char* base, AttnWs* ws) {
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t at = off;
    off = align_up(off + bytes, 256);
    return base ? base + at : nullptr;
  };
  const bool one = T <= kAsMaxTokens;
  const size_t K = (size_t)heads * hd, R = 2 * K + 2 * (size_t)kvh * hd;
  auto words = [&](size_t n) { return reinterpret_cast<uint64_t*>(take(one ? n * 8 : 0)); };
  ws->tw.tickets = reinterpret_cast<uint32_t*>(take(16 * sizeof(uint32_t)));
  ws->tw.started = words(kAsMaxGrid);
  ws->tw.qkv = words((size_t)T * R);
  ws->tw.part = words((size_t)T * heads * kAsMaxChunks * (hd + 2));
  ws->tw.gated = words((size_t)T * K);
  ws->tw.cpart = words((K + kAsKcu - 1) / kAsKcu * T * kAsMaxH);
  auto floats = [&](size_t n) { return reinterpret_cast<float*>(take(n * 4)); };
  ws->qg = floats((size_t)T * heads * 2 * hd);
  ws->k = floats((size_t)T * kvh * hd);
  ws->v = floats((size_t)T * kvh * hd);
  ws->gated = floats((size_t)T * heads * hd);
  ws->part = floats((size_t)T * heads * kAttnMaxChunks * (hd + 2));
  return off;
}

// Single-launch step: chunks per (token, kv head, group of 4 query heads)
// on a grid of G workgroups (every workgroup an attention unit when that
// allows 64 chunks or fewer), or 0 when the shape is not one the kernel
// handles.
static int attn_step_chunks(int T, int H, int heads, int kvh, int hd, int weight_dt, int G) {
  if (weight_dt != FK_DTYPE_BF16 || T < 1 || T > kAsMaxTokens || G < 1 || G > kAsMaxGrid) return 0;
  if (H < 512 || H > kAsMaxH || H % 512 || hd < kAsMDims || hd > kAttnMaxHeadDim || (hd & (hd - 1))) return 0;
  if (heads < 1 || kvh < 1 || heads % kvh || heads / kvh > kAsMaxG) return 0;
  const int Gq = heads / kvh, hsplit = Gq > kAsGu ? Gq / kAsGu : 1;
  if (Gq > kAsGu && Gq % kAsGu) return 0;
  const int K = heads * hd, R = 2 * K + 2 * kvh * hd;
  if (K % kAsKcu || K > 4096) return 0;
  if (R / G < kAsWaves || (R + G - 1) / G > kAsWaves * kAsMaxRows) return 0;  // 1 .. kAsMaxRows rows per wavefront
  const int n_c1 = (H / kAsRb) * (K / kAsKcu), n_m = T * heads * (hd / kAsMDims);
  if (n_c1 > G || H / 16 > G || n_m > G) return 0;
  int nch = G / (T * kvh * hsplit);
  if (nch > kAsMaxChunks) nch = kAsMaxChunks;
  return nch > 0 ? nch : 0;
}

// Grid of the single-launch step (one workgroup per CU, capped at the
// co-resident capacity), or 0 when the device cannot host it.
template <bool BX, bool CB>
static int attn_step_grid() {
  static int cap_cache[64] = {0};
  static int attr_ok[64] = {0};  // 0 unknown, 1 set, -1 refused
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (attr_ok[dev] == 0)
    attr_ok[dev] = hipFuncSetAttribute(reinterpret_cast<const void*>(attn_step_kernel<BX, CB>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)kAsMaxLds) == hipSuccess
                       ? 1
                       : -1;
  if (attr_ok[dev] < 0) {
    (void)hipGetLastError();
    return 0;
  }
  const int cap = resident_capacity(attn_step_kernel<BX, CB>, kAsThreads, kAsMaxLds, cap_cache);
  const int cus = device_cus();
  const int G = cap < cus ? cap : cus;
  return G > kAsMaxGrid ? kAsMaxGrid : G;
}

static int attn_step_grid_for(bool bx, bool cb) {
  if (bx) return cb ? attn_step_grid<true, true>() : attn_step_grid<true, false>();
  return cb ? attn_step_grid<false, true>() : attn_step_grid<false, false>();
}

static int check_attn_shape(int tokens, int hidden_size, int heads, int kv_heads, int head_dim, int rope_dim) {
  if (tokens < 1 || tokens > kAttnMaxTokens) return fail(FK_ERR_UNSUPPORTED, "tokens must be in [1, %d]", kAttnMaxTokens);
  if (hidden_size < 8 || hidden_size % 8 || hidden_size > 4096)
    return fail(FK_ERR_ALIGNMENT, "hidden_size must be a multiple of 8 in [8, 4096]");
  if (heads < 1 || kv_heads < 1 || heads % kv_heads) return fail(FK_ERR_INVALID, "heads must be a positive multiple of kv_heads");
  if (heads / kv_heads > 8) return fail(FK_ERR_UNSUPPORTED, "at most 8 query heads per kv head");
  if (kv_heads > kAttnMaxKvHeads) return fail(FK_ERR_UNSUPPORTED, "kv_heads must be <= %d", kAttnMaxKvHeads);
  if (head_dim < 4 || head_dim > kAttnMaxHeadDim || head_dim % 4)
    return fail(FK_ERR_UNSUPPORTED, "head_dim must be a multiple of 4 in [4, %d]", kAttnMaxHeadDim);
  if ((long long)heads * head_dim > 4096 || (heads * head_dim) % 8)
    return fail(FK_ERR_UNSUPPORTED, "heads * head_dim must be a multiple of 8 and <= 4096");
  if (rope_dim < 0) return fail(FK_ERR_INVALID, "rope_dim must be >= 0");
  return FK_OK;
}

}  // namespace fk

using namespace fk;

extern "C" {

size_t fk_attention_workspace_bytes(int tokens, int heads, int kv_heads, int head_dim) {
  if (tokens < 1 || heads < 1 || kv_heads < 1 || head_dim < 1) return 0;
  AttnWs ws;
  return attn_ws_layout(tokens, heads, kv_heads, head_dim, nullptr, &ws);
}

int fk_attention_project(const void* hidden, int hidden_dtype, const void* norm_weight, int norm_dtype,
                         const void* q_proj, const void* k_proj, const void* v_proj, int weight_dtype, int tokens,
                         int hidden_size, int q_rows, int kv_rows, float eps, float norm_offset, float* q_out,
                         float* k_out, float* v_out, void* stream) {
  if (tokens < 1) return fail(FK_ERR_INVALID, "tokens must be positive");
  if (hidden_size < 8 || hidden_size % 8 || hidden_size > 4096)
    return fail(FK_ERR_ALIGNMENT, "hidden_size must be a multiple of 8 in [8, 4096]");
  if (q_rows < 1 || kv_rows < 1) return fail(FK_ERR_INVALID, "projection row counts must be positive");
  if (!is_float_dtype(hidden_dtype) || !is_float_dtype(norm_dtype) || !is_float_dtype(weight_dtype))
    return fail(FK_ERR_DTYPE, "projection inputs must be f32 or bf16");
  if (!hidden || !norm_weight || !q_proj || !k_proj || !v_proj || !q_out || !k_out || !v_out)
    return fail(FK_ERR_INVALID, "projection pointers must be non-NULL");
  if (!aligned16(hidden) || !aligned16(norm_weight) || !aligned16(q_proj) || !aligned16(k_proj) || !aligned16(v_proj))
    return fail(FK_ERR_ALIGNMENT, "hidden, norm_weight and projection weights must be 16-byte aligned");
  if (hidden_size <= 2048 && q_rows % 4 == 0 && kv_rows % 4 == 0) {
    AttnProjArgs pa;
    pa.x = hidden;
    pa.nw = norm_weight;
    pa.nw_dt = norm_dtype;
    pa.w[0] = q_proj;
    pa.w[1] = k_proj;
    pa.w[2] = v_proj;
    pa.out[0] = q_out;
    pa.out[1] = k_out;
    pa.out[2] = v_out;
    pa.rows[0] = q_rows;
    pa.rows[1] = kv_rows;
    pa.rows[2] = kv_rows;
    pa.T = tokens;
    pa.H = hidden_size;
    pa.eps = eps;
    pa.off = norm_offset;
    const dim3 grid((unsigned)((q_rows + 2 * kv_rows + kAttnProjRows - 1) / kAttnProjRows));
    const bool bw = weight_dtype == FK_DTYPE_BF16, bx = hidden_dtype == FK_DTYPE_BF16;
    const hipStream_t s = as_stream(stream);
    if (bw && bx) hipLaunchKernelGGL((attn_proj_kernel<true, true>), grid, dim3(256), 0, s, pa);
    else if (bw) hipLaunchKernelGGL((attn_proj_kernel<true, false>), grid, dim3(256), 0, s, pa);
    else if (bx) hipLaunchKernelGGL((attn_proj_kernel<false, true>), grid, dim3(256), 0, s, pa);
    else hipLaunchKernelGGL((attn_proj_kernel<false, false>), grid, dim3(256), 0, s, pa);
    return check_launch("attn_proj_kernel");
  }
  const void* const w[4] = {q_proj, k_proj, v_proj, nullptr};
  const int rows[4] = {q_rows, kv_rows, kv_rows, 0};
  float* const out[4] = {q_out, k_out, v_out, nullptr};
  return launch_norm_projection(hidden, hidden_dtype, norm_weight, norm_dtype, w, rows, out, weight_dtype, tokens,
                                hidden_size, eps, norm_offset, as_stream(stream));
}

int fk_attention_decode(const void* hidden, int hidden_dtype, const void* norm_weight, int norm_dtype,
                        const void* q_proj, const void* k_proj, const void* v_proj, const void* o_proj,
                        int weight_dtype, const void* q_norm_weight, const void* k_norm_weight, int qk_norm_dtype,
                        void* key_cache, void* value_cache, int cache_dtype, int max_positions, int start_position,
                        const int32_t* start_position_device, int tokens, int hidden_size, int heads, int kv_heads, int head_dim, int rope_dim,
                        float rope_theta, int rope_interleaved, float eps, float qk_eps, float* update,
                        float* hidden_out, void* workspace, size_t workspace_bytes, void* stream) {
  int st = check_attn_shape(tokens, hidden_size, heads, kv_heads, head_dim, rope_dim);
  if (st) return st;
  if (max_positions < 1) return fail(FK_ERR_INVALID, "max_positions must be positive");
  if (!start_position_device && (start_position < 0 || start_position + tokens > max_positions))
    return fail(FK_ERR_INVALID, "decode positions [%d, %d) exceed the cache length %d", start_position,
                start_position + tokens, max_positions);
  if (!is_float_dtype(cache_dtype) || !is_float_dtype(qk_norm_dtype)) return fail(FK_ERR_DTYPE, "caches and q/k norms must be f32 or bf16");
  if (!key_cache || !value_cache || !o_proj || !q_norm_weight || !k_norm_weight || !update)
    return fail(FK_ERR_INVALID, "attention pointers must be non-NULL");
  if (!aligned16(o_proj) || !aligned16(key_cache) || !aligned16(value_cache))
    return fail(FK_ERR_ALIGNMENT, "o_proj and the caches must be 16-byte aligned");
  if (!rope_interleaved && rope_dim % 2) return fail(FK_ERR_INVALID, "half-split RoPE needs an even rope_dim");
  AttnWs ws;
  const size_t need = attn_ws_layout(tokens, heads, kv_heads, head_dim, nullptr, &ws);
  if (!workspace || workspace_bytes < need)
    return fail(FK_ERR_WORKSPACE, "attention workspace needs %zu bytes (got %zu)", need, workspace_bytes);
  attn_ws_layout(tokens, heads, kv_heads, head_dim, reinterpret_cast<char*>(workspace), &ws);
  const hipStream_t s = as_stream(stream);
  const int rd = rope_dim < head_dim ? rope_dim : head_dim;
  if (!is_float_dtype(hidden_dtype) || !is_float_dtype(norm_dtype) || !is_float_dtype(weight_dtype))
    return fail(FK_ERR_DTYPE, "projection inputs must be f32 or bf16");
  if (!hidden || !norm_weight || !q_proj || !k_proj || !v_proj)
    return fail(FK_ERR_INVALID, "projection pointers must be non-NULL");
  if (!aligned16(hidden) || !aligned16(norm_weight) || !aligned16(q_proj) || !aligned16(k_proj) || !aligned16(v_proj))
    return fail(FK_ERR_ALIGNMENT, "hidden, norm_weight and projection weights must be 16-byte aligned");
  if (tokens <= kAsMaxTokens) {
    const bool bx = hidden_dtype == FK_DTYPE_BF16, cb = cache_dtype == FK_DTYPE_BF16;
    const int G = attn_step_grid_for(bx, cb);
    const int nch = attn_step_chunks(tokens, hidden_size, heads, kv_heads, head_dim, weight_dtype, G);
    if (nch > 0) {
      AttnStepArgs sa;
      sa.x = hidden;
      sa.nw = norm_weight;
      sa.nw_dt = norm_dtype;
      sa.wq = q_proj;
      sa.wk = k_proj;
      sa.wv = v_proj;
      sa.wo = o_proj;
      sa.qn_w = q_norm_weight;
      sa.kn_w = k_norm_weight;
      sa.qn_dt = sa.kn_dt = qk_norm_dtype;
      sa.kc = key_cache;
      sa.vc = value_cache;
      sa.start_dev = const_cast<int*>(start_position_device);
      sa.start = start_position;
      sa.max_pos = max_positions;
      sa.T = tokens;
      sa.H = hidden_size;
      sa.heads = heads;
      sa.kvh = kv_heads;
      sa.hd = head_dim;
      sa.rope_dim = rd - rd % 2;
      sa.interleaved = rope_interleaved;
      sa.nch = nch;
      sa.theta_log2 = log2f(rope_theta);
      sa.eps = eps;
      sa.qk_eps = qk_eps;
      sa.update = update;
      sa.hidden_out = hidden_out;
      sa.tw = ws.tw;
      if (bx && cb) hipLaunchKernelGGL((attn_step_kernel<true, true>), dim3(G), dim3(kAsThreads), kAsMaxLds, s, sa);
      else if (bx) hipLaunchKernelGGL((attn_step_kernel<true, false>), dim3(G), dim3(kAsThreads), kAsMaxLds, s, sa);
      else if (cb) hipLaunchKernelGGL((attn_step_kernel<false, true>), dim3(G), dim3(kAsThreads), kAsMaxLds, s, sa);
      else hipLaunchKernelGGL((attn_step_kernel<false, false>), dim3(G), dim3(kAsThreads), kAsMaxLds, s, sa);
      return check_launch("attn_step_kernel");
    }
  }
  st = fk_attention_project(hidden, hidden_dtype, norm_weight, norm_dtype, q_proj, k_proj, v_proj, weight_dtype,
                            tokens, hidden_size, 2 * heads * head_dim, kv_heads * head_dim, eps, 1.0f, ws.qg, ws.k,
                            ws.v, stream);
  if (st) return st;
  AttnArgs a;
  a.qg = ws.qg;
  a.k = ws.k;
  a.v = ws.v;
  a.qn_w = q_norm_weight;
  a.kn_w = k_norm_weight;
  a.qn_dt = a.kn_dt = qk_norm_dtype;
  a.kc = key_cache;
  a.vc = value_cache;
  a.start = start_position;
  a.start_dev = start_position_device;
  a.max_pos = max_positions;
  a.T = tokens;
  a.heads = heads;
  a.kvh = kv_heads;
  a.hd = head_dim;
  a.rope_dim = rd - rd % 2;
  a.theta_log2 = log2f(rope_theta);
  a.eps = qk_eps;
  a.interleaved = rope_interleaved;
  a.gated = ws.gated;
  a.part = ws.part;
  // chunks of >= 32 positions, at most kAttnMaxChunks of them over the
  // positions the step can reach (the cache length when the position is
  // only known on the device)
  const int reach = start_position_device ? max_positions : start_position + tokens;
  a.chunk = (reach + kAttnMaxChunks - 1) / kAttnMaxChunks;
  if (a.chunk < 32) a.chunk = 32;  // contexts below 32 positions: one chunk, no merge
  a.max_chunks = kAttnMaxChunks;
  const int nchunks = (reach + a.chunk - 1) / a.chunk;
  // split a kv head's query heads over workgroups while the grid is small
  // (short contexts); long contexts keep them together (rows read once)
  const int G = heads / kv_heads;
  a.hsplit = 1;
  while (a.hsplit * 2 <= G && G % (a.hsplit * 2) == 0 && nchunks * kv_heads * tokens * a.hsplit < 128) a.hsplit *= 2;
  const dim3 grid((unsigned)nchunks, (unsigned)(kv_heads * a.hsplit), (unsigned)tokens);
  const size_t shm = (size_t)(8 + tokens) * head_dim * sizeof(float);
  if (cache_dtype == FK_DTYPE_BF16) hipLaunchKernelGGL(attn_split_kernel<true>, grid, dim3(256), shm, s, a);
  else hipLaunchKernelGGL(attn_split_kernel<false>, grid, dim3(256), shm, s, a);
  st = check_launch("attn_split_kernel");
  if (st) return st;
  if (nchunks > 1) {
    AttnMergeArgs ma;
    ma.qg = ws.qg;
    ma.part = ws.part;
    ma.gated = ws.gated;
    ma.start_dev = start_position_device;
    ma.start = start_position;
    ma.max_pos = max_positions;
    ma.T = tokens;
    ma.heads = heads;
    ma.hd = head_dim;
    ma.chunk = a.chunk;
    ma.max_chunks = kAttnMaxChunks;
    hipLaunchKernelGGL(attn_merge_kernel, dim3((unsigned)heads, (unsigned)tokens), dim3(256), 0, s, ma);
    st = check_launch("attn_merge_kernel");
    if (st) return st;
  }
  AttnOutArgs o;
  o.gated = ws.gated;
  o.wo = o_proj;
  o.x = hidden;
  o.x_dt = hidden_dtype;
  o.T = tokens;
  o.H = hidden_size;
  o.K = heads * head_dim;
  o.update = update;
  o.hidden_out = hidden_out;
  o.advance = const_cast<int*>(start_position_device);
  o.max_pos = max_positions;
  o.err = ws.tw.tickets + kWorkspaceErrorWord;
  const dim3 ogrid((unsigned)((hidden_size + kAttnOutRows - 1) / kAttnOutRows));
  if (weight_dtype == FK_DTYPE_BF16) hipLaunchKernelGGL(attn_out_kernel<true>, ogrid, dim3(256), 0, s, o);
  else hipLaunchKernelGGL(attn_out_kernel<false>, ogrid, dim3(256), 0, s, o);
  return check_launch("attn_out_kernel");
}

}  // extern "C"
