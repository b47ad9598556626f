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
// Kernels (four launches per step):
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

struct AttnWs {
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
    return base ? reinterpret_cast<float*>(base + at) : nullptr;
  };
  ws->qg = take((size_t)T * heads * 2 * hd * 4);
  ws->k = take((size_t)T * kvh * hd * 4);
  ws->v = take((size_t)T * kvh * hd * 4);
  ws->gated = take((size_t)T * heads * hd * 4);
  ws->part = take((size_t)T * heads * kAttnMaxChunks * (hd + 2) * 4);
  return off;
}

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
  // the attention launch before this one has read the position
  if (a.advance && blockIdx.x == 0 && threadIdx.x == 0) *a.advance += a.T;
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
  const int rd = rope_dim < head_dim ? rope_dim : head_dim;
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
  const dim3 ogrid((unsigned)((hidden_size + kAttnOutRows - 1) / kAttnOutRows));
  if (weight_dtype == FK_DTYPE_BF16) hipLaunchKernelGGL(attn_out_kernel<true>, ogrid, dim3(256), 0, s, o);
  else hipLaunchKernelGGL(attn_out_kernel<false>, ogrid, dim3(256), 0, s, o);
  return check_launch("attn_out_kernel");
}

}  // extern "C"
