// Small standalone operators: expert histogram, fused SwiGLU, residual add,
// and the single-workgroup synthetic (tiny-spec) MoE and DeltaNet blocks used
// by the --moe-impl / --deltanet-impl switch of the synthetic decode bench.
#include "fk_common.h"
#include "fk_host.h"

namespace fk {

__device__ __forceinline__ long long load_index(const void* p, int dtype, size_t i) {
  return dtype == FK_DTYPE_I64 ? reinterpret_cast<const long long*>(p)[i]
                               : (long long)reinterpret_cast<const int*>(p)[i];
}

__global__ void fill_i32_kernel(int32_t* p, int n, int32_t v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

__global__ void histogram_kernel(const void* ids, int ids_dt, long long n, int E, int32_t* counts) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const long long e = load_index(ids, ids_dt, (size_t)i);
  if (e >= 0 && e < E) atomicAdd(&counts[e], 1);
}

__global__ void swiglu_kernel(const void* gu, int dt, long long rows, int I, void* out) {
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * I) return;
  const long long r = idx / I, i = idx - r * I;
  const float g = load_scalar(gu, dt, (size_t)(r * 2 * I + i));
  const float u = load_scalar(gu, dt, (size_t)(r * 2 * I + I + i));
  store_scalar(out, dt, (size_t)idx, silu(g) * u);
}

__global__ void residual_add_kernel(const void* x, int x_dt, const float* u, long long n, float* out) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = load_scalar(x, x_dt, (size_t)i) + u[i];
}

// ---------------------------------------------------------------------------
// Synthetic MoE (one token, one workgroup).  Semantics of
// reference_qwen36_moe_decode (reference/qwen36_decode.py:212-224): router on
// x * rsqrt(mean x^2 + eps) * w (plain weight), softmax top-k renormalised,
// routed experts + ungated shared expert on the raw x, plus the residual.
// ---------------------------------------------------------------------------
constexpr int kSynMax = 1024;

struct SynMoeArgs {
  const void* x;
  int x_dt;
  const void* nw;
  const void* rw;
  const void* gu;
  const void* dn;
  const void* sgu;
  const void* sdn;
  int w_dt;
  int H, E, I, K;
  float eps;
  void* out;
  int out_dt;
};

__global__ __launch_bounds__(256) void synthetic_moe_kernel(SynMoeArgs a) {
  __shared__ float s_x[kSynMax], s_n[kSynMax], s_logit[kSynMax], s_act[kSynMax], s_acc[kSynMax];
  __shared__ float s_red[4];
  __shared__ int s_sel[8];
  __shared__ float s_w[8];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  float ss = 0.f;
  for (int h = tid; h < a.H; h += 256) {
    const float v = load_scalar(a.x, a.x_dt, h);
    s_x[h] = v;
    ss = fmaf(v, v, ss);
    s_acc[h] = 0.f;
  }
  ss = wave_sum(ss);
  if (lane == 0) s_red[wave] = ss;
  __syncthreads();
  const float rs = rsqrtf((s_red[0] + s_red[1] + s_red[2] + s_red[3]) / (float)a.H + a.eps);
  for (int h = tid; h < a.H; h += 256) s_n[h] = s_x[h] * rs * load_scalar(a.nw, a.w_dt, h);
  __syncthreads();
  for (int e = tid; e < a.E; e += 256) {
    float d = 0.f;
    for (int h = 0; h < a.H; ++h) d = fmaf(s_n[h], load_scalar(a.rw, a.w_dt, (size_t)e * a.H + h), d);
    s_logit[e] = d;
  }
  __syncthreads();
  if (wave == 0) {
    float p[16];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int e = lane + kWave * j;
      p[j] = e < a.E ? s_logit[e] : -INFINITY;
      m = fmaxf(m, p[j]);
    }
    m = wave_max(m);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int e = lane + kWave * j;
      p[j] = e < a.E ? expf(p[j] - m) : 0.f;
      s += p[j];
    }
    s = wave_sum(s);
#pragma unroll
    for (int j = 0; j < 16; ++j) p[j] = p[j] / s;
    uint32_t taken = 0;
    float denom = 0.f;
    for (int k = 0; k < a.K; ++k) {
      uint64_t best = 0;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int e = lane + kWave * j;
        if (e < a.E && !((taken >> j) & 1u)) {
          const uint64_t key = ((uint64_t)__float_as_uint(p[j]) << 32) | (uint64_t)(0xffffffffu - (uint32_t)e);
          best = key > best ? key : best;
        }
      }
      best = wave_max_u64(best);
      const int sel = (int)(0xffffffffu - (uint32_t)(best & 0xffffffffu));
      const float v = __uint_as_float((uint32_t)(best >> 32));
      if ((sel & 63) == lane) taken |= 1u << (sel >> 6);
      denom += v;
      if (lane == 0) {
        s_sel[k] = sel;
        s_w[k] = v;
      }
    }
    if (lane == 0)
      for (int k = 0; k < a.K; ++k) s_w[k] /= denom;
  }
  __syncthreads();
  const size_t esz = a.w_dt == FK_DTYPE_BF16 ? 2 : 4;
  for (int k = 0; k <= a.K; ++k) {
    const bool shared = k == a.K;
    const char* gu = shared ? reinterpret_cast<const char*>(a.sgu)
                            : reinterpret_cast<const char*>(a.gu) + (size_t)s_sel[k] * 2 * a.I * a.H * esz;
    const char* dn = shared ? reinterpret_cast<const char*>(a.sdn)
                            : reinterpret_cast<const char*>(a.dn) + (size_t)s_sel[k] * a.H * a.I * esz;
    const float wk = shared ? 1.f : s_w[k];
    for (int i = tid; i < a.I; i += 256) {
      float g = 0.f, u = 0.f;
      for (int h = 0; h < a.H; ++h) {
        g = fmaf(load_scalar(gu, a.w_dt, (size_t)i * a.H + h), s_x[h], g);
        u = fmaf(load_scalar(gu, a.w_dt, (size_t)(a.I + i) * a.H + h), s_x[h], u);
      }
      s_act[i] = silu(g) * u;
    }
    __syncthreads();
    for (int h = tid; h < a.H; h += 256) {
      float d = 0.f;
      for (int i = 0; i < a.I; ++i) d = fmaf(load_scalar(dn, a.w_dt, (size_t)h * a.I + i), s_act[i], d);
      s_acc[h] = fmaf(wk, d, s_acc[h]);
    }
    __syncthreads();
  }
  for (int h = tid; h < a.H; h += 256) store_scalar(a.out, a.out_dt, h, s_x[h] + s_acc[h]);
}

// ---------------------------------------------------------------------------
// Synthetic DeltaNet (one token, one workgroup).  Semantics of
// reference_qwen36_deltanet_decode (reference/qwen36_decode.py:155-171).
// ---------------------------------------------------------------------------
struct SynDnArgs {
  const void* x;
  int x_dt;
  const void* state;
  int s_dt;
  const void* nw;
  const void* qw;
  const void* kw;
  const void* vw;
  const void* gw;
  const void* ow;
  int w_dt;
  int H, Hk, D, Vd;
  float eps;
  void* x_out;
  void* s_out;
};

__global__ __launch_bounds__(256) void synthetic_deltanet_kernel(SynDnArgs a) {
  __shared__ float s_x[kSynMax], s_xn[kSynMax], s_q[kSynMax], s_k[kSynMax], s_v[kSynMax], s_g[kSynMax], s_r[kSynMax];
  __shared__ float s_red[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int QW = a.Hk * a.D, VW = a.Hk * a.Vd;
  float ss = 0.f;
  for (int h = tid; h < a.H; h += 256) {
    const float v = load_scalar(a.x, a.x_dt, h);
    s_x[h] = v;
    ss = fmaf(v, v, ss);
  }
  ss = wave_sum(ss);
  if (lane == 0) s_red[wave] = ss;
  __syncthreads();
  const float rs = rsqrtf((s_red[0] + s_red[1] + s_red[2] + s_red[3]) / (float)a.H + a.eps);
  for (int h = tid; h < a.H; h += 256) s_xn[h] = s_x[h] * rs * load_scalar(a.nw, a.w_dt, h);
  __syncthreads();
  for (int r = tid; r < QW; r += 256) {
    float q = 0.f, k = 0.f;
    for (int h = 0; h < a.H; ++h) {
      q = fmaf(load_scalar(a.qw, a.w_dt, (size_t)r * a.H + h), s_xn[h], q);
      k = fmaf(load_scalar(a.kw, a.w_dt, (size_t)r * a.H + h), s_xn[h], k);
    }
    s_q[r] = q;
    s_k[r] = k;
  }
  for (int r = tid; r < VW; r += 256) {
    float v = 0.f, g = 0.f;
    for (int h = 0; h < a.H; ++h) {
      v = fmaf(load_scalar(a.vw, a.w_dt, (size_t)r * a.H + h), s_xn[h], v);
      g = fmaf(load_scalar(a.gw, a.w_dt, (size_t)r * a.H + h), s_xn[h], g);
    }
    s_v[r] = v;
    s_g[r] = sigmoid(g);
  }
  __syncthreads();
  // New state and the gated read-out, one thread per (head, value column).
  for (int hv = tid; hv < VW; hv += 256) {
    const int hh = hv / a.Vd, vv = hv - hh * a.Vd;
    float r = 0.f;
    for (int d = 0; d < a.D; ++d) {
      const size_t si = ((size_t)hh * a.D + d) * a.Vd + vv;
      const float ns = 0.95f * load_scalar(a.state, a.s_dt, si) + s_k[hh * a.D + d] * s_v[hv];
      store_scalar(a.s_out, a.s_dt, si, ns);
      r = fmaf(s_q[hh * a.D + d], ns, r);
    }
    s_r[hv] = r * s_g[hv];
  }
  __syncthreads();
  for (int h = tid; h < a.H; h += 256) {
    float d = 0.f;
    for (int j = 0; j < VW; ++j) d = fmaf(load_scalar(a.ow, a.w_dt, (size_t)h * VW + j), s_r[j], d);
    store_scalar(a.x_out, a.x_dt, h, s_x[h] + d);
  }
}

// ---------------------------------------------------------------------------
// Synthetic grouped-query attention (one token, one workgroup).  Semantics of
// reference_qwen36_attention_decode (reference/qwen36_decode.py:174-209),
// rounded where triton_synthetic_qwen36_attention_decode
// (kernels/triton/qwen36_attention.py:852-998) stores its intermediates:
// q, k and v are projected in fp32 from the plain-weight RMSNorm and held in
// the hidden dtype; RoPE (interleaved pairs, angle position / 10^4^(2i/r))
// turns q (held in the hidden dtype) and k; the new k and v rows go to row
// `position` of the caches (cache dtype); every query head attends over
// cache rows 0..position of its kv head (softmax of q.k / sqrt(head_dim));
// out = x + W_o attended, attended held in the hidden dtype.
// ---------------------------------------------------------------------------
constexpr int kSynAttnMax = 128;  // hidden, query and kv widths, cache rows

struct SynAttnArgs {
  const void* x;
  int x_dt;
  void* kc;
  void* vc;
  int c_dt;
  const void* nw;
  const void* qw;
  const void* kw;
  const void* vw;
  const void* ow;
  int w_dt;
  int H, heads, kvh, hd, rope_dim, pos;
  float eps;
  void* out;
};

__device__ __forceinline__ float round_to_dtype(int dtype, float v) {
  return dtype == FK_DTYPE_BF16 ? bf16_bits_to_f32(f32_to_bf16_bits(v)) : v;
}

__global__ __launch_bounds__(256) void synthetic_attention_kernel(SynAttnArgs a) {
  __shared__ float s_x[kSynAttnMax], s_xn[kSynAttnMax], s_p[3 * kSynAttnMax];  // s_p: q | k | v (hidden dtype)
  __shared__ float s_q[kSynAttnMax], s_k[kSynAttnMax], s_v[kSynAttnMax], s_att[kSynAttnMax];
  __shared__ float s_red[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int QW = a.heads * a.hd, KW = a.kvh * a.hd, P = a.pos + 1;
  float ss = 0.f;
  for (int h = tid; h < a.H; h += 256) {
    const float v = load_scalar(a.x, a.x_dt, h);
    s_x[h] = v;
    ss = fmaf(v, v, ss);
  }
  ss = wave_sum(ss);
  if (lane == 0) s_red[wave] = ss;
  __syncthreads();
  const float rs = rsqrtf((s_red[0] + s_red[1] + s_red[2] + s_red[3]) / (float)a.H + a.eps);
  for (int h = tid; h < a.H; h += 256) s_xn[h] = s_x[h] * rs * load_scalar(a.nw, a.w_dt, h);
  __syncthreads();
  // q | k | v rows, held in the hidden dtype
  for (int r = tid; r < QW + 2 * KW; r += 256) {
    const void* w = r < QW ? a.qw : r < QW + KW ? a.kw : a.vw;
    const int row = r < QW ? r : r < QW + KW ? r - QW : r - QW - KW;
    float acc = 0.f;
    for (int h = 0; h < a.H; ++h) acc = fmaf(load_scalar(w, a.w_dt, (size_t)row * a.H + h), s_xn[h], acc);
    s_p[r] = round_to_dtype(a.x_dt, acc);
  }
  __syncthreads();
  // RoPE on q and k; the new k and v rows into the caches
  int rot = a.rope_dim < a.hd ? a.rope_dim : a.hd;
  rot -= rot % 2;
  for (int i = tid; i < QW + KW; i += 256) {
    const bool isq = i < QW;
    const int j = isq ? i : i - QW, dim = j % a.hd;
    const float* src = isq ? s_p : s_p + QW;
    float v = src[j];
    if (dim < rot) {
      const float pair = src[j - dim + (dim ^ 1)];
      const float ang = (float)a.pos / expf(logf(10000.0f) * ((float)(dim & ~1) / (float)rot));
      const float c = cosf(ang), sn = sinf(ang);
      v = (dim & 1) ? pair * sn + v * c : v * c - pair * sn;
    }
    if (isq) {
      s_q[j] = round_to_dtype(a.x_dt, v);
    } else {
      s_k[j] = round_to_dtype(a.c_dt, v);
      const float vv = s_p[QW + KW + j];
      s_v[j] = round_to_dtype(a.c_dt, vv);
      store_scalar(a.kc, a.c_dt, (size_t)a.pos * KW + j, v);
      store_scalar(a.vc, a.c_dt, (size_t)a.pos * KW + j, vv);
    }
  }
  __syncthreads();
  // Wavefront w takes query heads w, w + 4, ...; lane l positions l, l + 64
  // (the new row from LDS, older rows from the cache).
  const float scale = rsqrtf((float)a.hd);
  const int group = a.heads / a.kvh;
  for (int h = wave; h < a.heads; h += 4) {
    const int kv = h / group;
    float sc[2], e[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int t = lane + 64 * u;
      sc[u] = -INFINITY;
      if (t < P) {
        float d = 0.f;
        for (int dd = 0; dd < a.hd; ++dd) {
          const float kvl = t == a.pos ? s_k[kv * a.hd + dd] : load_scalar(a.kc, a.c_dt, (size_t)t * KW + kv * a.hd + dd);
          d = fmaf(kvl, s_q[h * a.hd + dd], d);
        }
        sc[u] = d * scale;
      }
    }
    const float m = wave_max(fmaxf(sc[0], sc[1]));
#pragma unroll
    for (int u = 0; u < 2; ++u) e[u] = lane + 64 * u < P ? expf(sc[u] - m) : 0.f;
    const float den = wave_sum(e[0] + e[1]);
    for (int dd = 0; dd < a.hd; ++dd) {
      float part = 0.f;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int t = lane + 64 * u;
        if (t < P) {
          const float vl = t == a.pos ? s_v[kv * a.hd + dd] : load_scalar(a.vc, a.c_dt, (size_t)t * KW + kv * a.hd + dd);
          part = fmaf(e[u] / den, vl, part);
        }
      }
      part = wave_sum(part);
      if (lane == 0) s_att[h * a.hd + dd] = round_to_dtype(a.x_dt, part);
    }
  }
  __syncthreads();
  for (int h = tid; h < a.H; h += 256) {
    float d = 0.f;
    for (int j = 0; j < QW; ++j) d = fmaf(load_scalar(a.ow, a.w_dt, (size_t)h * QW + j), s_att[j], d);
    store_scalar(a.out, a.x_dt, h, s_x[h] + d);
  }
}

}  // namespace fk

using namespace fk;

// Read-only stream (bandwidth probe): workgroup g loads the 16 KiB at
// [src + 16 KiB g, + 16 KiB) once, non-temporal, each wavefront its own
// 4 KiB as four 1 KiB instructions all in flight, so every workgroup is a
// short one-shot burst like an expert-stage work item.  Of the read shapes
// measured over 4 GiB on this part this one was the fastest (7.1-7.2 TB/s;
// one-shot chunks of 4-32 KiB per workgroup all reach 7.1, a grid-stride
// stream 6.5-6.8).  The values feed an XOR whose result is stored only if it
// hits a value the host never passes, so the loads stay and nothing is
// written; vectors past n16 (a partial last chunk) are not loaded.
constexpr int kStreamChunk16 = 1024;  // 16-byte vectors per workgroup (16 KiB)
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* src, size_t n16, uint32_t never,
                                                          uint32_t* sink) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const size_t base = (size_t)blockIdx.x * kStreamChunk16 + (size_t)w * 256 + lane;
  u32x4 v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const size_t i = base + (size_t)j * 64;
    v[j] = i < n16 ? __builtin_nontemporal_load(src + i) : u32x4{0u, 0u, 0u, 0u};
  }
  uint32_t acc = 0u;
#pragma unroll
  for (int j = 0; j < 4; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
  if (acc == never) sink[0] = acc;
}

extern "C" {

int fk_stream_read(const void* src, size_t bytes, uint32_t* sink, void* stream) {
  if (!src || !sink) return fail(FK_ERR_INVALID, "src and sink must be non-NULL");
  if (!aligned16(src) || bytes % 16) return fail(FK_ERR_ALIGNMENT, "src must be 16-byte aligned and bytes a multiple of 16");
  const size_t n16 = bytes / 16, groups = (n16 + kStreamChunk16 - 1) / kStreamChunk16;
  if (groups == 0) return FK_OK;
  if (groups > 0x7fffffffull) return fail(FK_ERR_UNSUPPORTED, "bytes must be below 32 TiB");
  hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)groups), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const u32x4*>(src), n16, 0x9e3779b9u, sink);
  return check_launch("stream_read_kernel");
}

int fk_expert_histogram(const void* ids, int ids_dtype, int64_t n, int num_experts, int32_t* counts, void* stream) {
  if (!is_index_dtype(ids_dtype)) return fail(FK_ERR_DTYPE, "ids must be int32 or int64");
  if (num_experts < 1) return fail(FK_ERR_INVALID, "num_experts must be positive");
  if (n < 0) return fail(FK_ERR_INVALID, "n must be >= 0");
  if (!counts || (n > 0 && !ids)) return fail(FK_ERR_INVALID, "ids/counts must be non-NULL");
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(fill_i32_kernel, dim3((num_experts + 255) / 256), dim3(256), 0, s, counts, num_experts, 0);
  int st = check_launch("fill_i32_kernel");
  if (st || n == 0) return st;
  hipLaunchKernelGGL(histogram_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, ids, ids_dtype,
                     (long long)n, num_experts, counts);
  return check_launch("histogram_kernel");
}

int fk_fused_swiglu(const void* gate_up, int dtype, int64_t rows, int intermediate, void* out, void* stream) {
  if (!is_float_dtype(dtype)) return fail(FK_ERR_DTYPE, "gate_up must be f32 or bf16");
  if (rows < 0 || intermediate < 1) return fail(FK_ERR_INVALID, "rows must be >= 0 and intermediate positive");
  const long long n = (long long)rows * intermediate;
  if (n == 0) return FK_OK;
  if (!gate_up || !out) return fail(FK_ERR_INVALID, "gate_up/out must be non-NULL");
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, as_stream(stream), gate_up,
                     dtype, (long long)rows, intermediate, out);
  return check_launch("swiglu_kernel");
}

int fk_residual_add(const void* hidden, int hidden_dtype, const float* update, int64_t n, float* out, void* stream) {
  if (!is_float_dtype(hidden_dtype)) return fail(FK_ERR_DTYPE, "hidden must be f32 or bf16");
  if (n < 0) return fail(FK_ERR_INVALID, "n must be >= 0");
  if (n == 0) return FK_OK;
  if (!hidden || !update || !out) return fail(FK_ERR_INVALID, "pointers must be non-NULL");
  hipLaunchKernelGGL(residual_add_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, as_stream(stream), hidden,
                     hidden_dtype, update, (long long)n, out);
  return check_launch("residual_add_kernel");
}

int fk_synthetic_moe(const void* hidden, int hidden_dtype, const void* norm_weight, const void* router_weight,
                     const void* gate_up, const void* down, const void* shared_gate_up, const void* shared_down,
                     int weight_dtype, int hidden_size, int num_experts, int intermediate, int top_k, float eps,
                     void* out, int out_dtype, void* stream) {
  if (!is_float_dtype(hidden_dtype) || !is_float_dtype(weight_dtype) || !is_float_dtype(out_dtype))
    return fail(FK_ERR_DTYPE, "synthetic MoE tensors must be f32 or bf16");
  if (hidden_size < 1 || hidden_size > kSynMax || intermediate < 1 || intermediate > kSynMax)
    return fail(FK_ERR_UNSUPPORTED, "synthetic MoE supports hidden/intermediate in [1, %d]", kSynMax);
  if (num_experts < 1 || num_experts > kSynMax) return fail(FK_ERR_UNSUPPORTED, "num_experts must be in [1, %d]", kSynMax);
  if (top_k < 1 || top_k > 8 || top_k > num_experts) return fail(FK_ERR_INVALID, "top_k must be in [1, min(8, experts)]");
  if (!hidden || !norm_weight || !router_weight || !gate_up || !down || !shared_gate_up || !shared_down || !out)
    return fail(FK_ERR_INVALID, "synthetic MoE pointers must be non-NULL");
  SynMoeArgs sa;
  sa.x = hidden;
  sa.x_dt = hidden_dtype;
  sa.nw = norm_weight;
  sa.rw = router_weight;
  sa.gu = gate_up;
  sa.dn = down;
  sa.sgu = shared_gate_up;
  sa.sdn = shared_down;
  sa.w_dt = weight_dtype;
  sa.H = hidden_size;
  sa.E = num_experts;
  sa.I = intermediate;
  sa.K = top_k;
  sa.eps = eps;
  sa.out = out;
  sa.out_dt = out_dtype;
  hipLaunchKernelGGL(synthetic_moe_kernel, dim3(1), dim3(256), 0, as_stream(stream), sa);
  return check_launch("synthetic_moe_kernel");
}

int fk_synthetic_deltanet(const void* hidden, int hidden_dtype, const void* state, int state_dtype,
                          const void* norm_weight, const void* q_weight, const void* k_weight, const void* v_weight,
                          const void* gate_weight, const void* out_weight, int weight_dtype, int hidden_size,
                          int qk_heads, int head_dim, int value_dim_per_head, float eps, void* hidden_out,
                          void* state_out, void* stream) {
  if (!is_float_dtype(hidden_dtype) || !is_float_dtype(state_dtype) || !is_float_dtype(weight_dtype))
    return fail(FK_ERR_DTYPE, "synthetic DeltaNet tensors must be f32 or bf16");
  if (hidden_size < 1 || qk_heads < 1 || head_dim < 1 || value_dim_per_head < 1)
    return fail(FK_ERR_INVALID, "synthetic DeltaNet sizes must be positive");
  if (hidden_size > kSynMax || qk_heads * head_dim > kSynMax || qk_heads * value_dim_per_head > kSynMax)
    return fail(FK_ERR_UNSUPPORTED, "synthetic DeltaNet widths must be <= %d", kSynMax);
  if (!hidden || !state || !norm_weight || !q_weight || !k_weight || !v_weight || !gate_weight || !out_weight ||
      !hidden_out || !state_out)
    return fail(FK_ERR_INVALID, "synthetic DeltaNet pointers must be non-NULL");
  SynDnArgs da;
  da.x = hidden;
  da.x_dt = hidden_dtype;
  da.state = state;
  da.s_dt = state_dtype;
  da.nw = norm_weight;
  da.qw = q_weight;
  da.kw = k_weight;
  da.vw = v_weight;
  da.gw = gate_weight;
  da.ow = out_weight;
  da.w_dt = weight_dtype;
  da.H = hidden_size;
  da.Hk = qk_heads;
  da.D = head_dim;
  da.Vd = value_dim_per_head;
  da.eps = eps;
  da.x_out = hidden_out;
  da.s_out = state_out;
  hipLaunchKernelGGL(synthetic_deltanet_kernel, dim3(1), dim3(256), 0, as_stream(stream), da);
  return check_launch("synthetic_deltanet_kernel");
}

int fk_synthetic_attention(const void* hidden, int hidden_dtype, void* key_cache, void* value_cache, int cache_dtype,
                           const void* norm_weight, const void* q_weight, const void* k_weight, const void* v_weight,
                           const void* out_weight, int weight_dtype, int hidden_size, int attention_heads,
                           int kv_heads, int head_dim, int rope_dim, int position, int max_positions, float eps,
                           void* out, void* stream) {
  if (!is_float_dtype(hidden_dtype) || !is_float_dtype(cache_dtype) || !is_float_dtype(weight_dtype))
    return fail(FK_ERR_DTYPE, "synthetic attention tensors must be f32 or bf16");
  if (hidden_size < 1 || attention_heads < 1 || kv_heads < 1 || head_dim < 1 || max_positions < 1)
    return fail(FK_ERR_INVALID, "synthetic attention sizes must be positive");
  if (attention_heads % kv_heads != 0) return fail(FK_ERR_INVALID, "attention_heads must be a multiple of kv_heads");
  if (position < 0 || position >= max_positions) return fail(FK_ERR_INVALID, "position must be in [0, max_positions)");
  if (hidden_size > kSynAttnMax || attention_heads * head_dim > kSynAttnMax || kv_heads * head_dim > kSynAttnMax ||
      max_positions > kSynAttnMax)
    return fail(FK_ERR_UNSUPPORTED, "synthetic attention widths and cache length must be <= %d", kSynAttnMax);
  if (!hidden || !key_cache || !value_cache || !norm_weight || !q_weight || !k_weight || !v_weight || !out_weight ||
      !out)
    return fail(FK_ERR_INVALID, "synthetic attention pointers must be non-NULL");
  SynAttnArgs sa;
  sa.x = hidden;
  sa.x_dt = hidden_dtype;
  sa.kc = key_cache;
  sa.vc = value_cache;
  sa.c_dt = cache_dtype;
  sa.nw = norm_weight;
  sa.qw = q_weight;
  sa.kw = k_weight;
  sa.vw = v_weight;
  sa.ow = out_weight;
  sa.w_dt = weight_dtype;
  sa.H = hidden_size;
  sa.heads = attention_heads;
  sa.kvh = kv_heads;
  sa.hd = head_dim;
  sa.rope_dim = rope_dim < 0 ? 0 : rope_dim;
  sa.pos = position;
  sa.eps = eps;
  sa.out = out;
  hipLaunchKernelGGL(synthetic_attention_kernel, dim3(1), dim3(256), 0, as_stream(stream), sa);
  return check_launch("synthetic_attention_kernel");
}

}  // extern "C"
