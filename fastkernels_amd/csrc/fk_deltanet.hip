// Qwen3.6 Gated DeltaNet decode step for gfx950.
//
// Semantics follow the reference oracle (reference/qwen36_real.py:111-260):
//   xn = RMSNorm(x) * (1 + w)                       projections qkv, z, a, b
//   conv: y_t = silu(sum_j w[c,j] * [state | qkv^T][c, t+1+j]); state' = last KS columns
//   per value head h (qk head h / (Hv/Hk)), tokens in order through one state S[h] (D x D):
//     q = l2n(q) * D^-1/2, k = l2n(k), beta = sigmoid(b), g = -exp(A_log) * softplus(a + dt_bias)
//     S *= exp(g);  delta = (v - k^T S) * beta;  S += k delta^T;  o = q^T S
//   core = o * rsqrt(mean(o^2) + eps) * w_lin * silu(z)   (plain weight, per head)
//   update = core W_out^T
//
// Kernels:
//   deltanet_project_kernel   grid ceil(R/16): 16 rows of the concatenated
//                             [qkv | z | a | b] weight space per workgroup,
//                             streamed once and applied to every token.
//   deltanet_conv_kernel      one thread per channel, sliding window in registers.
//   deltanet_recurrent_kernel grid (Hv, ceil(D/32)); a workgroup owns a
//                             D x 32 fp32 state tile in registers (16 rows per
//                             thread at D=128) for all tokens.  The last of a
//                             head's workgroups to finish (atomic ticket) applies
//                             the gated RMSNorm for that head.
//   deltanet_out_kernel       grid ceil(hidden/8): GEMV over W_out rows plus
//                             the optional residual.
#include "fk_common.h"
#include "fk_host.h"

namespace fk {

constexpr int kProjRows = 16;   // rows per projection workgroup (4 per wave)
constexpr int kRecCols = 32;    // state columns per recurrent workgroup
constexpr int kRecMaxRows = 16; // state rows per thread (D <= 128)
constexpr int kOutRows = 8;     // W_out rows per workgroup (2 per wave)

struct DnWs {
  uint32_t* tickets;  // [Hv]
  float* core;        // [T, Hv*D] raw recurrent output
  float* normed;      // [T, Hv*D] gated-RMSNorm output
};

static size_t dn_ws_layout(int T, int Hv, int D, char* base, DnWs* ws) {
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t at = off;
    off = align_up(off + bytes, 256);
    return base ? base + at : nullptr;
  };
  ws->tickets = reinterpret_cast<uint32_t*>(take((size_t)Hv * 4));
  ws->core = reinterpret_cast<float*>(take((size_t)T * Hv * D * 4));
  ws->normed = reinterpret_cast<float*>(take((size_t)T * Hv * D * 4));
  return off;
}

// ---------------------------------------------------------------------------
// Projections
// ---------------------------------------------------------------------------
struct ProjArgs {
  const void* x;
  const void* nw;
  int nw_dt;
  const void* w[4];
  float* out[4];
  int rows[4];
  int T, H;
  float eps, off;
};

template <bool BFW, bool BFX, int NJ>
__global__ __launch_bounds__(256) void deltanet_project_kernel(ProjArgs a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nch = a.H >> 3;
  const int R = a.rows[0] + a.rows[1] + a.rows[2] + a.rows[3];
  const int rbase = blockIdx.x * kProjRows + wave * 4;
  const size_t esz = BFW ? 2 : 4;

  const char* wp[4];
  float* op[4];
  int ostride[4];
  bool ok[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    int row = rbase + r;
    ok[r] = row < R;
    int which = 0;
    if (ok[r]) {
      while (row >= a.rows[which]) {
        row -= a.rows[which];
        ++which;
      }
    } else {
      row = 0;
    }
    wp[r] = reinterpret_cast<const char*>(a.w[which]) + (size_t)row * a.H * esz;
    op[r] = a.out[which] + row;
    ostride[r] = a.rows[which];
  }

  Raw8<BFW> wr[4][NJ];
  float nwv[NJ][8];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int c = lane + kWave * j;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (c < nch && ok[r]) wr[r][j] = load_raw8_stream<BFW>(wp[r], (size_t)c * 8);
#pragma unroll
    for (int q = 0; q < 8; ++q) nwv[j][q] = c < nch ? a.off + load_scalar(a.nw, a.nw_dt, (size_t)c * 8 + q) : 0.f;
  }

  for (int t = 0; t < a.T; ++t) {
    float ss = 0.f;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int c = lane + kWave * j;
      if (c < nch) {
        float x8[8];
        load8_f32<BFX>(a.x, (size_t)t * a.H + (size_t)c * 8, x8);
        float xn[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          ss = fmaf(x8[q], x8[q], ss);
          xn[q] = x8[q] * nwv[j][q];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (ok[r]) {
            float w8[8];
            raw8_to_f32<BFW>(wr[r][j], w8);
#pragma unroll
            for (int q = 0; q < 8; ++q) acc[r] = fmaf(w8[q], xn[q], acc[r]);
          }
        }
      }
    }
    ss = wave_sum(ss);
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = wave_sum(acc[r]);
    const float rs = rsqrtf(ss / (float)a.H + a.eps);
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (ok[r]) op[r][(size_t)t * ostride[r]] = acc[r] * rs;
    }
  }
}

// ---------------------------------------------------------------------------
// Causal depthwise conv + SiLU + state roll
// ---------------------------------------------------------------------------
struct ConvArgs {
  const void* mixed;
  int mixed_dt;
  const void* state;
  int state_dt;
  const void* w;
  int w_dt;
  int T, C, KS;
  float* out;
  void* next_state;
};

__global__ __launch_bounds__(256) void deltanet_conv_kernel(ConvArgs a) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= a.C) return;
  float win[8];
  float wk[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    win[j] = j < a.KS ? load_scalar(a.state, a.state_dt, (size_t)c * a.KS + j) : 0.f;
    wk[j] = j < a.KS ? load_scalar(a.w, a.w_dt, (size_t)c * a.KS + j) : 0.f;
  }
  for (int t = 0; t < a.T; ++t) {
    const float v = load_scalar(a.mixed, a.mixed_dt, (size_t)t * a.C + c);
#pragma unroll
    for (int j = 0; j < 7; ++j)
      if (j + 1 < a.KS) win[j] = win[j + 1];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (j == a.KS - 1) win[j] = v;
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (j < a.KS) acc = fmaf(wk[j], win[j], acc);
    a.out[(size_t)t * a.C + c] = silu(acc);
  }
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (j < a.KS) store_scalar(a.next_state, a.state_dt, (size_t)c * a.KS + j, win[j]);
}

// ---------------------------------------------------------------------------
// Recurrent gated delta rule + per-head gated RMSNorm
// ---------------------------------------------------------------------------
struct RecArgs {
  const void* mixed;
  const void* z;
  const void* a_in;
  const void* b_in;
  const void* state;
  const void* lnw;
  const void* a_log;
  const void* dt_bias;
  int dt[10];  // mixed, z, a, b, state, out_w, lnw, a_log, dt_bias, residual
  int T, Hk, Hv, D;
  float eps;
  void* next_state;
  DnWs ws;
};

__device__ __forceinline__ float softplus_stable(float x) {
  return fmaxf(x, 0.f) + log1pf(expf(-fabsf(x)));
}

__global__ __launch_bounds__(256) void deltanet_recurrent_kernel(RecArgs a) {
  __shared__ float s_q[128];
  __shared__ float s_k[128];
  __shared__ float s_red[256];
  __shared__ float s_scal[4];  // decay, beta, q scale, k scale
  __shared__ int s_last;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = blockIdx.x;
  const int CB = a.D < kRecCols ? a.D : kRecCols;
  const int RG = 256 / CB;                      // row groups
  const int RPT = (a.D + RG - 1) / RG;          // rows per thread (<= 16)
  const int col = tid % CB, rg = tid / CB;
  const int c = blockIdx.y * CB + col;
  const bool col_ok = c < a.D && rg < RG;
  const int qk_head = h / (a.Hv / a.Hk);
  const size_t mixed_w = (size_t)2 * a.Hk * a.D + (size_t)a.Hv * a.D;
  const size_t sbase = (size_t)h * a.D * a.D;

  float S[kRecMaxRows];
#pragma unroll
  for (int k = 0; k < kRecMaxRows; ++k) {
    const int i = rg * RPT + k;
    S[k] = (col_ok && k < RPT && i < a.D) ? load_scalar(a.state, a.dt[4], sbase + (size_t)i * a.D + c) : 0.f;
  }
  const float a_log = load_scalar(a.a_log, a.dt[7], h);
  const float dt_bias = load_scalar(a.dt_bias, a.dt[8], h);

  for (int t = 0; t < a.T; ++t) {
    const size_t mrow = (size_t)t * mixed_w;
    if (tid < a.D) {
      s_q[tid] = load_scalar(a.mixed, a.dt[0], mrow + (size_t)qk_head * a.D + tid);
      s_k[tid] = load_scalar(a.mixed, a.dt[0], mrow + (size_t)a.Hk * a.D + (size_t)qk_head * a.D + tid);
    }
    __syncthreads();
    if (wave == 0) {
      float sq = 0.f, sk = 0.f;
      for (int i = lane; i < a.D; i += kWave) {
        sq = fmaf(s_q[i], s_q[i], sq);
        sk = fmaf(s_k[i], s_k[i], sk);
      }
      sq = wave_sum(sq);
      sk = wave_sum(sk);
      if (lane == 0) {
        const float gin = load_scalar(a.a_in, a.dt[2], (size_t)t * a.Hv + h) + dt_bias;
        const float g = -expf(a_log) * softplus_stable(gin);
        s_scal[0] = expf(g);
        s_scal[1] = 1.f / (1.f + expf(-load_scalar(a.b_in, a.dt[3], (size_t)t * a.Hv + h)));
        s_scal[2] = rsqrtf(sq + a.eps) * rsqrtf((float)a.D);
        s_scal[3] = rsqrtf(sk + a.eps);
      }
    }
    __syncthreads();
    const float decay = s_scal[0], beta = s_scal[1], qs = s_scal[2], ks = s_scal[3];
    float kv[kRecMaxRows], qv[kRecMaxRows];
    float part = 0.f;
#pragma unroll
    for (int k = 0; k < kRecMaxRows; ++k) {
      const int i = rg * RPT + k;
      const bool ok = col_ok && k < RPT && i < a.D;
      kv[k] = ok ? s_k[i] * ks : 0.f;
      qv[k] = ok ? s_q[i] * qs : 0.f;
      S[k] *= decay;
      part = fmaf(S[k], kv[k], part);
    }
    s_red[tid] = part;
    __syncthreads();
    float proj = 0.f;
    for (int g = 0; g < RG; ++g) proj += s_red[g * CB + col];
    const float v = col_ok ? load_scalar(a.mixed, a.dt[0], mrow + (size_t)2 * a.Hk * a.D + (size_t)h * a.D + c) : 0.f;
    const float delta = (v - proj) * beta;
    float opart = 0.f;
#pragma unroll
    for (int k = 0; k < kRecMaxRows; ++k) {
      S[k] = fmaf(kv[k], delta, S[k]);
      opart = fmaf(S[k], qv[k], opart);
    }
    __syncthreads();  // everyone has read s_red
    s_red[tid] = opart;
    __syncthreads();
    if (rg == 0 && c < a.D) {
      float o = 0.f;
      for (int g = 0; g < RG; ++g) o += s_red[g * CB + col];
      a.ws.core[(size_t)t * a.Hv * a.D + (size_t)h * a.D + c] = o;
    }
    __syncthreads();
  }

#pragma unroll
  for (int k = 0; k < kRecMaxRows; ++k) {
    const int i = rg * RPT + k;
    if (col_ok && k < RPT && i < a.D) store_scalar(a.next_state, a.dt[4], sbase + (size_t)i * a.D + c, S[k]);
  }

  // The last column block of head h applies the gated RMSNorm for the head.
  __threadfence();
  __syncthreads();
  if (tid == 0) s_last = atomicAdd(&a.ws.tickets[h], 1u) == gridDim.y - 1;
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  for (int t = wave; t < a.T; t += 4) {
    const size_t base = (size_t)t * a.Hv * a.D + (size_t)h * a.D;
    float ss = 0.f;
    for (int j = lane; j < a.D; j += kWave) {
      const float o = __builtin_nontemporal_load(a.ws.core + base + j);
      ss = fmaf(o, o, ss);
    }
    ss = wave_sum(ss);
    const float rs = rsqrtf(ss / (float)a.D + a.eps);
    for (int j = lane; j < a.D; j += kWave) {
      const float o = __builtin_nontemporal_load(a.ws.core + base + j);
      const float zz = load_scalar(a.z, a.dt[1], base + j);
      a.ws.normed[base + j] = o * rs * load_scalar(a.lnw, a.dt[6], j) * silu(zz);
    }
  }
  if (tid == 0) a.ws.tickets[h] = 0u;
}

// ---------------------------------------------------------------------------
// Output projection (+ residual)
// ---------------------------------------------------------------------------
struct OutArgs {
  const void* w;
  const float* in;  // normed [T, V]
  const void* residual;
  int residual_dt;
  int T, V, Hout;
  float* update;
  float* residual_out;
};

template <bool BFW, int NJ>
__global__ __launch_bounds__(256) void deltanet_out_kernel(OutArgs a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r0 = blockIdx.x * kOutRows + wave * 2;
  const int nch = a.V >> 3;
  const bool ok[2] = {r0 < a.Hout, r0 + 1 < a.Hout};
  Raw8<BFW> wr[2][NJ];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int c = lane + kWave * j;
      if (c < nch && ok[r]) wr[r][j] = load_raw8_stream<BFW>(a.w, (size_t)(r0 + r) * a.V + (size_t)c * 8);
    }
  for (int t = 0; t < a.T; ++t) {
    float acc[2] = {0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int c = lane + kWave * j;
      if (c < nch) {
        float v8[8];
        load8_act(a.in, (size_t)t * a.V + (size_t)c * 8, v8);
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          float w8[8];
          raw8_to_f32<BFW>(wr[r][j], w8);
#pragma unroll
          for (int q = 0; q < 8; ++q) acc[r] = fmaf(w8[q], v8[q], acc[r]);
        }
      }
    }
    acc[0] = wave_sum(acc[0]);
    acc[1] = wave_sum(acc[1]);
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        if (!ok[r]) continue;
        const size_t o = (size_t)t * a.Hout + r0 + r;
        a.update[o] = acc[r];
        if (a.residual_out) a.residual_out[o] = load_scalar(a.residual, a.residual_dt, o) + acc[r];
      }
    }
  }
}

}  // namespace fk

using namespace fk;

extern "C" {

int fk_deltanet_project(const void* hidden, int hidden_dtype, const void* norm_weight, int norm_dtype,
                        const void* w_qkv, const void* w_z, const void* w_a, const void* w_b, int weight_dtype,
                        int tokens, int hidden_size, int qkv_rows, int z_rows, int ab_rows, float eps,
                        float norm_offset, float* mixed_qkv, float* z, float* a_logits, float* b_logits,
                        void* stream) {
  if (tokens < 1) return fail(FK_ERR_INVALID, "tokens must be positive");
  if (hidden_size < 8 || hidden_size % 8) return fail(FK_ERR_ALIGNMENT, "hidden_size must be a positive multiple of 8");
  if (hidden_size > 4096) return fail(FK_ERR_UNSUPPORTED, "hidden_size must be <= 4096");
  if (qkv_rows < 1 || z_rows < 1 || ab_rows < 1) return fail(FK_ERR_INVALID, "projection row counts must be positive");
  if (!is_float_dtype(hidden_dtype) || !is_float_dtype(norm_dtype) || !is_float_dtype(weight_dtype))
    return fail(FK_ERR_DTYPE, "projection inputs must be f32 or bf16");
  if (!hidden || !norm_weight || !w_qkv || !w_z || !w_a || !w_b || !mixed_qkv || !z || !a_logits || !b_logits)
    return fail(FK_ERR_INVALID, "projection pointers must be non-NULL");
  if (!aligned16(hidden) || !aligned16(w_qkv) || !aligned16(w_z) || !aligned16(w_a) || !aligned16(w_b))
    return fail(FK_ERR_ALIGNMENT, "hidden and projection weights must be 16-byte aligned");
  ProjArgs pa;
  pa.x = hidden;
  pa.nw = norm_weight;
  pa.nw_dt = norm_dtype;
  pa.w[0] = w_qkv;
  pa.w[1] = w_z;
  pa.w[2] = w_a;
  pa.w[3] = w_b;
  pa.out[0] = mixed_qkv;
  pa.out[1] = z;
  pa.out[2] = a_logits;
  pa.out[3] = b_logits;
  pa.rows[0] = qkv_rows;
  pa.rows[1] = z_rows;
  pa.rows[2] = ab_rows;
  pa.rows[3] = ab_rows;
  pa.T = tokens;
  pa.H = hidden_size;
  pa.eps = eps;
  pa.off = norm_offset;
  const int R = qkv_rows + z_rows + 2 * ab_rows;
  const int grid = (R + kProjRows - 1) / kProjRows;
  const bool bfw = weight_dtype == FK_DTYPE_BF16, bfx = hidden_dtype == FK_DTYPE_BF16, wide = hidden_size > 2048;
  hipStream_t s = as_stream(stream);
#define FK_PROJ(BW, BX)                                                                                   \
  if (wide) hipLaunchKernelGGL((deltanet_project_kernel<BW, BX, 8>), dim3(grid), dim3(256), 0, s, pa); \
  else hipLaunchKernelGGL((deltanet_project_kernel<BW, BX, 4>), dim3(grid), dim3(256), 0, s, pa);
  if (bfw && bfx) {
    FK_PROJ(true, true)
  } else if (bfw) {
    FK_PROJ(true, false)
  } else if (bfx) {
    FK_PROJ(false, true)
  } else {
    FK_PROJ(false, false)
  }
#undef FK_PROJ
  return check_launch("deltanet_project_kernel");
}

int fk_deltanet_conv(const void* mixed, int mixed_dtype, const void* conv_state, int state_dtype,
                     const void* conv_weight, int weight_dtype, int tokens, int channels, int kernel_size,
                     float* conv_out, void* next_state, void* stream) {
  if (tokens < 1) return fail(FK_ERR_INVALID, "tokens must be positive");
  if (channels < 1) return fail(FK_ERR_INVALID, "channels must be positive");
  if (kernel_size < 1 || kernel_size > 8) return fail(FK_ERR_UNSUPPORTED, "kernel_size must be in [1, 8]");
  if (!is_float_dtype(mixed_dtype) || !is_float_dtype(state_dtype) || !is_float_dtype(weight_dtype))
    return fail(FK_ERR_DTYPE, "conv inputs must be f32 or bf16");
  if (!mixed || !conv_state || !conv_weight || !conv_out || !next_state)
    return fail(FK_ERR_INVALID, "conv pointers must be non-NULL");
  ConvArgs ca;
  ca.mixed = mixed;
  ca.mixed_dt = mixed_dtype;
  ca.state = conv_state;
  ca.state_dt = state_dtype;
  ca.w = conv_weight;
  ca.w_dt = weight_dtype;
  ca.T = tokens;
  ca.C = channels;
  ca.KS = kernel_size;
  ca.out = conv_out;
  ca.next_state = next_state;
  hipLaunchKernelGGL(deltanet_conv_kernel, dim3((channels + 255) / 256), dim3(256), 0, as_stream(stream), ca);
  return check_launch("deltanet_conv_kernel");
}

size_t fk_deltanet_workspace_bytes(int tokens, int value_heads, int head_dim) {
  if (tokens < 1 || value_heads < 1 || head_dim < 1) return 0;
  DnWs ws;
  return dn_ws_layout(tokens, value_heads, head_dim, nullptr, &ws);
}

int fk_deltanet_recurrent_output(const void* mixed_qkv, const void* z, const void* a_logits, const void* b_logits,
                                 const void* recurrent_state, const void* out_proj_weight,
                                 const void* linear_norm_weight, const void* a_log, const void* dt_bias,
                                 const void* residual, const int32_t* tensor_dtypes, int tokens, int qk_heads,
                                 int value_heads, int head_dim, int hidden_size, float eps, float* update,
                                 void* next_state, float* residual_out, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  if (tokens < 1) return fail(FK_ERR_INVALID, "tokens must be positive");
  if (qk_heads < 1 || value_heads < 1 || value_heads % qk_heads)
    return fail(FK_ERR_INVALID, "value_heads must be a positive multiple of qk_heads");
  if (head_dim < 1 || head_dim > 128) return fail(FK_ERR_UNSUPPORTED, "head_dim must be in [1, 128]");
  if (hidden_size < 1) return fail(FK_ERR_INVALID, "hidden_size must be positive");
  const int V = value_heads * head_dim;
  if (V % 8) return fail(FK_ERR_ALIGNMENT, "value_heads * head_dim must be a multiple of 8");
  if (V > 4096) return fail(FK_ERR_UNSUPPORTED, "value_heads * head_dim must be <= 4096");
  if (!tensor_dtypes) return fail(FK_ERR_INVALID, "tensor_dtypes must be non-NULL");
  for (int i = 0; i < 10; ++i) {
    if (i == 9 && !residual) continue;
    if (!is_float_dtype(tensor_dtypes[i])) return fail(FK_ERR_DTYPE, "tensor_dtypes[%d] must be f32 or bf16", i);
  }
  if (!mixed_qkv || !z || !a_logits || !b_logits || !recurrent_state || !out_proj_weight || !linear_norm_weight ||
      !a_log || !dt_bias || !update || !next_state)
    return fail(FK_ERR_INVALID, "recurrent/output pointers must be non-NULL");
  if ((residual == nullptr) != (residual_out == nullptr))
    return fail(FK_ERR_INVALID, "residual and residual_out must both be set or both NULL");
  if (!aligned16(out_proj_weight)) return fail(FK_ERR_ALIGNMENT, "out_proj_weight must be 16-byte aligned");
  DnWs ws;
  const size_t need = dn_ws_layout(tokens, value_heads, head_dim, nullptr, &ws);
  if (!workspace || workspace_bytes < need)
    return fail(FK_ERR_WORKSPACE, "workspace has %zu bytes, need %zu", workspace ? workspace_bytes : 0, need);
  if (!aligned16(workspace)) return fail(FK_ERR_ALIGNMENT, "workspace must be 16-byte aligned");
  dn_ws_layout(tokens, value_heads, head_dim, reinterpret_cast<char*>(workspace), &ws);

  RecArgs ra;
  ra.mixed = mixed_qkv;
  ra.z = z;
  ra.a_in = a_logits;
  ra.b_in = b_logits;
  ra.state = recurrent_state;
  ra.lnw = linear_norm_weight;
  ra.a_log = a_log;
  ra.dt_bias = dt_bias;
  for (int i = 0; i < 10; ++i) ra.dt[i] = tensor_dtypes[i];
  ra.T = tokens;
  ra.Hk = qk_heads;
  ra.Hv = value_heads;
  ra.D = head_dim;
  ra.eps = eps;
  ra.next_state = next_state;
  ra.ws = ws;
  const int cb = head_dim < kRecCols ? head_dim : kRecCols;
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(deltanet_recurrent_kernel, dim3(value_heads, (head_dim + cb - 1) / cb), dim3(256), 0, s, ra);
  int st = check_launch("deltanet_recurrent_kernel");
  if (st) return st;

  OutArgs oa;
  oa.w = out_proj_weight;
  oa.in = ws.normed;
  oa.residual = residual;
  oa.residual_dt = residual ? tensor_dtypes[9] : FK_DTYPE_F32;
  oa.T = tokens;
  oa.V = V;
  oa.Hout = hidden_size;
  oa.update = update;
  oa.residual_out = residual_out;
  const int grid = (hidden_size + kOutRows - 1) / kOutRows;
  const bool bfw = tensor_dtypes[5] == FK_DTYPE_BF16;
  if (V > 2048) {
    if (bfw) hipLaunchKernelGGL((deltanet_out_kernel<true, 8>), dim3(grid), dim3(256), 0, s, oa);
    else hipLaunchKernelGGL((deltanet_out_kernel<false, 8>), dim3(grid), dim3(256), 0, s, oa);
  } else {
    if (bfw) hipLaunchKernelGGL((deltanet_out_kernel<true, 4>), dim3(grid), dim3(256), 0, s, oa);
    else hipLaunchKernelGGL((deltanet_out_kernel<false, 4>), dim3(grid), dim3(256), 0, s, oa);
  }
  return check_launch("deltanet_out_kernel");
}

}  // extern "C"
