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
  float* out[4];  // out[0] (raw mixed_qkv) may be NULL when the conv is fused
  int rows[4];
  int T, H;
  float eps, off;
  // Fused causal conv over the qkv rows (conv_out == NULL: not fused).
  const void* conv_state;
  int cs_dt;
  const void* conv_w;
  int cw_dt;
  int KS;
  float* conv_out;
  void* next_state;
};

constexpr int kProjMaxFusedTokens = 64;

template <bool BFW, bool BFX, int NJ>
__global__ __launch_bounds__(256) void deltanet_project_kernel(ProjArgs a) {
  __shared__ float s_proj[4][4][kProjMaxFusedTokens];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nch = a.H >> 3;
  const int R = a.rows[0] + a.rows[1] + a.rows[2] + a.rows[3];
  const int rbase = blockIdx.x * kProjRows + wave * 4;
  const size_t esz = BFW ? 2 : 4;
  const bool fuse_conv = a.conv_out != nullptr;

  const char* wp[4];
  float* op[4];
  int ostride[4], lrow[4], which[4];
  bool ok[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    int row = rbase + r;
    ok[r] = row < R;
    int wh = 0;
    if (ok[r]) {
      while (row >= a.rows[wh]) {
        row -= a.rows[wh];
        ++wh;
      }
    } else {
      row = 0;
    }
    which[r] = wh;
    lrow[r] = row;
    wp[r] = reinterpret_cast<const char*>(a.w[wh]) + (size_t)row * a.H * esz;
    op[r] = a.out[wh] ? a.out[wh] + row : nullptr;
    ostride[r] = a.rows[wh];
  }

  Raw8<BFW> wr[4][NJ];
  float nwv[NJ][8];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int c = lane + kWave * j;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (c < nch && ok[r]) wr[r][j] = load_raw8_stream<BFW>(wp[r], (size_t)c * 8);
    if (c < nch) {
      load8_any(a.nw, a.nw_dt, (size_t)c * 8, nwv[j]);
#pragma unroll
      for (int q = 0; q < 8; ++q) nwv[j][q] += a.off;
    } else {
#pragma unroll
      for (int q = 0; q < 8; ++q) nwv[j][q] = 0.f;
    }
  }

  constexpr int TB = 2;  // tokens per batch: independent x loads and reductions
  for (int t0 = 0; t0 < a.T; t0 += TB) {
    float ss[TB];
    float acc[TB][4];
#pragma unroll
    for (int tt = 0; tt < TB; ++tt) {
      ss[tt] = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[tt][r] = 0.f;
      const int t = t0 + tt;
      if (t < a.T) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const int c = lane + kWave * j;
          if (c < nch) {
            float x8[8], xn[8];
            load8_f32<BFX>(a.x, (size_t)t * a.H + (size_t)c * 8, x8);
#pragma unroll
            for (int q = 0; q < 8; ++q) {
              ss[tt] = fmaf(x8[q], x8[q], ss[tt]);
              xn[q] = x8[q] * nwv[j][q];
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              if (ok[r]) {
                float w8[8];
                raw8_to_f32<BFW>(wr[r][j], w8);
#pragma unroll
                for (int q = 0; q < 8; ++q) acc[tt][r] = fmaf(w8[q], xn[q], acc[tt][r]);
              }
            }
          }
        }
      }
    }
#pragma unroll
    for (int tt = 0; tt < TB; ++tt) {
      ss[tt] = wave_sum(ss[tt]);
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[tt][r] = wave_sum(acc[tt][r]);
    }
    if (lane == 0) {
#pragma unroll
      for (int tt = 0; tt < TB; ++tt) {
        const int t = t0 + tt;
        if (t >= a.T) continue;
        const float rs = rsqrtf(ss[tt] / (float)a.H + a.eps);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (!ok[r]) continue;
          const float v = acc[tt][r] * rs;
          if (op[r]) op[r][(size_t)t * ostride[r]] = v;
          if (fuse_conv) s_proj[wave][r][t] = v;
        }
      }
    }
  }

  if (fuse_conv) {
    __syncthreads();
    // Lanes 0..3: causal depthwise conv of channel lrow[r] over
    // [state | projections], SiLU, and the rolled state.
    if (lane < 4) {
      const int r = lane;
      int ch = 0, wh = 1;
      bool rok = false;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (q == r) {
          ch = lrow[q];
          wh = which[q];
          rok = ok[q];
        }
      if (rok && wh == 0) {
        const int C = a.rows[0];
        float win[8], wk[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          win[j] = j < a.KS ? load_scalar(a.conv_state, a.cs_dt, (size_t)ch * a.KS + j) : 0.f;
          wk[j] = j < a.KS ? load_scalar(a.conv_w, a.cw_dt, (size_t)ch * a.KS + j) : 0.f;
        }
        for (int t = 0; t < a.T; ++t) {
          const float v = s_proj[wave][r][t];
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
          a.conv_out[(size_t)t * C + ch] = silu(acc);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (j < a.KS) store_scalar(a.next_state, a.cs_dt, (size_t)ch * a.KS + j, win[j]);
      }
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

constexpr int kRecChunk = 16;  // tokens whose inputs are staged in LDS at once

// Workgroup (head h, column block): thread (col, rg) owns S[rg*RPT .. +RPT, col]
// of the head's fp32 state in registers.  Each chunk of up to 16 tokens
// first stages q, k (the head's qk head), v (this block's columns) and the
// per-token scalars (decay, beta, q/k l2 scales) in LDS in parallel; the
// sequential state update then reads only LDS and needs two barriers per
// token (double-buffered partial sums).
__global__ __launch_bounds__(256) void deltanet_recurrent_kernel(RecArgs a) {
  __shared__ float s_q[kRecChunk][128];
  __shared__ float s_k[kRecChunk][128];
  __shared__ float s_v[kRecChunk][kRecCols];
  __shared__ float s_sc[kRecChunk][4];  // decay, beta, q scale, k scale
  __shared__ float s_red[2][256];
  __shared__ float s_red2[2][256];
  __shared__ int s_last;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = blockIdx.x;
  const int CB = a.D < kRecCols ? a.D : kRecCols;
  const int RG = 256 / CB;              // row groups
  const int RPT = (a.D + RG - 1) / RG;  // rows per thread (<= 16)
  const int col = tid % CB, rg = tid / CB;
  const int c0 = blockIdx.y * CB;
  const int c = c0 + col;
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
  const float neg_a = -expf(load_scalar(a.a_log, a.dt[7], h));
  const float dt_bias = load_scalar(a.dt_bias, a.dt[8], h);

  for (int tc = 0; tc < a.T; tc += kRecChunk) {
    const int nt = min(kRecChunk, a.T - tc);
    // Stage the chunk's inputs.
    for (int idx = tid; idx < nt * a.D; idx += 256) {
      const int tt = idx / a.D, i = idx - tt * a.D;
      const size_t mrow = (size_t)(tc + tt) * mixed_w;
      s_q[tt][i] = load_scalar(a.mixed, a.dt[0], mrow + (size_t)qk_head * a.D + i);
      s_k[tt][i] = load_scalar(a.mixed, a.dt[0], mrow + (size_t)a.Hk * a.D + (size_t)qk_head * a.D + i);
    }
    for (int idx = tid; idx < nt * CB; idx += 256) {
      const int tt = idx / CB, j = idx - tt * CB;
      const int cc = c0 + j;
      s_v[tt][j] = cc < a.D ? load_scalar(a.mixed, a.dt[0], (size_t)(tc + tt) * mixed_w + (size_t)2 * a.Hk * a.D +
                                                                 (size_t)h * a.D + cc)
                            : 0.f;
    }
    __syncthreads();
    for (int tt = wave; tt < nt; tt += 4) {
      float sq = 0.f, sk = 0.f;
      for (int i = lane; i < a.D; i += kWave) {
        sq = fmaf(s_q[tt][i], s_q[tt][i], sq);
        sk = fmaf(s_k[tt][i], s_k[tt][i], sk);
      }
      sq = wave_sum(sq);
      sk = wave_sum(sk);
      if (lane == 0) {
        const int t = tc + tt;
        const float gin = load_scalar(a.a_in, a.dt[2], (size_t)t * a.Hv + h) + dt_bias;
        s_sc[tt][0] = expf(neg_a * softplus_stable(gin));
        s_sc[tt][1] = 1.f / (1.f + expf(-load_scalar(a.b_in, a.dt[3], (size_t)t * a.Hv + h)));
        s_sc[tt][2] = rsqrtf(sq + a.eps) * rsqrtf((float)a.D);
        s_sc[tt][3] = rsqrtf(sk + a.eps);
      }
    }
    __syncthreads();

    for (int tt = 0; tt < nt; ++tt) {
      const int buf = tt & 1;
      const float decay = s_sc[tt][0], beta = s_sc[tt][1], qs = s_sc[tt][2], ks = s_sc[tt][3];
      float kv[kRecMaxRows], qv[kRecMaxRows];
      float part = 0.f;
#pragma unroll
      for (int k = 0; k < kRecMaxRows; ++k) {
        const int i = rg * RPT + k;
        const bool ok = col_ok && k < RPT && i < a.D;
        kv[k] = ok ? s_k[tt][i] * ks : 0.f;
        qv[k] = ok ? s_q[tt][i] * qs : 0.f;
        S[k] *= decay;
        part = fmaf(S[k], kv[k], part);
      }
      s_red[buf][tid] = part;
      __syncthreads();
      float proj = 0.f;
      for (int g = 0; g < RG; ++g) proj += s_red[buf][g * CB + col];
      const float delta = (s_v[tt][col] - proj) * beta;
      float opart = 0.f;
#pragma unroll
      for (int k = 0; k < kRecMaxRows; ++k) {
        S[k] = fmaf(kv[k], delta, S[k]);
        opart = fmaf(S[k], qv[k], opart);
      }
      s_red2[buf][tid] = opart;
      __syncthreads();
      if (rg == 0 && c < a.D) {
        float o = 0.f;
        for (int g = 0; g < RG; ++g) o += s_red2[buf][g * CB + col];
        store_coherent(a.ws.core + (size_t)(tc + tt) * a.Hv * a.D + (size_t)h * a.D + c, o);
      }
    }
    __syncthreads();  // the next chunk overwrites the staged inputs
  }

#pragma unroll
  for (int k = 0; k < kRecMaxRows; ++k) {
    const int i = rg * RPT + k;
    if (col_ok && k < RPT && i < a.D) store_scalar(a.next_state, a.dt[4], sbase + (size_t)i * a.D + c, S[k]);
  }

  // The last column block of head h applies the gated RMSNorm for the head
  // (core values were published with coherent stores; no L2-wide fence).
  publish_wait();
  __syncthreads();
  if (tid == 0) s_last = ticket_add(&a.ws.tickets[h]) == gridDim.y - 1;
  __syncthreads();
  if (!s_last) return;
  for (int t = wave; t < a.T; t += 4) {
    const size_t base = (size_t)t * a.Hv * a.D + (size_t)h * a.D;
    float ss = 0.f;
    for (int j = lane; j < a.D; j += kWave) {
      const float o = load_coherent(a.ws.core + base + j);
      ss = fmaf(o, o, ss);
    }
    ss = wave_sum(ss);
    const float rs = rsqrtf(ss / (float)a.D + a.eps);
    for (int j = lane; j < a.D; j += kWave) {
      const float o = load_coherent(a.ws.core + base + j);
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
  constexpr int TB = 2;  // tokens per batch: independent input loads and reductions
  for (int t0 = 0; t0 < a.T; t0 += TB) {
    float acc[TB][2];
#pragma unroll
    for (int tt = 0; tt < TB; ++tt) {
      acc[tt][0] = 0.f;
      acc[tt][1] = 0.f;
      if (t0 + tt >= a.T) continue;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int c = lane + kWave * j;
        if (c < nch) {
          float v8[8];
          load8_act(a.in, (size_t)(t0 + tt) * a.V + (size_t)c * 8, v8);
#pragma unroll
          for (int r = 0; r < 2; ++r) {
            float w8[8];
            raw8_to_f32<BFW>(wr[r][j], w8);
#pragma unroll
            for (int q = 0; q < 8; ++q) acc[tt][r] = fmaf(w8[q], v8[q], acc[tt][r]);
          }
        }
      }
    }
#pragma unroll
    for (int tt = 0; tt < TB; ++tt) {
      acc[tt][0] = wave_sum(acc[tt][0]);
      acc[tt][1] = wave_sum(acc[tt][1]);
    }
    if (lane == 0) {
#pragma unroll
      for (int tt = 0; tt < TB; ++tt) {
        const int t = t0 + tt;
        if (t >= a.T) continue;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          if (!ok[r]) continue;
          const size_t o = (size_t)t * a.Hout + r0 + r;
          a.update[o] = acc[tt][r];
          if (a.residual_out) a.residual_out[o] = load_scalar(a.residual, a.residual_dt, o) + acc[tt][r];
        }
      }
    }
  }
}


// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
static int launch_project(const ProjArgs& pa, int weight_dtype, int hidden_dtype, hipStream_t s) {
  const int R = pa.rows[0] + pa.rows[1] + pa.rows[2] + pa.rows[3];
  const int grid = (R + kProjRows - 1) / kProjRows;
  const bool bfw = weight_dtype == FK_DTYPE_BF16, bfx = hidden_dtype == FK_DTYPE_BF16, wide = pa.H > 2048;
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

static int check_project_args(const void* hidden, int hidden_dtype, const void* norm_weight, int norm_dtype,
                              const void* w_qkv, const void* w_z, const void* w_a, const void* w_b,
                              int weight_dtype, int tokens, int hidden_size) {
  if (tokens < 1) return fail(FK_ERR_INVALID, "tokens must be positive");
  if (hidden_size < 8 || hidden_size % 8) return fail(FK_ERR_ALIGNMENT, "hidden_size must be a positive multiple of 8");
  if (hidden_size > 4096) return fail(FK_ERR_UNSUPPORTED, "hidden_size must be <= 4096");
  if (!is_float_dtype(hidden_dtype) || !is_float_dtype(norm_dtype) || !is_float_dtype(weight_dtype))
    return fail(FK_ERR_DTYPE, "projection inputs must be f32 or bf16");
  if (!hidden || !norm_weight || !w_qkv || !w_z || !w_a || !w_b)
    return fail(FK_ERR_INVALID, "projection pointers must be non-NULL");
  if (!aligned16(hidden) || !aligned16(norm_weight) || !aligned16(w_qkv) || !aligned16(w_z) || !aligned16(w_a) ||
      !aligned16(w_b))
    return fail(FK_ERR_ALIGNMENT, "hidden, norm_weight and projection weights must be 16-byte aligned");
  return FK_OK;
}

static int check_recurrent_shape(int tokens, int qk_heads, int value_heads, int head_dim, int hidden_size) {
  if (tokens < 1) return fail(FK_ERR_INVALID, "tokens must be positive");
  if (qk_heads < 1 || value_heads < 1 || value_heads % qk_heads)
    return fail(FK_ERR_INVALID, "value_heads must be a positive multiple of qk_heads");
  if (head_dim < 1 || head_dim > 128) return fail(FK_ERR_UNSUPPORTED, "head_dim must be in [1, 128]");
  if (hidden_size < 1) return fail(FK_ERR_INVALID, "hidden_size must be positive");
  const int V = value_heads * head_dim;
  if (V % 8) return fail(FK_ERR_ALIGNMENT, "value_heads * head_dim must be a multiple of 8");
  if (V > 4096) return fail(FK_ERR_UNSUPPORTED, "value_heads * head_dim must be <= 4096");
  return FK_OK;
}

static int launch_recurrent_output(const RecArgs& ra, const void* out_proj_weight, int out_dt,
                                   const void* residual, int residual_dt, int hidden_size, float* update,
                                   float* residual_out, hipStream_t s) {
  const int cb = ra.D < kRecCols ? ra.D : kRecCols;
  hipLaunchKernelGGL(deltanet_recurrent_kernel, dim3(ra.Hv, (ra.D + cb - 1) / cb), dim3(256), 0, s, ra);
  int st = check_launch("deltanet_recurrent_kernel");
  if (st) return st;
  OutArgs oa;
  oa.w = out_proj_weight;
  oa.in = ra.ws.normed;
  oa.residual = residual;
  oa.residual_dt = residual_dt;
  oa.T = ra.T;
  oa.V = ra.Hv * ra.D;
  oa.Hout = hidden_size;
  oa.update = update;
  oa.residual_out = residual_out;
  const int grid = (hidden_size + kOutRows - 1) / kOutRows;
  const bool bfw = out_dt == FK_DTYPE_BF16;
  if (oa.V > 2048) {
    if (bfw) hipLaunchKernelGGL((deltanet_out_kernel<true, 8>), dim3(grid), dim3(256), 0, s, oa);
    else hipLaunchKernelGGL((deltanet_out_kernel<false, 8>), dim3(grid), dim3(256), 0, s, oa);
  } else {
    if (bfw) hipLaunchKernelGGL((deltanet_out_kernel<true, 4>), dim3(grid), dim3(256), 0, s, oa);
    else hipLaunchKernelGGL((deltanet_out_kernel<false, 4>), dim3(grid), dim3(256), 0, s, oa);
  }
  return check_launch("deltanet_out_kernel");
}

// Step workspace: the recurrent/output workspace followed by the fused
// projection outputs (conv'd mixed qkv, z, a, b) of every token.
struct StepWs {
  DnWs dn;
  float* mixed;
  float* z;
  float* a;
  float* b;
};

static size_t step_ws_layout(int T, int Hk, int Hv, int D, char* base, StepWs* ws) {
  size_t off = align_up(dn_ws_layout(T, Hv, D, base, &ws->dn), 256);
  auto take = [&](size_t bytes) {
    size_t at = off;
    off = align_up(off + bytes, 256);
    return base ? reinterpret_cast<float*>(base + at) : nullptr;
  };
  ws->mixed = take((size_t)T * (2 * Hk + Hv) * D * 4);
  ws->z = take((size_t)T * Hv * D * 4);
  ws->a = take((size_t)T * Hv * 4);
  ws->b = take((size_t)T * Hv * 4);
  return off;
}

}  // namespace fk

using namespace fk;

extern "C" {

int fk_deltanet_project(const void* hidden, int hidden_dtype, const void* norm_weight, int norm_dtype,
                        const void* w_qkv, const void* w_z, const void* w_a, const void* w_b, int weight_dtype,
                        int tokens, int hidden_size, int qkv_rows, int z_rows, int ab_rows, float eps,
                        float norm_offset, float* mixed_qkv, float* z, float* a_logits, float* b_logits,
                        void* stream) {
  int st = check_project_args(hidden, hidden_dtype, norm_weight, norm_dtype, w_qkv, w_z, w_a, w_b, weight_dtype,
                              tokens, hidden_size);
  if (st) return st;
  if (qkv_rows < 1 || z_rows < 1 || ab_rows < 1) return fail(FK_ERR_INVALID, "projection row counts must be positive");
  if (!mixed_qkv || !z || !a_logits || !b_logits) return fail(FK_ERR_INVALID, "projection outputs must be non-NULL");
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
  pa.conv_state = nullptr;
  pa.cs_dt = FK_DTYPE_F32;
  pa.conv_w = nullptr;
  pa.cw_dt = FK_DTYPE_F32;
  pa.KS = 0;
  pa.conv_out = nullptr;
  pa.next_state = nullptr;
  return launch_project(pa, weight_dtype, hidden_dtype, as_stream(stream));
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
  int st = check_recurrent_shape(tokens, qk_heads, value_heads, head_dim, hidden_size);
  if (st) return st;
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
  return launch_recurrent_output(ra, out_proj_weight, tensor_dtypes[5], residual,
                                 residual ? tensor_dtypes[9] : FK_DTYPE_F32, hidden_size, update, residual_out,
                                 as_stream(stream));
}

size_t fk_deltanet_step_workspace_bytes(int tokens, int qk_heads, int value_heads, int head_dim) {
  if (tokens < 1 || qk_heads < 1 || value_heads < 1 || head_dim < 1) return 0;
  StepWs ws;
  return step_ws_layout(tokens, qk_heads, value_heads, head_dim, nullptr, &ws);
}

int fk_deltanet_step(const void* hidden, const void* input_norm_weight, const void* w_qkv, const void* w_z,
                     const void* w_a, const void* w_b, const void* conv_state, const void* conv_weight,
                     const void* recurrent_state, const void* out_proj_weight, const void* linear_norm_weight,
                     const void* a_log, const void* dt_bias, const int32_t* dtypes, int tokens, int hidden_size,
                     int qk_heads, int value_heads, int head_dim, int kernel_size, float eps, float* update,
                     float* hidden_out, void* next_conv_state, void* next_recurrent_state, void* workspace,
                     size_t workspace_bytes, void* stream) {
  if (!dtypes) return fail(FK_ERR_INVALID, "dtypes must be non-NULL");
  for (int i = 0; i < 10; ++i)
    if (!is_float_dtype(dtypes[i])) return fail(FK_ERR_DTYPE, "dtypes[%d] must be f32 or bf16", i);
  int st = check_project_args(hidden, dtypes[0], input_norm_weight, dtypes[1], w_qkv, w_z, w_a, w_b, dtypes[2],
                              tokens, hidden_size);
  if (st) return st;
  st = check_recurrent_shape(tokens, qk_heads, value_heads, head_dim, hidden_size);
  if (st) return st;
  if (tokens > kProjMaxFusedTokens) return fail(FK_ERR_UNSUPPORTED, "fused DeltaNet step supports tokens <= %d", kProjMaxFusedTokens);
  if (kernel_size < 1 || kernel_size > 8) return fail(FK_ERR_UNSUPPORTED, "kernel_size must be in [1, 8]");
  if (!conv_state || !conv_weight || !recurrent_state || !out_proj_weight || !linear_norm_weight || !a_log ||
      !dt_bias || !update || !next_conv_state || !next_recurrent_state)
    return fail(FK_ERR_INVALID, "DeltaNet step pointers must be non-NULL");
  if (!aligned16(out_proj_weight)) return fail(FK_ERR_ALIGNMENT, "out_proj_weight must be 16-byte aligned");
  StepWs ws;
  const size_t need = step_ws_layout(tokens, qk_heads, value_heads, head_dim, nullptr, &ws);
  if (!workspace || workspace_bytes < need)
    return fail(FK_ERR_WORKSPACE, "workspace has %zu bytes, need %zu", workspace ? workspace_bytes : 0, need);
  if (!aligned16(workspace)) return fail(FK_ERR_ALIGNMENT, "workspace must be 16-byte aligned");
  step_ws_layout(tokens, qk_heads, value_heads, head_dim, reinterpret_cast<char*>(workspace), &ws);
  hipStream_t s = as_stream(stream);

  const int conv_dim = (2 * qk_heads + value_heads) * head_dim;
  ProjArgs pa;
  pa.x = hidden;
  pa.nw = input_norm_weight;
  pa.nw_dt = dtypes[1];
  pa.w[0] = w_qkv;
  pa.w[1] = w_z;
  pa.w[2] = w_a;
  pa.w[3] = w_b;
  pa.out[0] = nullptr;  // only the conv'd values are needed
  pa.out[1] = ws.z;
  pa.out[2] = ws.a;
  pa.out[3] = ws.b;
  pa.rows[0] = conv_dim;
  pa.rows[1] = value_heads * head_dim;
  pa.rows[2] = value_heads;
  pa.rows[3] = value_heads;
  pa.T = tokens;
  pa.H = hidden_size;
  pa.eps = eps;
  pa.off = 1.0f;
  pa.conv_state = conv_state;
  pa.cs_dt = dtypes[3];
  pa.conv_w = conv_weight;
  pa.cw_dt = dtypes[4];
  pa.KS = kernel_size;
  pa.conv_out = ws.mixed;
  pa.next_state = next_conv_state;
  st = launch_project(pa, dtypes[2], dtypes[0], s);
  if (st) return st;

  RecArgs ra;
  ra.mixed = ws.mixed;
  ra.z = ws.z;
  ra.a_in = ws.a;
  ra.b_in = ws.b;
  ra.state = recurrent_state;
  ra.lnw = linear_norm_weight;
  ra.a_log = a_log;
  ra.dt_bias = dt_bias;
  const int rec_dt[10] = {FK_DTYPE_F32, FK_DTYPE_F32, FK_DTYPE_F32, FK_DTYPE_F32, dtypes[5],
                          dtypes[6],    dtypes[7],    dtypes[8],    dtypes[9],    dtypes[0]};
  for (int i = 0; i < 10; ++i) ra.dt[i] = rec_dt[i];
  ra.T = tokens;
  ra.Hk = qk_heads;
  ra.Hv = value_heads;
  ra.D = head_dim;
  ra.eps = eps;
  ra.next_state = next_recurrent_state;
  ra.ws = ws.dn;
  return launch_recurrent_output(ra, out_proj_weight, dtypes[6], hidden_out ? hidden : nullptr, dtypes[0],
                                 hidden_size, update, hidden_out, s);
}

}  // extern "C"
