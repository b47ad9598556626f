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
    const void* wbase = wh == 0 ? a.w[0] : wh == 1 ? a.w[1] : wh == 2 ? a.w[2] : a.w[3];  // no indexed kernarg load
    wp[r] = reinterpret_cast<const char*>(wbase) + (size_t)row * a.H * esz;
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
// Single-launch DeltaNet step (fk_deltanet_step for T <= 8, D = 128, bf16
// weights).  One 512-thread workgroup per CU, grid capped at co-resident
// capacity, phases joined by launch-tagged words (the MoE layer's protocol:
// value + 32-bit launch tag per 8-byte word, polled by consumers; the epoch
// advances once every workgroup's started record carries the tag):
//   A  projections: workgroup b owns row tiles b, b + G, b + 2G (16 rows of
//      the concatenated [qkv | z] weights).  T <= 2: whole-row dot products
//      on the VALU; T > 2: its 8 wavefronts split K and run
//      v_mfma_f32_16x16x32_bf16 with the normalised tokens as bf16 hi + lo
//      columns (2 per token, so the fp32 activations keep ~16 mantissa
//      bits), partial tiles summed through LDS.  The owner of a qkv row
//      applies the causal conv + SiLU over the tokens and rolls the conv
//      state.  Outputs leave tagged.  A head workgroup (below) also computes
//      its head's a and b logits from its own staged tokens.
//   B  four workgroups per value head, a quarter of its value columns each:
//      the fp32 state (prefetched into registers: thread (column jl, group
//      g) holds rows 8g .. 8g + 7 of its column, the column sums reduce over
//      16 lanes with DPP) runs the gated delta rule over the tokens; the
//      gated values o * w * silu(z) and the quarter's sum of squares of o
//      leave tagged.
//   C1 unit (rb, ks): rows 128 rb .. + 128 of W_out restricted to the
//      columns of a few heads (fetched into registers after phase A); it
//      applies each head's RMSNorm scale (from the four quarter sums) while
//      staging the gated values as hi + lo columns, runs the MFMAs and
//      leaves partial sums tagged.
//   C2 workgroup b < H / 16 sums the partials of rows 16b .. 16b + 15:
//      update (and hidden_out = x + update).
// ---------------------------------------------------------------------------
constexpr int kStepMaxTokens = 8;
constexpr int kStepWaves = 8;
constexpr int kStepMaxGrid = 1024;
constexpr int kStepTilesPerWG = 3;  // phase A row tiles per workgroup (host checks)
constexpr int kStepD = 128;
constexpr size_t kStepMixWords = (size_t)kStepMaxTokens * 8192;
constexpr size_t kStepVWords = (size_t)kStepMaxTokens * 4096;
constexpr size_t kStepPartWords = (size_t)8 * kStepMaxTokens * 2048;  // [V/512 <= 8][T][H <= 2048]
constexpr int kStepHeadWGs = 4;  // workgroups per value head (value columns split four ways)
constexpr int kStepQCols = kStepD / kStepHeadWGs;  // value columns per head workgroup
constexpr int kStepInPitch = 2 * kStepD + 2 * kStepQCols + 4;  // head workgroup inputs per token (q, k, v, z, a, b, pad)
constexpr int kStepHssPitch = 64 * kStepHeadWGs;  // (head, quarter) words per token
constexpr int kStepStPitch = kStepD + 4;  // LDS pitch of a state column in phase B (floats)
constexpr int kStepTilesAhead = 2;  // phase A weight tiles in flight per wavefront
constexpr int kStepTicketEpoch = kWorkspaceEpochWord;
constexpr int kStepTicketError = kWorkspaceErrorWord;


struct StepTagWs {
  uint32_t* tickets;  // [16] workspace header: epoch, poll bound, error flag (fk_host.h)
  uint64_t* mix;      // [T, C] conv'd qkv
  uint64_t* z;        // [T, V]
  uint64_t* norm;     // [T, V] gated values o * w * silu(z), before the RMSNorm scale
  uint64_t* started;  // [grid]
  uint64_t* hss;        // [kStepMaxTokens][kStepHssPitch] head quarters' sums of squares
  uint64_t* part;       // [V / 512][T][H] phase C partial sums
};

struct StepArgs {
  const void* x;
  const void* nw;
  const void* w[4];  // qkv, z, a, b (bf16, rows of H)
  const void* conv_state;
  const void* conv_w;
  const void* rec_state;
  const void* w_out;  // bf16 [H, V]
  const void* lnw;
  const void* a_log;
  const void* dt_bias;
  int T, H, Hk, Hv, C, V, R, KS;
  float eps;
  float* update;
  float* hidden_out;
  void* next_conv;
  void* next_rec;
  StepTagWs tw;
};

// Slot of column n of chunk c in an MFMA B-operand staging area
// [chunks][ncp][8 bf16] (ncp a power of two >= the columns in use).  The
// column is XOR-swizzled by the chunk: a wavefront writing one column of 64
// consecutive chunks then spreads over all LDS banks (without it the
// 16 * ncp-byte chunk stride puts every lane on the same banks), and the 16
// columns of one chunk that an MFMA operand read takes stay a permutation of
// the chunk's slots.
__device__ __forceinline__ int bcol_slot(int c, int n, int ncp) { return c * ncp + (n ^ (c & (ncp - 1))); }

// Sum over the 16 lanes of a DPP row (every lane of the row gets it).
__device__ __forceinline__ float row16_sum(float v) {
  v += __uint_as_float(dpp_u32<kDppQuadXor1>(__float_as_uint(v)));
  v += __uint_as_float(dpp_u32<kDppQuadXor2>(__float_as_uint(v)));
  v += __uint_as_float(dpp_u32<kDppRowHalfMirror>(__float_as_uint(v)));
  v += __uint_as_float(dpp_u32<kDppRowMirror>(__float_as_uint(v)));
  return v;
}

// NT: compile-time bound on the tokens (2 or 8), which sizes the token
// registers; NT = 2 also takes the VALU projections (H = 2048 only).  BFX: hidden states in bf16 (else fp32).  Every other operand
// has the dtype of the model's own decode: bf16 weights, norm weights, conv
// state and decay parameters, fp32 recurrent state (the host sends other
// combinations to the staged kernels).
FK_TIMELINE_BUFFER(deltanet_step)

template <bool BFX, int NT>
__global__ __launch_bounds__(512) void deltanet_step_kernel(StepArgs a) {
  FK_TIMELINE_DECL;
  FK_MARK(0);  // (timeline markers: diagnostic builds only)
  // T <= 2 (and H = 2048, which the host checks): phase A on the VALU.
  constexpr bool VALU_A = NT <= 2;
  extern __shared__ float4 s_dyn_v[];
  char* s_dyn = reinterpret_cast<char*>(s_dyn_v);
  __shared__ float s_rs[kStepMaxTokens];
  __shared__ float s_part[kStepMaxTokens][kStepWaves];  // [token][wavefront of that token]
  __shared__ float s_sc[kStepMaxTokens][2];  // decay, beta (head workgroups)
  __shared__ uint32_t s_hdr[3];  // the workspace header words wavefront 0 loaded
  __shared__ int s_fail;
  __shared__ float s_abp[kStepMaxTokens][kStepWaves][2];  // head workgroups: a and b logit parts [token][wavefront]
  // (the wavefront index is uniform: kept in a scalar register, so that
  // addresses derived from it stay scalar too)
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = gridDim.x, b = blockIdx.x;
  const int T = a.T, H = VALU_A ? 2048 : a.H, C = a.C, V = a.V, R = a.R, Hv = a.Hv;
  const int NC = 2 * T;  // MFMA columns in use: (hi, lo) per token
  const int NCP = NC <= 2 ? 2 : NC <= 4 ? 4 : NC <= 8 ? 8 : 16;  // staging columns (power of two)
  // The workspace header (epoch, poll bound, error word) is loaded by
  // wavefront 0 alone and shared through LDS at the staging barrier: the
  // words are read past the caches (coherent loads), and the same lines
  // read by every wavefront of the grid at once queue behind each other
  // (T = 8 25.3 -> 24.8 us, T = 1 20.1 -> 20.0 us).  Every wavefront has the
  // epoch once the barrier is passed, before the started record is stored.
  WaitHeader hdr{0u, 0u, 0u};
  if (wave == 0) hdr = load_wait_header(a.tw.tickets, kStepTicketEpoch);
  const int n = lane & 15, g4 = lane >> 4;  // MFMA lane -> (column / A row, k group)

  // Roles.  Each value head runs on kStepHeadWGs workgroups at the end of
  // the grid (a quarter of the head's value columns each); the phase C
  // units and the output rows sit on the first workgroups.
  const int qb = b - (G - kStepHeadWGs * Hv);
  const bool is_head = qb >= 0;
  const int head = is_head ? qb / kStepHeadWGs : 0, quarter = is_head ? qb % kStepHeadWGs : 0;
  const bool is_out = b < H / 16;

  // The token chunks and the norm weight are loaded before any weight load
  // is issued: behind the 50 MB weight stream of every workgroup, their few
  // lines would come back with the last weight tile.
  constexpr int XCH = NT * 2048 / 8 / 512;  // token chunks per thread at H <= 2048
  // H and V are powers of two (the host checks): indices split by shifts.
  const int lh = 31 - __builtin_clz((unsigned)H);
  const int cpt_sh = lh - 3;  // 8-element chunks per token row: H / 8
  const int cpt = H >> 3, nchunk = T * cpt;
  Raw8<BFX> xr[XCH];
  Raw8<true> nr[XCH];
#pragma unroll
  for (int q = 0; q < XCH; ++q) {
    const int idx8 = tid + q * 512;
    if (idx8 < nchunk) {
      xr[q] = load_raw8<BFX>(a.x, (size_t)idx8 * 8);
      nr[q] = load_raw8<true>(a.nw, (size_t)(idx8 & (cpt - 1)) * 8);
    }
  }
  // The a and b rows of a head workgroup's own head: each head computes its
  // a and b logits while it stages the tokens (below), so that no head waits
  // for other workgroups' a/b projections.  Thread tid takes chunk
  // tid % (H / 8) of both rows (for every token it stages); every workgroup
  // issues the loads, the others on the head-0 rows, unused: no branch
  // around a load.
  Raw8<true> war, wbr;
  {
    const size_t o = ((size_t)head * H + (size_t)((tid & ((H >> 3) - 1)) << 3));
    war = load_raw8<true>(a.w[2], o);
    wbr = load_raw8<true>(a.w[3], o);
  }
  // Small operands of phase B, fetched with the tokens, ahead of the weight
  // tiles: the head's norm weight and decay parameters, and (head
  // workgroups) the head quarter's state, [128 rows][32 columns] fp32, for
  // the recurrence's layout (thread (jl, g): rows 8g .. 8g + 7 of value
  // column jcol = quarter * 32 + jl).  T > 2 (MFMA path): read coalesced,
  // thread tid loading columns 4 (tid % 8) .. + 3 of rows tid / 8 and
  // tid / 8 + 64 (two 16-byte loads, eight threads per 128-byte row), and
  // handed over through LDS in phase B.  T <= 2: gathered in the layout
  // directly, one float per row (1,024 line requests per workgroup instead
  // of 128).  The coalesced read lets the head workgroups finish issuing
  // their first tile ~1 us sooner, which at T = 8 brings the heads' inputs
  // 1.5 us earlier (24.6 -> 23.2 us); at T = 1 the heads are not on the
  // critical path but the W_out blocks of the other workgroups are, and
  // the head workgroups' faster start took HBM share from those workgroups'
  // projection tiles, so their W_out blocks came later (19.3 -> 19.9 us).
  // Issued after the staging instead, these loads sat between the tiles'
  // loads, and the waits for the tiles (counted over both paths) waited for
  // them too.
  uint32_t lnw1[1], alog[1], dtb1[1];
  gather_raw<true>(a.lnw, quarter * kStepQCols + (lane & (kStepQCols - 1)), 0, 1, lnw1);
  gather_raw<true>(a.a_log, is_head ? head : 0, 0, 1, alog);
  gather_raw<true>(a.dt_bias, is_head ? head : 0, 0, 1, dtb1);
  const int sjl = tid >> 4, sgr = tid & 15, jcol = quarter * kStepQCols + sjl;
  u32x4 S_ld[2];       // T > 2
  uint32_t S_raw[8];   // T <= 2
  if (is_head) {
    if constexpr (VALU_A) {
      gather_raw<false>(a.rec_state, ((size_t)head * kStepD + (size_t)sgr * 8) * kStepD + jcol, kStepD, 8, S_raw);
    } else {
#pragma unroll
      for (int j = 0; j < 2; ++j)
        S_ld[j] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const float*>(a.rec_state) +
                                                  ((size_t)head * kStepD + (size_t)(tid >> 3) + 64 * j) * kStepD +
                                                  quarter * kStepQCols + (tid & 7) * 4);
    }
  }
  // (kept ahead of the weight tiles: the scheduler would otherwise sink the
  // a/b and state loads towards their use, behind the tiles, and the waits
  // for them would then wait for the tiles too)
  __builtin_amdgcn_sched_barrier(0);
  FK_MARK(10);

  // The first weight tile is issued right behind the token chunks: the
  // staging below waits for the chunks only (loads retire in order), so the
  // weight stream runs while the tokens are normalised and staged.
  // Conv taps (state and weights) of this workgroup's qkv rows, needed by
  // the first tile's epilogue on the VALU path, so issued before the tiles.
  uint32_t cwin_raw[8], cwk_raw[8];
  {
    // MFMA path: thread (tile, row, token) of the epilogue below; VALU path:
    // lane 2i + rr < 8 of wavefront w, row 2w + rr of tile i.
    const int row = VALU_A ? (b + ((lane >> 1) & 3) * G) * 16 + 2 * wave + (lane & 1)
                           : (b + (tid >> 7) * G) * 16 + ((tid >> 3) & 15);
    const bool conv_row = row < C;
    const int nk = conv_row ? a.KS : 0;
    gather_raw<true>(a.conv_state, (size_t)(conv_row ? row : 0) * a.KS, 1, nk, cwin_raw);
    gather_raw<true>(a.conv_w, (size_t)(conv_row ? row : 0) * a.KS, 1, nk, cwk_raw);
  }

  // ---- phase A weight tiles ----------------------------------------------
  // Loads are issued in the order their data is consumed (the vector memory
  // counter retires in order): the phase A weight tiles, then the operands
  // of the later phases.
  const int ntiles = (R + 15) / 16;
  const int kw = H >> 3;  // K range of one wavefront's MFMAs (H / 8 waves)
  const int ks = kw >> 5;  // MFMA steps per tile (H <= 2048: <= 8); also load slots per tile
  // Whole-row loads: wavefront w reads rows 2w and 2w + 1 of each tile, one
  // 1 KiB piece of a row per instruction (slot s: row 2w + s / LPR, piece
  // s % LPR, LPR = H / 512 pieces per row).  Reading the wavefront's MFMA K
  // range of all 16 rows instead streams at 4.0 TB/s against 5.0 TB/s for
  // whole rows on this part.  The rows meet in the workgroup's LDS tile.
  const int lpr_sh = lh - 9;  // log2 of the 1 KiB pieces per row
  const int LPR = 1 << lpr_sh;
  int ntl = 0;
  u32x4 av[kStepTilesPerWG][8];
#pragma unroll
  for (int i = 0; i < kStepTilesPerWG; ++i)
    if (b + i * G < ntiles) ntl = i + 1;
  // The matrix boundary C and R = C + V are multiples of 16
  // (the host checks), so a tile lies in one matrix and the base address of
  // each load is uniform; the lane adds a fixed byte offset.  Every slot
  // issues its load: one outside the weights (past the last tile or past
  // the row) reads the first KiB of the qkv weight, the same line in every
  // workgroup, and its data is never used.  A load under a condition would
  // make the compiler's waits below count it as not issued and wait for
  // later loads too.
  const uint32_t lane_off = (uint32_t)((wave << (lh + 2)) + (lane << 4));  // rows 2w.. (2H bytes each) + lane
  const char* spare = reinterpret_cast<const char*>(a.w[0]);
  auto issue_tile = [&](int i) {
    const int tile = b + i * G;
    const int row0 = tile * 16;
    const bool zt = row0 >= C;
    const char* tp = reinterpret_cast<const char*>(zt ? a.w[1] : a.w[0]) +
                     ((size_t)(tile < ntiles ? row0 - (zt ? C : 0) : 0) << (lh + 1));
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const bool live = s < ks && tile < ntiles;
      const size_t so = ((size_t)(s >> lpr_sh) << (lh + 1)) + ((size_t)(s & (LPR - 1)) << 10);
      av[i][s] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(live ? tp + so + lane_off : spare + (lane << 4)));
    }
  };
  // kStepTilesAhead tiles ahead of the one being reduced, so that tiles
  // complete one after another and the per-tile work (VALU dot products, or
  // LDS staging and MFMAs) runs under the stream: issued all at once, a
  // wavefront's first tile completes about as late as its last, and the
  // wavefront cannot even issue the rest until the memory pipeline drains.
  // Only the first tile is issued before the staging, the next one right
  // after it: issuing a tile's loads takes each wavefront about a
  // microsecond (the CU's memory pipeline backpressures), and the staging's
  // barriers wait for the last wavefront to finish issuing, so with two
  // tiles ahead the tokens were staged 1.3-1.6 us later (T = 1 20.05 ->
  // 19.27 us, T = 8 24.97 -> 24.66 us).  (Every load of the tile goes out
  // before the staging: left to itself, the scheduler hoists the staging's
  // first token conversions between them, and the wait for the tokens then
  // holds back the rest of the tile.)
  issue_tile(0);
  __builtin_amdgcn_sched_barrier(0);
  FK_MARK(11);


  // ---- stage the normalised tokens -----------------------------------------
  uint32_t tag = 0u, plim = 0u;
  // MFMA path: bf16 hi/lo columns in s_xb [H/8 chunks][NCP][8] (bcol_slot);
  // VALU path: fp32 in s_x [T][H].  Chunk q of thread tid is token-major
  // chunk tid + 512 q; H % 512 == 0, so a wavefront's 64 chunks belong to one
  // token and the sum of squares reduces in a fixed order.
  uint16_t* s_xb = reinterpret_cast<uint16_t*>(s_dyn);
  {
    if constexpr (XCH == 4) {
      // the four chunks' sums of squares in one transposed reduction (lane
      // 16q holds chunk q's sum)
      float p4[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float xv[8];
        raw8_to_f32<BFX>(xr[q], xv);
        float p = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) p = fmaf(xv[e], xv[e], p);
        p4[q] = tid + q * 512 < nchunk ? p : 0.f;
      }
      const float ps = rows4_sum(p4);
      const int base = (tid & ~63) + (lane >> 4) * 512;
      if ((lane & 15) == 0 && base < nchunk) s_part[base >> cpt_sh][(base & (cpt - 1)) >> 6] = ps;
    } else {
#pragma unroll
      for (int q = 0; q < XCH; ++q) {
        const int idx8 = tid + q * 512;
        if (idx8 < nchunk) {  // uniform per wavefront
          float xv[8];
          raw8_to_f32<BFX>(xr[q], xv);
          float p = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) p = fmaf(xv[e], xv[e], p);
          p = wave_sum(p);
          if (lane == 0) s_part[idx8 >> cpt_sh][(idx8 & (cpt - 1)) >> 6] = p;
        }
      }
    }
    FK_MARK(12);
    if (tid == 0) {
      s_fail = 0;
      s_hdr[0] = hdr.epoch;
      s_hdr[1] = hdr.set;
      s_hdr[2] = hdr.err;
    }
    __syncthreads();
    {
      WaitHeader h{s_hdr[0], s_hdr[1], s_hdr[2]};
      const WaitLimits wl = h.limits();
      tag = wl.tag;
      plim = wl.poll;
    }
    if (tid < T) {
      float tot = 0.f;
      for (int w = 0; w < (cpt >> 6); ++w) tot += s_part[tid][w];
      s_rs[tid] = rsqrtf(tot / (float)H + a.eps);
    }
    if (tid == 0) store_tagged(a.tw.started + b, 0.f, tag);
    __syncthreads();
    // (four chunks: the head workgroups' a and b logit parts of all four in
    // one transposed reduction, lane 8i holding part i = 2 q + (a: 0, b: 1))
    float dab[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) dab[i] = 0.f;
#pragma unroll
    for (int q = 0; q < XCH; ++q) {
      const int idx8 = tid + q * 512;
      if (idx8 < nchunk) {
        const int t = idx8 >> cpt_sh, k0 = (idx8 & (cpt - 1)) << 3;
        float xv[8], nv[8], y[8];
        raw8_to_f32<BFX>(xr[q], xv);
        raw8_to_f32<true>(nr[q], nv);
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = xv[e] * s_rs[t] * (1.0f + nv[e]);
        if (XCH == 4 && is_head) {
          float wa[8], wb[8], da = 0.f, db = 0.f;
          raw8_to_f32<true>(war, wa);
          raw8_to_f32<true>(wbr, wb);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            da = fmaf(wa[e], y[e], da);
            db = fmaf(wb[e], y[e], db);
          }
          dab[(2 * q) & 7] = da;
          dab[(2 * q + 1) & 7] = db;
        } else if (is_head) {  // this chunk's share of the a and b logits of token t
          float wa[8], wb[8], da = 0.f, db = 0.f;
          raw8_to_f32<true>(war, wa);
          raw8_to_f32<true>(wbr, wb);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            da = fmaf(wa[e], y[e], da);
            db = fmaf(wb[e], y[e], db);
          }
          da = wave_sum(da);
          db = wave_sum(db);
          if (lane == 0) {
            s_abp[t][(idx8 & (cpt - 1)) >> 6][0] = da;
            s_abp[t][(idx8 & (cpt - 1)) >> 6][1] = db;
          }
        }
        if constexpr (VALU_A) {
          float4* dst = reinterpret_cast<float4*>(reinterpret_cast<float*>(s_dyn) + (size_t)t * H + k0);
          dst[0] = make_float4(y[0], y[1], y[2], y[3]);
          dst[1] = make_float4(y[4], y[5], y[6], y[7]);
        } else {
          u32x4 vh, vl;
          split_hi_lo8(y, vh, vl);
          const int c = k0 >> 3;
          *reinterpret_cast<u32x4*>(s_xb + (size_t)bcol_slot(c, 2 * t, NCP) * 8) = vh;
          *reinterpret_cast<u32x4*>(s_xb + (size_t)bcol_slot(c, 2 * t + 1, NCP) * 8) = vl;
        }
      }
    }
    if (XCH == 4 && is_head) {
      const float ab = rows8_sum(dab);
      const int i = lane >> 3, base = (tid & ~63) + (i >> 1) * 512;
      if ((lane & 7) == 0 && base < nchunk) s_abp[base >> cpt_sh][(base & (cpt - 1)) >> 6][i & 1] = ab;
    }
    __syncthreads();
  }
  FK_MARK(1);
#pragma unroll
  for (int i = 1; i < kStepTilesPerWG; ++i)
    if (i < kStepTilesAhead) issue_tile(i);  // the rest of the tiles ahead

  if constexpr (VALU_A) {
    // ---- phase A (T <= 2): whole-row dot products on the VALU --------------
    // Each wavefront finishes its two rows of a tile as soon as the tile's
    // loads are in: no LDS round trip and no workgroup barrier, so the work
    // hides under the weight stream.  Lane l holds elements 512 p + 8 l .. + 7
    // of a row (p < 4); the tokens' matching elements come from s_x.
    const float* s_x = reinterpret_cast<const float*>(s_dyn);
    float xk[NT][4][8];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const float4* src = reinterpret_cast<const float4*>(s_x + (size_t)(t < T ? t : 0) * H + p * 512 + lane * 8);
        const float4 u0 = src[0], u1 = src[1];
        xk[t][p][0] = u0.x; xk[t][p][1] = u0.y; xk[t][p][2] = u0.z; xk[t][p][3] = u0.w;
        xk[t][p][4] = u1.x; xk[t][p][5] = u1.y; xk[t][p][6] = u1.z; xk[t][p][7] = u1.w;
      }
    // Results of the row this lane finishes (lane 2i + rr: row rr of tile i),
    // stored after the last tile: a store between two tiles' loads would be
    // waited for with them (stores share the loads' in-order counter;
    // -1 us at T = 1).  (A kernel size other than 4 takes the general form
    // below, which stores at once.)
    float o_val[NT];
    uint32_t o_nc[2] = {0u, 0u};
    int o_row = 0, o_kind = 0;  // 1: a qkv row (conv'd, and its next conv state), 2: a z row
#pragma unroll
    for (int t = 0; t < NT; ++t) o_val[t] = 0.f;
#pragma unroll
    for (int i = 0; i < kStepTilesPerWG; ++i) {
      if (i < ntl) {  // uniform per workgroup
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
          const int row = (b + i * G) * 16 + 2 * wave + rr;
          float v[NT];
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            v[t] = 0.f;
            if (t < T) {
              float d = 0.f;
#pragma unroll
              for (int p = 0; p < 4; ++p) {
                float w8[8];
                raw8_to_f32<true>(Raw8<true>{av[i][rr * 4 + p]}, w8);
#pragma unroll
                for (int e = 0; e < 8; ++e) d = fmaf(w8[e], xk[t][p][e], d);
              }
              v[t] = wave_sum(d);
            }
          }
          // the lane holding the row's conv taps finishes the row
          if (lane == 2 * i + rr) {
            if (row < C && a.KS == 4) {
              // The model's kernel size: the window entries are known at
              // compile time (the general form below selects every entry
              // through run-time compares, ~800 instructions per row that
              // every wavefront issues).  Same products in the same order.
              float sq[4 + NT], wk[4];
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                sq[j] = raw_value<true>(cwin_raw[j]);
                wk[j] = raw_value<true>(cwk_raw[j]);
              }
#pragma unroll
              for (int t = 0; t < NT; ++t) sq[4 + t] = v[t];
#pragma unroll
              for (int t = 0; t < NT; ++t) {
                float cv = 0.f;
#pragma unroll
                for (int j = 0; j < 4; ++j) cv = fmaf(wk[j], sq[t + 1 + j], cv);
                o_val[t] = silu(cv);
              }
              // the next state: entries T .. T + 3
              uint32_t nb[4];
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                float e = sq[j];
#pragma unroll
                for (int tt = 1; tt <= NT; ++tt) e = T == tt ? sq[tt + j] : e;
                nb[j] = f32_to_bf16_bits(e);
              }
              o_nc[0] = nb[0] | (nb[1] << 16);
              o_nc[1] = nb[2] | (nb[3] << 16);
              o_row = row;
              o_kind = 1;
            } else if (row < C) {
              // causal conv + SiLU: token t's window is entries t + 1 .. t + KS
              // of [conv state (KS) | tokens]
              float st[8], wk[8];
#pragma unroll
              for (int j = 0; j < 8; ++j) {
                st[j] = raw_value<true>(cwin_raw[j]);
                wk[j] = raw_value<true>(cwk_raw[j]);
              }
              auto seq = [&](int q) {
                float r = 0.f;
#pragma unroll
                for (int j = 0; j < 8; ++j) r = q == j && j < a.KS ? st[j] : r;
#pragma unroll
                for (int t = 0; t < NT; ++t) r = q == a.KS + t ? v[t] : r;
                return r;
              };
#pragma unroll
              for (int t = 0; t < NT; ++t) {
                if (t < T) {
                  float cv = 0.f;
#pragma unroll
                  for (int j = 0; j < 8; ++j)
                    if (j < a.KS) cv = fmaf(wk[j], seq(t + 1 + j), cv);
                  store_tagged(a.tw.mix + (size_t)t * C + row, silu(cv), tag);
                }
              }
#pragma unroll
              for (int j = 0; j < 8; ++j)
                if (j < a.KS) reinterpret_cast<uint16_t*>(a.next_conv)[(size_t)row * a.KS + j] = f32_to_bf16_bits(seq(T + j));
            } else {
#pragma unroll
              for (int t = 0; t < NT; ++t) o_val[t] = v[t];
              o_row = row;
              o_kind = 2;
            }
          }
        }
      }
      if (i + kStepTilesAhead < kStepTilesPerWG) issue_tile(i + kStepTilesAhead);
    }
    if (o_kind == 1) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
        if (t < T) store_tagged(a.tw.mix + (size_t)t * C + o_row, o_val[t], tag);
      uint16_t* nc = reinterpret_cast<uint16_t*>(a.next_conv) + (size_t)o_row * 4;
      nc[0] = (uint16_t)o_nc[0];
      nc[1] = (uint16_t)(o_nc[0] >> 16);
      nc[2] = (uint16_t)o_nc[1];
      nc[3] = (uint16_t)(o_nc[1] >> 16);
    } else if (o_kind == 2) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
        if (t < T) store_tagged(a.tw.z + (size_t)t * V + (o_row - C), o_val[t], tag);
    }
    __syncthreads();  // phases B and C reuse the dynamic LDS
  } else {
  // ---- phase A: projections ---------------------------------------------
  // LDS: s_xb | the workgroup's tile [16 rows][2H + 16 B] (row pitch padded
  // by 16 B: the 16 rows of an operand read fall in distinct banks).  Per
  // tile the wavefronts write their rows, then each runs the MFMAs of its K
  // range (H / 8) over all 16 rows.  The partial sums [wave][tile][16][NC]
  // go to the tile area once every tile is done.
  const int pitch = 2 * H + 16;
  char* s_tile = s_dyn + (size_t)H * NCP * 2;
  {
    // the tokens' B operands of this wavefront's K range, the same for every
    // tile: read from LDS once (the staging ends with a barrier)
    u32x4 bvr[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int c = (wave * kw + s * 32 + g4 * 8) >> 3;
      bvr[s] = s < ks && n < NC ? *reinterpret_cast<const u32x4*>(s_xb + (size_t)bcol_slot(c, n, NCP) * 8) : u32x4{0, 0, 0, 0};
    }
    f32x4_t acc[kStepTilesPerWG];
#pragma unroll
    for (int i = 0; i < kStepTilesPerWG; ++i) {
      acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      if (i < ntl) {  // uniform per workgroup
#pragma unroll
        for (int s = 0; s < 8; ++s)
          if (s < ks)
            *reinterpret_cast<u32x4*>(s_tile + (2 * wave + (s >> lpr_sh)) * pitch + ((s & (LPR - 1)) << 10) + (lane << 4)) =
                av[i][s];
        __syncthreads();
        // MFMA steps: operand lane (row n, k group g4) reads 8 k of its row
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          if (s < ks) {
            const int k = wave * kw + s * 32 + g4 * 8;
            const u32x4 wv = *reinterpret_cast<const u32x4*>(s_tile + n * pitch + k * 2);
            acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, wv),
                                                             __builtin_bit_cast(bf16x8_t, bvr[s]), acc[i], 0, 0, 0);
          }
        }
        __syncthreads();
      }
      if (i + kStepTilesAhead < kStepTilesPerWG) issue_tile(i + kStepTilesAhead);
    }
    float* s_red = reinterpret_cast<float*>(s_tile);  // [wave][tile][16][NC]
    const int red_w = kStepTilesPerWG * 16 * NC;
    if (n < NC) {
#pragma unroll
      for (int i = 0; i < kStepTilesPerWG; ++i)
        if (i < ntl)
#pragma unroll
          for (int q = 0; q < 4; ++q) s_red[(size_t)wave * red_w + ((size_t)i * 16 + g4 * 4 + q) * NC + n] = acc[i][q];
    }
    __syncthreads();
    // One thread per (tile, row, token): sums the wavefronts' partials (hi +
    // lo) in wavefront order.  A qkv row's sequence [conv state | tokens]
    // goes through LDS, and each token's thread applies the causal conv to
    // its window (entries t + 1 .. t + KS) and SiLU.
    float* s_seq = s_red + (size_t)kStepWaves * red_w;  // [tile][16][16]
    const int ei = tid >> 7, er = (tid >> 3) & 15, et = tid & 7;
    const int erow = (b + ei * G) * 16 + er;
    const bool elive = ei < ntl && erow < R && et < T;
    float* sq = s_seq + (ei * 16 + er) * 16;
    float ev = 0.f;
    if (elive) {
      const float* pr = s_red + ((size_t)ei * 16 + er) * NC + 2 * et;
      for (int w = 0; w < kStepWaves; ++w) ev += pr[(size_t)w * red_w] + pr[(size_t)w * red_w + 1];
      sq[a.KS + et] = ev;
      if (et == 0 && erow < C) {
#pragma unroll
        for (int q = 0; q < 8; ++q)
          if (q < a.KS) sq[q] = raw_value<true>(cwin_raw[q]);
      }
    }
    __syncthreads();
    if (elive) {
      if (erow < C) {
        float cv = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (j < a.KS) cv = fmaf(raw_value<true>(cwk_raw[j]), sq[et + 1 + j], cv);
        store_tagged(a.tw.mix + (size_t)et * C + erow, silu(cv), tag);
        if (et == 0) {
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (j < a.KS) reinterpret_cast<uint16_t*>(a.next_conv)[(size_t)erow * a.KS + j] = f32_to_bf16_bits(sq[T + j]);
        }
      } else {
        store_tagged(a.tw.z + (size_t)et * V + (erow - C), ev, tag);
      }
    }
    __syncthreads();  // phases B and C reuse the dynamic LDS
  }
  }

  FK_MARK(2);
  // ---- W_out for phase C, fetched while the heads run --------------------
  // Phase C is split over K.  Unit (rb, ks), on workgroup b = rb * nks + ks,
  // multiplies rows 128 rb .. + 128 of W_out, restricted to the columns
  // kcu ks .. + kcu of kcu / 128 heads (kcu = min(V, 512)), by those heads'
  // outputs: wavefront w holds rows 16 w .. + 16 of the block in the MFMA
  // operand layout.  Each unit reads T * kcu head outputs instead of T * V,
  // and each output row sums nks partials afterwards.
  const int kcu = V < 512 ? V : 512, nks = V / kcu, nunits = (H >> 7) * nks;
  const int ksc = kcu >> 5;  // MFMA steps per unit (<= 16)
  const bool is_unit = b < nunits;
  const int keeper = nunits - 1;  // the epoch keeper: the last unit (units wait longest for their inputs)
  const int urb = is_unit ? b / nks : 0, uks = is_unit ? b - urb * nks : 0;
  u32x4 ov[16];
  if (is_unit) {
    const uint16_t* wp =
        reinterpret_cast<const uint16_t*>(a.w_out) + (size_t)(urb * 128 + wave * 16 + n) * V + (size_t)uks * kcu;
#pragma unroll
    for (int s = 0; s < 16; ++s)
      if (s < ksc) ov[s] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wp + s * 32 + g4 * 8));
  }
  // residual inputs of this workgroup's output rows (thread t*16 + r)
  uint32_t xres[1];
  gather_raw<BFX>(a.x, is_out && tid < 16 * T ? (size_t)(tid >> 4) * H + b * 16 + (tid & 15) : 0, 0, 1, xres);

  // ---- epoch keeper ------------------------------------------------------
  if (b == keeper) {
    bool ok = true;
    for (int base = tid; base < G; base += 512 * 2) {
      uint64_t w[2];
      const uint64_t* srcs[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int r = base + j * 512;
        srcs[j] = r < G ? a.tw.started + r : nullptr;
        w[j] = srcs[j] ? load_tagged(srcs[j]) : 0ull;
      }
      ok = poll_tagged<2>(w, srcs, tag, plim) && ok;
    }
    if (!ok) s_fail = 1;
    __syncthreads();
    // (not after a failed wait: a workgroup that has not read the epoch yet
    // would take the next launch's tag; the error word poisons later launches)
    if (tid == 0 && !s_fail) store_coherent(&a.tw.tickets[kStepTicketEpoch], tag);
  }

  // ---- phase B: gated delta rule, a quarter of one value head ------------
  if (is_head) {
    // s_in: [T][kStepInPitch]: q[128], k[128] (normalised), v[32], z[32]
    // (this quarter's value columns); then s_o [T][32].  a and b are this
    // workgroup's own (s_abp).
    float* s_in = reinterpret_cast<float*>(s_dyn);
    float* s_o = s_in + (size_t)T * kStepInPitch;
    // the state quarter, column-major [32][kStepStPitch] (rows padded by 4:
    // the transposing writes of one wavefront fall in two banks' worth of
    // distinct rows)
    float* s_st = s_o + (size_t)T * kStepQCols;
    const int hq = head / (Hv / a.Hk);
    bool ok = true;
    // The consumers poll their inputs directly (tagged words re-read until
    // they carry this launch's tag): with hint words per tile first, a round
    // trip more, the step took 0.3-0.4 us longer at 3-8 tokens.
    __syncthreads();
    // Wavefront t < T reads token t's inputs (lane: q and k rows lane and
    // lane + 64, and v (lanes < 32) or z of this quarter's columns), l2-
    // normalises q (times D^-1/2) and k with two wavefront sums and stages
    // them; its lane 0 computes the token's decay and beta from the a/b
    // logit parts (in wavefront order).
    if (wave < T) {
      const int t = wave;
      const uint64_t* mrow = a.tw.mix + (size_t)t * C;
      const uint64_t* qrow = mrow + (size_t)hq * kStepD;
      const uint64_t* krow = mrow + (size_t)(a.Hk + hq) * kStepD;
      const uint64_t* srcs[5] = {
          qrow + lane, qrow + lane + 64, krow + lane, krow + lane + 64,
          lane < kStepQCols ? mrow + (size_t)(2 * a.Hk + head) * kStepD + quarter * kStepQCols + lane
                            : a.tw.z + (size_t)t * V + (size_t)head * kStepD + quarter * kStepQCols + (lane - kStepQCols)};
      uint64_t w[5];
#pragma unroll
      for (int j = 0; j < 5; ++j) w[j] = load_tagged(srcs[j]);
      ok = poll_tagged<5>(w, srcs, tag, plim);
      const float q0 = value_of(w[0]), q1 = value_of(w[1]), k0 = value_of(w[2]), k1 = value_of(w[3]);
      const float sq = wave_sum(q0 * q0 + q1 * q1), sk = wave_sum(k0 * k0 + k1 * k1);
      const float qs = rsqrtf(sq + a.eps) * rsqrtf((float)kStepD), kss = rsqrtf(sk + a.eps);
      float* tin = s_in + (size_t)t * kStepInPitch;
      tin[lane] = q0 * qs;
      tin[lane + 64] = q1 * qs;
      tin[kStepD + lane] = k0 * kss;
      tin[kStepD + lane + 64] = k1 * kss;
      tin[2 * kStepD + lane] = value_of(w[4]);  // v[32] then z[32]
      if (lane == 0) {
        float ab[2] = {0.f, 0.f};
        for (int q = 0; q < (cpt >> 6); ++q) {
          ab[0] += s_abp[t][q][0];
          ab[1] += s_abp[t][q][1];
        }
        const float neg_a = -expf(raw_value<true>(alog[0]));
        const float gin = ab[0] + raw_value<true>(dtb1[0]);
        s_sc[t][0] = expf(neg_a * (fmaxf(gin, 0.f) + log1pf(expf(-fabsf(gin)))));
        s_sc[t][1] = 1.f / (1.f + expf(-ab[1]));
      }
    }
    if (!ok) s_fail = 1;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if constexpr (VALU_A) break;
      const int r = (tid >> 3) + 64 * j, c0 = (tid & 7) * 4;
      s_st[(c0 + 0) * kStepStPitch + r] = __uint_as_float(S_ld[j][0]);
      s_st[(c0 + 1) * kStepStPitch + r] = __uint_as_float(S_ld[j][1]);
      s_st[(c0 + 2) * kStepStPitch + r] = __uint_as_float(S_ld[j][2]);
      s_st[(c0 + 3) * kStepStPitch + r] = __uint_as_float(S_ld[j][3]);
    }
    __syncthreads();
    FK_MARK(3);
    // inputs incomplete (a failed wait): the head's outputs and state are NaN
    const bool bad_in = s_fail;
    // Recurrence: lanes 16 jl' .. 16 jl' + 15 of a wavefront share a value
    // column; each holds 8 rows of the state and the column sums reduce over
    // the 16 lanes.  The next token's q, k and v are read from LDS while the
    // current one runs.
    float S[8];
    if constexpr (VALU_A) {
#pragma unroll
      for (int m = 0; m < 8; ++m) S[m] = raw_value<false>(S_raw[m]);
    } else {
      const float4* sp = reinterpret_cast<const float4*>(s_st + (size_t)sjl * kStepStPitch + sgr * 8);
      const float4 s0 = sp[0], s1 = sp[1];
      S[0] = s0.x; S[1] = s0.y; S[2] = s0.z; S[3] = s0.w;
      S[4] = s1.x; S[5] = s1.y; S[6] = s1.z; S[7] = s1.w;
    }
    auto load_tok = [&](int t, float (&k8)[8], float (&q8)[8], float& v) {
      const float* tin = s_in + (size_t)t * kStepInPitch;
      const float4* k4 = reinterpret_cast<const float4*>(tin + kStepD + sgr * 8);
      const float4* q4 = reinterpret_cast<const float4*>(tin + sgr * 8);
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const float4 kk = k4[m], qq = q4[m];
        k8[4 * m] = kk.x; k8[4 * m + 1] = kk.y; k8[4 * m + 2] = kk.z; k8[4 * m + 3] = kk.w;
        q8[4 * m] = qq.x; q8[4 * m + 1] = qq.y; q8[4 * m + 2] = qq.z; q8[4 * m + 3] = qq.w;
      }
      v = tin[2 * kStepD + sjl];
    };
    float kc[8], qc[8], vc;
    load_tok(0, kc, qc, vc);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (t < T) {
        const float decay = s_sc[t][0], beta = s_sc[t][1];
        float kx[8], qx[8], vx = 0.f;
        if (t + 1 < T) load_tok(t + 1, kx, qx, vx);
        float part = 0.f;
#pragma unroll
        for (int m = 0; m < 8; ++m) {
          S[m] *= decay;
          part = fmaf(S[m], kc[m], part);
        }
        const float ksum = row16_sum(part);
        const float delta = (vc - ksum) * beta;
        float op = 0.f;
#pragma unroll
        for (int m = 0; m < 8; ++m) {
          S[m] = fmaf(kc[m], delta, S[m]);
          op = fmaf(S[m], qc[m], op);
        }
        const float o = row16_sum(op);
        if (sgr == 0) s_o[t * kStepQCols + sjl] = o;
        if (t + 1 < T) {
#pragma unroll
          for (int m = 0; m < 8; ++m) {
            kc[m] = kx[m];
            qc[m] = qx[m];
          }
          vc = vx;
        }
      }
    }
    __syncthreads();
    FK_MARK(4);
    // Gated RMSNorm, its scale left to phase C: each quarter stores its
    // columns gated but not yet scaled, o * w * silu(z), and its sum of
    // squares of o; the phase C unit reading the head adds the four sums in
    // quarter order and scales the head's columns as it stages them.
    if (wave < T) {
      const int t = wave;
      const float o = lane < kStepQCols ? s_o[t * kStepQCols + lane] : 0.f;
      const float ss = wave_sum(o * o);
      if (lane == 0)
        store_tagged(a.tw.hss + (size_t)t * kStepHssPitch + head * kStepHeadWGs + quarter, poison_if(bad_in, ss), tag);
      if (lane < kStepQCols) {
        const float zz = s_in[(size_t)t * kStepInPitch + 2 * kStepD + kStepQCols + lane];
        store_tagged(a.tw.norm + (size_t)t * V + (size_t)head * kStepD + quarter * kStepQCols + lane,
                     poison_if(bad_in, o * raw_value<true>(lnw1[0]) * silu(zz)), tag);
      }
    }
    // (a barrier: every wavefront has issued its gated values and sums
    // above before any of the 16 KB of state stores below is issued, so
    // those stores do not sit in the CU's memory pipeline ahead of them;
    // without it the step took 0.2-0.9 us longer.  It does not wait for the
    // stores to be acknowledged: __syncthreads() compiles to s_barrier with
    // an LDS wait only on gfx950)
    __syncthreads();
    FK_MARK(5);
    {
      const size_t base = ((size_t)head * kStepD + (size_t)sgr * 8) * kStepD + jcol;
#pragma unroll
      for (int m = 0; m < 8; ++m) reinterpret_cast<float*>(a.next_rec)[base + (size_t)m * kStepD] = poison_if(bad_in, S[m]);
    }
    __syncthreads();  // s_dyn is reused below
  }

  // ---- phase C1: partial output projection of unit (urb, uks) ------------
  if (is_unit) {
    uint16_t* s_nb = reinterpret_cast<uint16_t*>(s_dyn);  // [kcu/8][NCP][8] bf16 (bcol_slot)
    const int h0 = uks * (kcu / kStepD), nh = kcu / kStepD;  // heads of the unit's columns
    bool ok = true;
    // (the heads' values polled directly, as the heads poll theirs: with
    // head hint words first the step took 0.6 us longer at 3-8 tokens)
    __syncthreads();
    // The T * kcu inputs, read coalesced (thread tid: words tid + 512 j of
    // the unit's [T][kcu] block) with the quarter sums of squares of its
    // heads, into LDS; then thread (t, c) scales the 8 columns of chunk c of
    // token t by their head's RMSNorm factor and stages them as hi + lo.
    const int lkcu = 31 - __builtin_clz((unsigned)kcu), lcu = lkcu - 3, cpu = 1 << lcu;  // chunks per token
    static_assert(kStepMaxTokens * 512 / 8 <= 512, "unit inputs exceed one chunk per thread");
    float* s_val = reinterpret_cast<float*>(s_dyn + (size_t)kcu * NCP * 2);  // [T][kcu]
    float* s_hss = s_val + (size_t)T * kcu;                                  // [T][nh * 4]
    {
      const int nhq = nh * kStepHeadWGs;
      uint64_t w[NT + 1];
      const uint64_t* srcs[NT + 1];
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int g = tid + 512 * j, t = g >> lkcu;
        srcs[j] = t < T ? a.tw.norm + (size_t)t * V + (size_t)uks * kcu + (g & (kcu - 1)) : nullptr;
      }
      {
        const int t = tid / nhq, hq = tid - t * nhq;
        srcs[NT] = t < T ? a.tw.hss + (size_t)t * kStepHssPitch + h0 * kStepHeadWGs + hq : nullptr;
      }
#pragma unroll
      for (int j = 0; j <= NT; ++j) w[j] = srcs[j] ? load_tagged(srcs[j]) : 0ull;
      ok = poll_tagged<NT + 1>(w, srcs, tag, plim);
#pragma unroll
      for (int j = 0; j < NT; ++j)
        if (srcs[j]) s_val[tid + 512 * j] = value_of(w[j]);
      if (srcs[NT]) s_hss[tid] = value_of(w[NT]);
    }
    __syncthreads();
    {
      const int t = tid >> lcu, c = tid & (cpu - 1);
      if (t < T) {
        float tot = 0.f;
#pragma unroll
        for (int q = 0; q < kStepHeadWGs; ++q) tot += s_hss[t * nh * kStepHeadWGs + (c >> 4) * kStepHeadWGs + q];
        const float scale = rsqrtf(tot / (float)kStepD + a.eps);
        const float4* vp = reinterpret_cast<const float4*>(s_val + (size_t)t * kcu + c * 8);
        const float4 v0 = vp[0], v1 = vp[1];
        float y[8] = {v0.x * scale, v0.y * scale, v0.z * scale, v0.w * scale,
                      v1.x * scale, v1.y * scale, v1.z * scale, v1.w * scale};
        u32x4 vh, vl;
        split_hi_lo8(y, vh, vl);
        *reinterpret_cast<u32x4*>(s_nb + (size_t)bcol_slot(c, 2 * t, NCP) * 8) = vh;
        *reinterpret_cast<u32x4*>(s_nb + (size_t)bcol_slot(c, 2 * t + 1, NCP) * 8) = vl;
      }
    }
    if (!ok) s_fail = 1;
    __syncthreads();
    const bool bad_unit = s_fail;
    FK_MARK(6);
    f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      if (s < ksc) {
        const int c = s * 4 + g4;
        const u32x4 bv = n < NC ? *reinterpret_cast<const u32x4*>(s_nb + (size_t)bcol_slot(c, n, NCP) * 8) : u32x4{0, 0, 0, 0};
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, ov[s]),
                                                      __builtin_bit_cast(bf16x8_t, bv), acc, 0, 0, 0);
      }
    }
    // hi + lo columns of token t sit in lanes n = 2t and 2t + 1
    float pq[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) pq[q] = acc[q] + __uint_as_float(dpp_u32<kDppQuadXor1>(__float_as_uint(acc[q])));
    if (n < NC && (n & 1) == 0) {
      const size_t o = ((size_t)uks * T + (n >> 1)) * H + (size_t)urb * 128 + wave * 16 + g4 * 4;
#pragma unroll
      for (int q = 0; q < 4; ++q) store_tagged(a.tw.part + o + q, poison_if(bad_unit, pq[q]), tag);
    }
  }

  FK_MARK(7);
  // ---- phase C2: rows 16b..16b+15 = sum of the nks unit partials ----------
  if (is_out) {
    // (nks partials per thread, polled directly)
    if (tid < 16 * T) {
      const int r = tid & 15, t = tid >> 4;
      uint64_t w[8];
      const uint64_t* srcs[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        srcs[j] = j < nks ? a.tw.part + ((size_t)j * T + t) * H + b * 16 + r : nullptr;
        w[j] = srcs[j] ? load_tagged(srcs[j]) : 0ull;
      }
      const bool pok = poll_tagged<8>(w, srcs, tag, plim);
      if (!pok) s_fail = 1;
      float v = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j < nks) v += value_of(w[j]);
      v = poison_if(!pok, v);
      FK_MARK(8);
      const size_t o = (size_t)t * H + b * 16 + r;
      a.update[o] = v;
      if (a.hidden_out) a.hidden_out[o] = raw_value<BFX>(xres[0]) + v;
    }
  }
  if (tid == 0 && s_fail)
    __hip_atomic_fetch_or(&a.tw.tickets[kStepTicketError], FK_DEVICE_ERR_BARRIER, __ATOMIC_RELAXED,
                          __HIP_MEMORY_SCOPE_AGENT);
  FK_MARK(9);
  FK_TIMELINE_COMMIT(deltanet_step, blockIdx.x);
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
  StepTagWs tw;  // single-launch step: fixed-size tagged hand-off region first
  DnWs dn;
  float* mixed;
  float* z;
  float* a;
  float* b;
};

static size_t step_tag_layout(char* base, StepTagWs* tw) {
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t at = off;
    off = align_up(off + bytes, 256);
    return base ? base + at : nullptr;
  };
  tw->tickets = reinterpret_cast<uint32_t*>(take(16 * sizeof(uint32_t)));
  tw->mix = reinterpret_cast<uint64_t*>(take(kStepMixWords * 8));
  tw->z = reinterpret_cast<uint64_t*>(take(kStepVWords * 8));
  tw->norm = reinterpret_cast<uint64_t*>(take(kStepVWords * 8));
  tw->started = reinterpret_cast<uint64_t*>(take((size_t)kStepMaxGrid * 8));
  tw->hss = reinterpret_cast<uint64_t*>(take((size_t)kStepMaxTokens * kStepHssPitch * 8));
  tw->part = reinterpret_cast<uint64_t*>(take(kStepPartWords * 8));
  return off;
}

static size_t step_ws_layout(int T, int Hk, int Hv, int D, char* base, StepWs* ws) {
  size_t off = step_tag_layout(base, &ws->tw);
  off = align_up(off + dn_ws_layout(T, Hv, D, base ? base + off : nullptr, &ws->dn), 256);
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

// Single-launch step: shapes the kernel handles (the real Qwen3.6 layer:
// H 2048, Hk 16, Hv 32, D 128, C 8192), bf16 projection and output weights.
// dt: the ten dtype codes of fk_deltanet_step (hidden, norm weight,
// projections, conv state, conv weight, recurrent state, out projection,
// gated-norm weight, a_log, dt_bias).
static bool step_fused_eligible(int T, int H, int Hk, int Hv, int D, const int* dt, int G) {
  const int C = (2 * Hk + Hv) * D, V = Hv * D, R = C + V;
  bool dtypes_ok = dt[5] == FK_DTYPE_F32;
  for (int i = 1; i < 10; ++i)
    if (i != 5 && dt[i] != FK_DTYPE_BF16) dtypes_ok = false;
  return dtypes_ok && T >= 1 && T <= kStepMaxTokens && D == kStepD && H >= 512 && H <= 2048 && (H & (H - 1)) == 0 &&
         (V & (V - 1)) == 0 && V >= 256 && V <= 4096 && C <= 8192 && Hv <= 64 && Hv % 16 == 0 &&
         G >= H / 16 && (H >> 7) * (V / (V < 512 ? V : 512)) + kStepHeadWGs * Hv <= G &&
         (R + 15) / 16 <= kStepTilesPerWG * G && G <= kStepMaxGrid;
}

static size_t step_fused_lds(int T, int H, int V) {
  // (the VALU projection runs at T <= 2 only with H = 2048, as the launch
  // selects it; other hidden sizes stage through the MFMA path's tile)
  const bool valu_a = T <= 2 && H == 2048;
  const size_t nc = 2 * (size_t)T, ncp = nc <= 2 ? 2 : nc <= 4 ? 4 : nc <= 8 ? 8 : 16;
  const size_t tile = (size_t)16 * (2 * (size_t)H + 16),
               red = ((size_t)kStepWaves * kStepTilesPerWG * 16 * nc + kStepTilesPerWG * 16 * 16) * 4;
  const size_t pa = valu_a ? (size_t)T * H * 4 : (size_t)H * ncp * 2 + (tile > red ? tile : red);
  const size_t pb = ((size_t)T * kStepInPitch + (size_t)T * kStepQCols + (size_t)kStepQCols * kStepStPitch) * 4;
  const size_t kcu = V < 512 ? V : 512;
  // phase C: the unit's staging [kcu/8][ncp][8] bf16, values [T][kcu], sums of squares [T][16]
  const size_t pc = kcu * ncp * 2 + ((size_t)T * kcu + (size_t)T * 4 * kStepHeadWGs) * 4;
  return pa > pb ? (pa > pc ? pa : pc) : (pb > pc ? pb : pc);
}

// Dynamic LDS reserved for the step kernel: its need at T = 8, H = 2048, V = 4096.
constexpr size_t kStepMaxLds = (size_t)4096 * 16 * 2 + (size_t)kStepWaves * 16 * 16 * 4;

// Grid of the single-launch step (one workgroup per CU, capped at the
// co-resident capacity), or 0 when the device cannot host it.
template <bool BX, int NT>
static int step_grid() {
  static int cap_cache[64] = {0};
  static int attr_ok[64] = {0};  // 0 unknown, 1 set, -1 refused
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (attr_ok[dev] == 0)
    attr_ok[dev] = hipFuncSetAttribute(reinterpret_cast<const void*>(deltanet_step_kernel<BX, NT>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)kStepMaxLds) == hipSuccess
                       ? 1
                       : -1;
  if (attr_ok[dev] < 0) {
    (void)hipGetLastError();
    return 0;
  }
  const int cap = resident_capacity(deltanet_step_kernel<BX, NT>, 512, kStepMaxLds, cap_cache);
  const int cus = device_cus();
  const int G = cap < cus ? cap : cus;
  return G > kStepMaxGrid ? kStepMaxGrid : G;
}

template <bool BX, int NT>
static int launch_step_fused(const StepArgs& sa, int G, hipStream_t s) {
  const size_t shm = step_fused_lds(sa.T, sa.H, sa.V);
  if (shm > kStepMaxLds) return fail(FK_ERR_UNSUPPORTED, "DeltaNet step needs %zu bytes of LDS", shm);
  hipLaunchKernelGGL((deltanet_step_kernel<BX, NT>), dim3(G), dim3(512), shm, s, sa);
  return check_launch("deltanet_step_kernel");
}

// RMSNorm(x) * (off + w) applied to up to four row-major weight matrices
// (rows[i] == 0: unused), f32 outputs [T, rows[i]]: the projection kernel
// without the fused conv, for the other mixers' projections.
int launch_norm_projection(const void* x, int x_dt, const void* nw, int nw_dt, const void* const (&w)[4],
                           const int (&rows)[4], float* const (&out)[4], int weight_dt, int T, int H, float eps,
                           float off, hipStream_t s) {
  ProjArgs pa;
  pa.x = x;
  pa.nw = nw;
  pa.nw_dt = nw_dt;
  for (int i = 0; i < 4; ++i) {
    pa.w[i] = w[i];
    pa.rows[i] = rows[i];
    pa.out[i] = out[i];
  }
  pa.T = T;
  pa.H = H;
  pa.eps = eps;
  pa.off = off;
  pa.conv_state = nullptr;
  pa.cs_dt = FK_DTYPE_F32;
  pa.conv_w = nullptr;
  pa.cw_dt = FK_DTYPE_F32;
  pa.KS = 0;
  pa.conv_out = nullptr;
  pa.next_state = nullptr;
  return launch_project(pa, weight_dt, x_dt, s);
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
  // T <= 2 takes the VALU projections, written for H = 2048
  const bool bx = dtypes[0] == FK_DTYPE_BF16, few = tokens <= 2 && hidden_size == 2048;
  const int G = bx ? (few ? step_grid<true, 2>() : step_grid<true, 8>())
                   : (few ? step_grid<false, 2>() : step_grid<false, 8>());
  // (the single launch reads the state 16 bytes at a time on its MFMA path)
  if (G > 0 && (few || aligned16(recurrent_state)) && step_fused_eligible(tokens, hidden_size, qk_heads, value_heads, head_dim, dtypes, G)) {
    StepArgs sa;
    sa.x = hidden;
    sa.nw = input_norm_weight;
    sa.w[0] = w_qkv;
    sa.w[1] = w_z;
    sa.w[2] = w_a;
    sa.w[3] = w_b;
    sa.conv_state = conv_state;
    sa.conv_w = conv_weight;
    sa.rec_state = recurrent_state;
    sa.w_out = out_proj_weight;
    sa.lnw = linear_norm_weight;
    sa.a_log = a_log;
    sa.dt_bias = dt_bias;
    sa.T = tokens;
    sa.H = hidden_size;
    sa.Hk = qk_heads;
    sa.Hv = value_heads;
    sa.C = conv_dim;
    sa.V = value_heads * head_dim;
    sa.R = conv_dim + sa.V;  // a and b: computed by the head workgroups
    sa.KS = kernel_size;
    sa.eps = eps;
    sa.update = update;
    sa.hidden_out = hidden_out;
    sa.next_conv = next_conv_state;
    sa.next_rec = next_recurrent_state;
    sa.tw = ws.tw;
    if (bx) return few ? launch_step_fused<true, 2>(sa, G, s) : launch_step_fused<true, 8>(sa, G, s);
    return few ? launch_step_fused<false, 2>(sa, G, s) : launch_step_fused<false, 8>(sa, G, s);
  }
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
