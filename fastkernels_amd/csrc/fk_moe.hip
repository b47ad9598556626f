// Qwen3.6 MoE decode layer for gfx950: router + top-k + routing tables,
// gate/up + SwiGLU, down-projection + weighted accumulate + residual.
//
// Data layout in HBM (all row-major, as the reference packs them,
// models/qwen36_weights.py:26-37):
//   router_weight  [E, H]          one 4 KB row per expert at H=2048 (bf16)
//   gate_up        [E, 2I, H]      gate rows 0..I-1, up rows I..2I-1
//   down           [E, H, I]       one 1 KB row per output feature at I=512
//   shared_gate_up [2I, H], shared_down [H, I], shared_gate [H]
// Workspace (fk_moe_workspace_bytes): counters, routing tables, the fp32
// SwiGLU activations act[(T*K + T), I] and the per-pair down-projection
// outputs y[(T*K + T), H].  Rows are indexed by the permuted position of a
// routed (token, slot) pair; the last T rows belong to the shared expert.
//
// Launch structure (one stream, no host synchronisation):
//   1. moe_router_kernel   grid ceil(E/4) x 256 threads.  One wavefront per
//      expert row (weights folded with the norm weight, held in registers,
//      tokens in batches of 4); the last workgroup to arrive (atomic ticket,
//      no cache-wide fence) runs softmax, top-k and the routing tables.
//   2. moe_gateup_kernel   grid slots x (I/8); a slot is one active expert or
//      the shared expert; each workgroup streams 8 gate + 8 up rows of its
//      expert once and applies them to every pair routed there.
//   3. moe_down_kernel     grid slots x (H/16); each workgroup streams 16
//      contiguous down rows (16 KB at I=512) of one expert and writes
//      y[pair, rows] for every pair routed there.
//   4. moe_combine_kernel  out[t] = sum_k w[t,k] y[pos(t,k)] + g_t y[shared t]
//      in slot order, and layer_out = x + out (deterministic, no atomics).
#include "fk_common.h"
#include "fk_host.h"

#include <algorithm>
#include <mutex>

namespace fk {

constexpr int kMaxPairs = 4096;    // T*K handled by the routing-table builder
constexpr int kMaxExperts = 1024;  // matches the reference router limit
constexpr int kGateUpRows = 8;     // intermediates per gate/up workgroup (2 per wave)
constexpr int kDownRowsPerWave = 4; // down rows per wavefront
constexpr int kDownRows = 4 * kDownRowsPerWave;  // down rows per workgroup

struct MoeWs {
  uint32_t* tickets;    // [16] arrival counters; [kTicketEpoch] = fused launch epoch
  // Single-launch layer (T = 1) and small-batch router (T <= 32): tagged hand-off words in
  // a fixed-size region, so that no offset depends on the problem shape
  // (fk_moe_router / fk_moe_align lay the workspace out without I and H).
  uint64_t* f_logits;   // [T, E] router logits (capacity 256 * 256)
  uint64_t* f_act;      // [(T*K + T), I] SwiGLU activations, permuted rows then shared rows (capacity 18 * 512)
  uint64_t* f_sgate;    // [T] shared-expert gates
  uint64_t* f_started;  // [grid] one tagged record per workgroup of the launch (capacity 1024)
  uint64_t* f_sel;      // [T, K] tagged router: expert ids chosen per token (capacity 256 * 8)
  uint64_t* f_y;        // [K, H] single-launch layer: each routed slot's down-projection outputs (capacity 8 * 2048)
  int32_t* counts;      // [E]
  int32_t* offsets;     // [E+1] exclusive prefix of counts
  int32_t* perm;        // [P] permuted position -> pair index t*K+k
  int32_t* inverse;     // [P] pair index -> permuted position
  int32_t* active;      // [E] ids of experts with count > 0, ascending
  int4* slots;          // [E] per active expert: {id, first permuted position, pair count, token of the first pair}
  int32_t* num_active;  // [1]
  int32_t* ids32;       // [P] clamped expert ids
  float* wts;           // [P] routing weights (fp32)
  float* sgate;         // [T] shared-expert gate sigmoid(w_g . x)
  float* act;           // [(P + T), I] SwiGLU activations
  float* y;             // [(P + T), H] per-pair down-projection outputs
};

// Counter slots of MoeWs::tickets.
constexpr int kTicketRouterBarrier = 0;
constexpr int kTicketRouterTables = 1;
constexpr int kTicketEpoch = 8;
constexpr int kTicketError = kWorkspaceErrorWord;
constexpr int kFusedMaxGrid = 1024;
constexpr size_t kFusedLogitWords = 256 * 256;  // tagged router: T <= 256
constexpr size_t kFusedActWords = (2 * 8 + 2) * 512;
constexpr size_t kFusedGateWords = 2;
constexpr size_t kFusedSelWords = 256 * 8;  // tagged router: T <= 256, K <= 8
constexpr size_t kFusedYWords = 8 * 2048;   // single-launch layer: K <= 8, H <= 2048

// Regions sized by I or H come last: fk_moe_router and fk_moe_align lay the
// workspace out with I = H = 0 and must find the routing tables where
// fk_moe_experts and fk_moe_layer do.
static size_t moe_ws_layout(int T, int K, int E, int I, int H, char* base, MoeWs* ws) {
  const size_t P = (size_t)T * K;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t at = off;
    off = align_up(off + bytes, 256);
    return base ? base + at : nullptr;
  };
  ws->tickets = reinterpret_cast<uint32_t*>(take(16 * sizeof(uint32_t)));
  ws->f_logits = reinterpret_cast<uint64_t*>(take(kFusedLogitWords * 8));
  ws->f_act = reinterpret_cast<uint64_t*>(take(kFusedActWords * 8));
  ws->f_sgate = reinterpret_cast<uint64_t*>(take(kFusedGateWords * 8));
  ws->f_started = reinterpret_cast<uint64_t*>(take((size_t)kFusedMaxGrid * 8));
  ws->f_sel = reinterpret_cast<uint64_t*>(take(kFusedSelWords * 8));
  ws->f_y = reinterpret_cast<uint64_t*>(take(kFusedYWords * 8));
  ws->counts = reinterpret_cast<int32_t*>(take((size_t)E * 4));
  ws->offsets = reinterpret_cast<int32_t*>(take((size_t)(E + 1) * 4));
  ws->perm = reinterpret_cast<int32_t*>(take(P * 4));
  ws->inverse = reinterpret_cast<int32_t*>(take(P * 4));
  ws->active = reinterpret_cast<int32_t*>(take((size_t)E * 4));
  ws->slots = reinterpret_cast<int4*>(take((size_t)E * 16));
  ws->num_active = reinterpret_cast<int32_t*>(take(4));
  ws->ids32 = reinterpret_cast<int32_t*>(take(P * 4));
  ws->wts = reinterpret_cast<float*>(take(P * 4));
  ws->sgate = reinterpret_cast<float*>(take((size_t)T * 4));
  ws->act = reinterpret_cast<float*>(take((P + T) * (size_t)I * 4));
  ws->y = reinterpret_cast<float*>(take((P + T) * (size_t)H * 4));
  return off;
}

// ---------------------------------------------------------------------------
// Routing tables (histogram, offsets, stable permutation, active experts).
// Runs inside one workgroup of NWV wavefronts; `s_ids` holds the P clamped ids.
// ---------------------------------------------------------------------------
// Inclusive prefix sum over the wavefront: within each 16-lane row by DPP
// row shifts (lanes shifted in from outside the row read 0), then each row
// adds the totals of the rows below it (read from lanes 15, 31 and 47).
__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
  v += (int)dpp_u32<0x111>((uint32_t)v);  // row_shr:1
  v += (int)dpp_u32<0x112>((uint32_t)v);  // row_shr:2
  v += (int)dpp_u32<0x114>((uint32_t)v);  // row_shr:4
  v += (int)dpp_u32<0x118>((uint32_t)v);  // row_shr:8
  const int r0 = __builtin_amdgcn_readlane(v, 15), r1 = __builtin_amdgcn_readlane(v, 31),
            r2 = __builtin_amdgcn_readlane(v, 47);
  const int row = lane >> 4;
  return v + (row == 0 ? 0 : row == 1 ? r0 : row == 2 ? r0 + r1 : r0 + r1 + r2);
}

// Deterministic, parallel stable counting sort of the P pairs by expert.
// Wave w owns the contiguous pair segment [w*seg, (w+1)*seg); it walks it in
// chunks of 64 (one pair per lane), ranks each pair among equal experts of
// the chunk by scanning the 64 ids through readlane broadcasts, and keeps
// running per-expert counts of its segment in s_wcnt[w][e].  A pair's
// permuted position is offsets[e] + (pairs of e in earlier segments) +
// (its rank inside its own segment), which preserves (token, slot) order.
// It also writes one record per active expert (ws.slots: id, first position,
// pair count, token of the first pair) for the expert kernels.
// LDS: s_ids[P] ids, s_rank[P], s_wcnt[NWV*E], s_cnt[E], s_off[E], s_aidx[E].
template <int NWV>
__device__ void build_routing_tables(const int* s_ids, int P, int E, int K, MoeWs ws, int* s_cnt, int* s_off, int* s_rank,
                                     int* s_wcnt, int* s_aidx) {
  constexpr int NTH = NWV * kWave;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  __shared__ int s_wtot[NWV][2];
  for (int i = tid; i < NWV * E; i += NTH) s_wcnt[i] = 0;
  __syncthreads();

  const int seg = (P + NWV - 1) / NWV;
  const int j0 = min(P, wave * seg), j1 = min(P, j0 + seg);
  int* wc = s_wcnt + wave * E;
  for (int c0 = j0; c0 < j1; c0 += kWave) {
    const int j = c0 + lane;
    const bool valid = j < j1;
    const int e = valid ? s_ids[j] : -1;
    const int n = min(kWave, j1 - c0);
    int below = 0, total = 0;
    for (int src = 0; src < n; ++src) {
      const int v = __builtin_amdgcn_readlane(e, src);
      below += (v == e) & (src < lane);
      total += (v == e);
    }
    int before = 0;
    if (valid) {
      before = wc[e];
      s_rank[j] = before + below;
    }
    // One lane per expert of the chunk (its last occurrence) advances the
    // running count; LDS operations of one wavefront complete in order.
    if (valid && below == total - 1) wc[e] = before + total;
  }
  __syncthreads();

  // Per-expert totals, and per-wave exclusive prefixes in place.
  for (int e = tid; e < E; e += NTH) {
    int run = 0;
    for (int w = 0; w < NWV; ++w) {
      const int c = s_wcnt[w * E + e];
      s_wcnt[w * E + e] = run;
      run += c;
    }
    s_cnt[e] = run;
  }
  __syncthreads();

  const int per = (E + NTH - 1) / NTH;  // bins per thread (<= 4)
  const int base = tid * per;
  int sum = 0, nz = 0;
  for (int q = 0; q < per; ++q) {
    int e = base + q;
    if (e < E) {
      sum += s_cnt[e];
      nz += s_cnt[e] > 0;
    }
  }
  int isum = wave_incl_scan(sum, lane);
  int inz = wave_incl_scan(nz, lane);
  if (lane == 63) {
    s_wtot[wave][0] = isum;
    s_wtot[wave][1] = inz;
  }
  __syncthreads();
  int psum = 0, pnz = 0;
  for (int w = 0; w < wave; ++w) {
    psum += s_wtot[w][0];
    pnz += s_wtot[w][1];
  }
  int run = psum + isum - sum;
  int runnz = pnz + inz - nz;
  for (int q = 0; q < per; ++q) {
    int e = base + q;
    if (e < E) {
      int c = s_cnt[e];
      s_off[e] = run;
      ws.offsets[e] = run;
      ws.counts[e] = c;
      if (c > 0) {
        ws.active[runnz] = e;
        ws.slots[runnz] = make_int4(e, run, c, 0);
        s_aidx[e] = runnz++;
      }
      run += c;
    }
  }
  if (tid == 0) {
    ws.offsets[E] = P;
    int na = 0;
    for (int w = 0; w < NWV; ++w) na += s_wtot[w][1];
    ws.num_active[0] = na;
  }
  __syncthreads();
  for (int j = tid; j < P; j += NTH) {
    const int w = j / seg;
    const int e = s_ids[j];
    const int r = s_off[e] + s_wcnt[w * E + e] + s_rank[j];
    ws.perm[r] = j;
    ws.inverse[j] = r;
    if (r == s_off[e]) ws.slots[s_aidx[e]].w = j / K;  // the expert's first pair
  }
}

// ---------------------------------------------------------------------------
// 1. Router
// ---------------------------------------------------------------------------
struct RouterArgs {
  const void* x;
  const void* nw;
  const void* W;
  const void* bias;
  int nw_dt, bias_dt;
  int T, H, E, K;
  int tu;  // tokens per workgroup of the small-batch router (set by its launcher)
  float eps, off;
  float* logits;
  int64_t* ids_out;
  float* w_out;
  MoeWs ws;
};

// Wave-wide reductions for the selection: DPP within each 16-lane row, then
// the four row results read into scalar registers and combined there (a
// uniform result, no lane swaps on the critical path of a lone wavefront).
__device__ __forceinline__ uint32_t wave_max_u32_rows(uint32_t v) {
  v = max(v, dpp_u32<kDppQuadXor1>(v));
  v = max(v, dpp_u32<kDppQuadXor2>(v));
  v = max(v, dpp_u32<kDppRowHalfMirror>(v));
  v = max(v, dpp_u32<kDppRowMirror>(v));
  const uint32_t r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
  const uint32_t r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
  return max(max(r0, r1), max(r2, r3));
}
__device__ __forceinline__ float wave_max_rows(float v) {
  v = fmaxf(v, __uint_as_float(dpp_u32<kDppQuadXor1>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp_u32<kDppQuadXor2>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp_u32<kDppRowHalfMirror>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp_u32<kDppRowMirror>(__float_as_uint(v))));
  const float r0 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 0));
  const float r1 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 16));
  const float r2 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 32));
  const float r3 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}
__device__ __forceinline__ float wave_sum_rows(float v) {
  v += __uint_as_float(dpp_u32<kDppQuadXor1>(__float_as_uint(v)));
  v += __uint_as_float(dpp_u32<kDppQuadXor2>(__float_as_uint(v)));
  v += __uint_as_float(dpp_u32<kDppRowHalfMirror>(__float_as_uint(v)));
  v += __uint_as_float(dpp_u32<kDppRowMirror>(__float_as_uint(v)));
  const float r0 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 0));
  const float r1 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 16));
  const float r2 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 32));
  const float r3 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 48));
  return (r0 + r1) + (r2 + r3);
}

// Softmax + top-k over logits held in registers (lane l holds experts
// l + 64 j; -inf where l + 64 j >= E).  Candidate (p, j) of a lane becomes
// the 32-bit key ((bits(p) + 1) << 2) | (3 - j): probabilities lie in [0, 1],
// so bits(p) + 1 <= 0x3F800001 and the key fits; 0 marks "no expert" or
// "taken".  Keys order by probability, then by lower j; two lanes can only
// hold equal keys for equal p and j, and then the lower lane has the lower
// expert id.  Each round takes the wave-wide maximum key and the lowest lane
// holding it, so experts are taken in (probability desc, expert id asc)
// order.  Each lane keeps its keys sorted, so giving up its head is a shift.
// Lane k < K ends with the k-th selection; weights are renormalised by the
// sum of the selected probabilities in selection order.
// NT tokens at once (token i in p[i]): the tokens' chains are independent,
// so their reductions interleave instead of running back to back.
// Softmax of NT tokens' logits and their 32-bit keys (the prologue of the
// selections below): p[i][j] becomes the probability of expert l + 64 j.
template <int NT>
__device__ __forceinline__ void softmax_keys32(float (&p)[NT][4], int E, int lane, uint32_t (&key)[NT][4]) {
  float m[NT], s[NT];
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    m[i] = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) m[i] = fmaxf(m[i], p[i][j]);
  }
#pragma unroll
  for (int i = 0; i < NT; ++i) m[i] = wave_max_rows(m[i]);
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    s[i] = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int ex = lane + kWave * j;
      p[i][j] = ex < E ? expf(p[i][j] - m[i]) : 0.f;
      s[i] += p[i][j];
    }
  }
#pragma unroll
  for (int i = 0; i < NT; ++i) s[i] = wave_sum_rows(s[i]);
#pragma unroll
  for (int i = 0; i < NT; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      p[i][j] = p[i][j] / s[i];
      key[i][j] = lane + kWave * j < E ? ((__float_as_uint(p[i][j]) + 1u) << 2) | (uint32_t)(3 - j) : 0u;
    }
}

// The K rounds of the selection on the keys of softmax_keys32.
template <int NT>
__device__ void select_rounds32(uint32_t (&key)[NT][4], int K, int lane, int (&out_id)[NT], float (&out_w)[NT]) {
  auto cswap = [](uint32_t& a, uint32_t& b) {
    const uint32_t hi = a > b ? a : b, lo = a > b ? b : a;
    a = hi;
    b = lo;
  };
  float denom[NT], my_v[NT];
  int my_id[NT];
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    // Sort the lane's keys descending (keys are distinct within a lane).
    cswap(key[i][0], key[i][1]);
    cswap(key[i][2], key[i][3]);
    cswap(key[i][0], key[i][2]);
    cswap(key[i][1], key[i][3]);
    cswap(key[i][1], key[i][2]);
    denom[i] = 0.f;
    my_id[i] = 0;
    my_v[i] = 0.f;
  }
  for (int k = 0; k < K; ++k) {
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      const uint32_t mk = wave_max_u32_rows(key[i][0]);
      const int sel_lane = __ffsll((unsigned long long)__ballot(key[i][0] == mk)) - 1;
      const int sel = sel_lane + kWave * (int)(3 - (mk & 3u));
      const float mv = __uint_as_float((mk >> 2) - 1u);
      const bool own = lane == sel_lane;
      key[i][0] = own ? key[i][1] : key[i][0];
      key[i][1] = own ? key[i][2] : key[i][1];
      key[i][2] = own ? key[i][3] : key[i][2];
      key[i][3] = own ? 0u : key[i][3];
      denom[i] += mv;
      if (lane == k) {
        my_id[i] = sel;
        my_v[i] = mv;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    out_id[i] = my_id[i];
    out_w[i] = my_v[i] / denom[i];
  }
}

template <int NT>
__device__ void topk_select_keys32_multi(float (&p)[NT][4], int E, int K, int lane, int (&out_id)[NT],
                                         float (&out_w)[NT]) {
  uint32_t key[NT][4];
  softmax_keys32<NT>(p, E, lane, key);
  select_rounds32<NT>(key, K, lane, out_id, out_w);
}

// LDS of topk_select_ranked (one wavefront's).
struct TopkLds {
  uint64_t cand[kWave];
};

// Order-preserving 32-bit key of a logit (-0 folded into +0, so equal
// logits have equal keys), and back.  0 is left for "no expert" (only a
// negative NaN with every payload bit set would map there; it takes 1).
__device__ __forceinline__ uint32_t logit_key(float l) {
  const uint32_t u = __float_as_uint(l + 0.0f);
  const uint32_t k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return k ? k : 1u;
}
__device__ __forceinline__ float key_logit(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Top-k of one token for E <= 256 (lane l holds the logits of experts
// l + 64 j, j < 4; any value where l + 64 j >= E) without K dependent
// wavefront maxima.  The softmax is increasing, so the experts are selected
// on their logits, in (logit desc, expert id asc) order: equal logits are
// equal probabilities and go to the lower id.  (Two different logits can
// round to one probability; which of them the reference takes is rounding,
// not its tie rule.)
//  1. threshold: tau = the smallest of the eight 8-lane groups' maximum
//     32-bit keys.  The eight group maxima are eight experts with key >=
//     tau, so each of the top K <= 8 has key >= tau (with a group holding no
//     expert, tau = 0 and every expert is a candidate).  The same chain of
//     lane swaps gives the largest key, the top logit.
//  2. rank: the candidates are compacted into LDS (ballot prefix counts)
//     with distinct 64-bit keys key << 32 | ~id, one per lane; a candidate's
//     rank is the number of larger keys, and rank r < K is selection r.
// More than 64 candidates (many equal logits) take K rounds of wavefront
// maxima of the same 64-bit keys instead.  Weights: w_k = e_k / sum_j e_j,
// e_j = exp(l_j - l_max) over the K selected logits (the renormalised
// softmax probabilities: the softmax denominator cancels), the sum over the
// selected lanes in a fixed lane order.  Selection r is written to
// sel_id[r] and sel_w[r] (the caller's LDS, visible after its barrier).
__device__ void topk_select_ranked(const float (&l)[4], int E, int K, int lane, TopkLds* lds, int* sel_id,
                                   float* sel_w) {
  uint32_t key[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) key[j] = lane + kWave * j < E ? logit_key(l[j]) : 0u;
  uint32_t gm = max(max(key[0], key[1]), max(key[2], key[3]));
  gm = max(gm, dpp_u32<kDppQuadXor1>(gm));
  gm = max(gm, dpp_u32<kDppQuadXor2>(gm));
  gm = max(gm, dpp_u32<kDppRowHalfMirror>(gm));
  const uint32_t gmo = dpp_u32<kDppRowMirror>(gm);
  uint32_t tau = min(gm, gmo), top = max(gm, gmo);
  tau = min(tau, xor16_u32(tau));
  top = max(top, xor16_u32(top));
  tau = min(tau, xor32_u32(tau));
  top = max(top, xor32_u32(top));
  const float lmax = key_logit(top);
  bool c[4];
  int pos[4];
  int C = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    c[j] = key[j] != 0u && key[j] >= tau;
    const uint64_t mask = __ballot(c[j]);
    pos[j] = C + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
    C += __popcll(mask);
  }
  C = __builtin_amdgcn_readfirstlane(C);
  uint64_t mine = 0;  // this lane's selection or candidate (64-bit key)
  int rank = K;       // its position, K: none
  if (C > kWave) {
    // K rounds: each takes the largest remaining 64-bit key of the wavefront.
    uint64_t k64[4];
    uint64_t head = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      k64[j] = key[j] ? ((uint64_t)key[j] << 32) | (uint32_t)~(lane + kWave * j) : 0ull;
      head = max_u64(head, k64[j]);
    }
    for (int k = 0; k < K; ++k) {
      const uint64_t mk = wave_max_u64(head);
      if (head == mk) {
        head = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          k64[j] = k64[j] == mk ? 0ull : k64[j];
          head = max_u64(head, k64[j]);
        }
      }
      if (lane == k) {
        mine = mk;
        rank = k;
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (c[j]) lds->cand[pos[j]] = ((uint64_t)key[j] << 32) | (uint32_t)~(lane + kWave * j);
    if (lane >= C) lds->cand[lane] = 0ull;  // pads the last group of eight
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    mine = lds->cand[lane];
    int r = 0;
    for (int i = 0; i < C; i += 8) {
      uint64_t kk[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) kk[q] = lds->cand[i + q];
#pragma unroll
      for (int q = 0; q < 8; ++q) r += (int)(kk[q] > mine);
    }
    rank = lane < C ? r : K;
  }
  const bool sel = rank < K;
  const float e = expf(key_logit((uint32_t)(mine >> 32)) - lmax);
  const float denom = wave_sum(sel ? e : 0.f);
  if (sel) {
    sel_id[rank] = min(max((int)~(uint32_t)mine, 0), E - 1);
    sel_w[rank] = e / denom;
  }
}

template <int NJE>
__device__ void topk_select_keys32(float (&p)[NJE], int E, int K, int lane, int& out_id, float& out_w) {
  static_assert(NJE == 4, "keys carry j in two bits");
  float pm[1][4] = {{p[0], p[1], p[2], p[3]}};
  int id[1];
  float w[1];
  topk_select_keys32_multi<1>(pm, E, K, lane, id, w);
  out_id = id[0];
  out_w = w[0];
}

// Same selection with 64-bit keys (bits(p) << 32 | ~expert id), for lanes
// holding more than 4 candidates (E > 256).
template <int NJE>
__device__ void topk_select_keys64(float (&p)[NJE], int E, int K, int lane, int& out_id, float& out_w) {
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < NJE; ++j) m = fmaxf(m, p[j]);
  m = wave_max(m);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NJE; ++j) {
    const int ex = lane + kWave * j;
    p[j] = ex < E ? expf(p[j] - m) : 0.f;
    s += p[j];
  }
  s = wave_sum(s);
  uint64_t key[NJE];
  uint64_t head = 0;
#pragma unroll
  for (int j = 0; j < NJE; ++j) {
    const int ex = lane + kWave * j;
    key[j] = ex < E ? ((uint64_t)__float_as_uint(p[j] / s) << 32) | (uint32_t)~ex : 0ull;
    head = max_u64(head, key[j]);
  }
  float denom = 0.f;
  int my_id = 0;
  float my_v = 0.f;
  for (int k = 0; k < K; ++k) {
    const uint64_t mk = wave_max_u64(head);
    if (head == mk) {
      head = 0;
#pragma unroll
      for (int j = 0; j < NJE; ++j) {
        key[j] = key[j] == mk ? 0ull : key[j];
        head = max_u64(head, key[j]);
      }
    }
    const float mv = __uint_as_float((uint32_t)(mk >> 32));
    denom += mv;
    if (lane == k) {
      my_id = (int)~(uint32_t)mk;
      my_v = mv;
    }
  }
  out_id = my_id;
  out_w = my_v / denom;
}

template <int NJE>
__device__ void topk_select_regs(float (&p)[NJE], int E, int K, int lane, int& out_id, float& out_w) {
  if constexpr (NJE == 4) topk_select_keys32<NJE>(p, E, K, lane, out_id, out_w);
  else topk_select_keys64<NJE>(p, E, K, lane, out_id, out_w);
}

template <int NJE>
__device__ void topk_select(const float* row, int E, int K, int lane, int& out_id, float& out_w) {
  float p[NJE];
#pragma unroll
  for (int j = 0; j < NJE; ++j) {
    const int ex = lane + kWave * j;
    p[j] = ex < E ? load_coherent(row + ex) : -INFINITY;
  }
  topk_select_regs<NJE>(p, E, K, lane, out_id, out_w);
}

// Softmax + top-k of one token by one wavefront: lane k < K ends with the
// k-th selection.  Lane l owns experts l + 64 j; each lane keeps its best
// remaining candidate ("head": highest probability, lowest id on ties) and
// every round takes the wave maximum of the heads, breaking probability ties
// toward the lowest expert id.  Weights are renormalised by the sum of the
// selected probabilities in selection order.  `bad`: the logits may be
// incomplete (a failed wait): ids are clamped in range, weights are NaN.
template <int NJE>
__device__ void router_topk_token(const RouterArgs& a, int t, int lane, bool bad) {
  int id;
  float w;
  topk_select<NJE>(a.logits + (size_t)t * a.E, a.E, a.K, lane, id, w);
  if (bad) {
    id = min(max(id, 0), a.E - 1);
    w = poison_if(true, w);
  }
  if (lane < a.K) {
    const size_t o = (size_t)t * a.K + lane;
    a.ids_out[o] = id;
    a.w_out[o] = w;
    store_coherent(a.ws.ids32 + o, id);
    a.ws.wts[o] = w;
  }
}

// Router.  Grid (ceil(E/4), token tiles), capped by the host at the number
// of co-resident workgroups.  Phase 1: one wavefront per expert row (weights
// folded with the norm weight, in registers) over the tile's tokens in
// batches of 4.  Grid barrier.  Phase 2: one wavefront per token runs
// softmax/top-k.  Phase 3: the last workgroup to finish builds the routing
// tables.  Cross-workgroup data moves through coherent stores/loads and
// device-scope tickets (no cache-wide fences).
template <bool BFW, bool BFX, int NJ, int NJE>
__global__ __launch_bounds__(256) void moe_router_kernel(RouterArgs a) {
  __shared__ int s_ids[kMaxPairs];
  __shared__ int s_rank[kMaxPairs];
  __shared__ int s_wcnt[4 * kMaxExperts];
  __shared__ int s_cnt[kMaxExperts];
  __shared__ int s_off[kMaxExperts];
  __shared__ int s_aidx[kMaxExperts];
  __shared__ int s_last;
  __shared__ int s_bad;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e = blockIdx.x * 4 + wave;
  WaitHeader hdr = load_wait_header(a.ws.tickets, kTicketEpoch);  // (limit taken at the barrier)
  const int nch = a.H >> 3;
  const int tile = (a.T + gridDim.y - 1) / gridDim.y;
  const int tb = blockIdx.y * tile;
  const int te = min(a.T, tb + tile);

  if (e < a.E && tb < te) {
    float wn[NJ][8];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int c = lane + kWave * j;
      if (c < nch) {
        float w8[8], n8[8];
        load8_f32<BFW>(a.W, (size_t)e * a.H + (size_t)c * 8, w8);
        load8_any(a.nw, a.nw_dt, (size_t)c * 8, n8);
#pragma unroll
        for (int q = 0; q < 8; ++q) wn[j][q] = w8[q] * (a.off + n8[q]);
      } else {
#pragma unroll
        for (int q = 0; q < 8; ++q) wn[j][q] = 0.f;
      }
    }
    const float bias = a.bias ? load_scalar(a.bias, a.bias_dt, e) : 0.f;
    // Lane (t - tb) keeps token t's logit and all lanes store once at the end:
    // write-through stores inside the loop would hold up the next batch's
    // loads (the vector-memory counter retires in order).
    const bool defer = te - tb <= kWave;
    float mine = 0.f;
    constexpr int TB = 4;  // tokens per batch: independent loads and reductions
    for (int t0 = tb; t0 < te; t0 += TB) {
      float ss[TB], d[TB];
#pragma unroll
      for (int tt = 0; tt < TB; ++tt) {
        ss[tt] = 0.f;
        d[tt] = 0.f;
        const int t = t0 + tt;
        if (t < te) {
#pragma unroll
          for (int j = 0; j < NJ; ++j) {
            const int c = lane + kWave * j;
            if (c < nch) {
              float x8[8];
              load8_f32<BFX>(a.x, (size_t)t * a.H + (size_t)c * 8, x8);
#pragma unroll
              for (int q = 0; q < 8; ++q) {
                ss[tt] = fmaf(x8[q], x8[q], ss[tt]);
                d[tt] = fmaf(x8[q], wn[j][q], d[tt]);
              }
            }
          }
        }
      }
#pragma unroll
      for (int tt = 0; tt < TB; ++tt) {
        ss[tt] = wave_sum(ss[tt]);
        d[tt] = wave_sum(d[tt]);
      }
#pragma unroll
      for (int tt = 0; tt < TB; ++tt) {
        const int t = t0 + tt;
        if (t >= te) continue;
        const float logit = d[tt] * rsqrtf(ss[tt] / (float)a.H + a.eps) + bias;
        if (defer) {
          mine = lane == t - tb ? logit : mine;
        } else if (lane == 0) {
          store_coherent(a.logits + (size_t)t * a.E + e, logit);
        }
      }
    }
    if (defer && lane < te - tb) store_coherent(a.logits + (size_t)(tb + lane) * a.E + e, mine);
  }

  const uint32_t G = gridDim.x * gridDim.y;
  publish_wait();
  __syncthreads();
  const uint32_t spin = hdr.limits().spin;
  if (threadIdx.x == 0)
    s_bad = !grid_arrive_and_wait(&a.ws.tickets[kTicketRouterBarrier], G, &a.ws.tickets[kTicketError], spin);
  __syncthreads();
  const bool bad = s_bad;

  const int gw = (blockIdx.y * gridDim.x + blockIdx.x) * 4 + wave;
  for (int t = gw; t < a.T; t += (int)G * 4) router_topk_token<NJE>(a, t, lane, bad);

  publish_wait();
  __syncthreads();
  if (threadIdx.x == 0) s_last = ticket_add(&a.ws.tickets[kTicketRouterTables]) == G - 1;
  __syncthreads();
  if (!s_last) return;
  const int P = a.T * a.K;
  for (int j = threadIdx.x; j < P; j += 256) s_ids[j] = load_coherent(a.ws.ids32 + j);
  __syncthreads();
  build_routing_tables<4>(s_ids, P, a.E, a.K, a.ws, s_cnt, s_off, s_rank, s_wcnt, s_aidx);
  if (threadIdx.x == 0) {
    // Every workgroup has passed the barrier (it counted into ticket 1).
    a.ws.tickets[kTicketRouterBarrier] = 0u;
    a.ws.tickets[kTicketRouterTables] = 0u;
  }
}

// Routing tables from caller-supplied ids (single workgroup).
struct AlignArgs {
  const void* ids;
  int ids_dt;
  const void* w;
  int w_dt;
  int T, K, E;
  MoeWs ws;
  int32_t* counts_out;
  int32_t* offsets_out;
  int32_t* perm_out;
  int32_t* inverse_out;
};

__global__ __launch_bounds__(256) void moe_align_kernel(AlignArgs a) {
  __shared__ int s_ids[kMaxPairs];
  __shared__ int s_rank[kMaxPairs];
  __shared__ int s_wcnt[4 * kMaxExperts];
  __shared__ int s_cnt[kMaxExperts];
  __shared__ int s_off[kMaxExperts];
  __shared__ int s_aidx[kMaxExperts];
  const int P = a.T * a.K;
  for (int j = threadIdx.x; j < P; j += 256) {
    long long v = a.ids_dt == FK_DTYPE_I64 ? reinterpret_cast<const long long*>(a.ids)[j]
                                           : (long long)reinterpret_cast<const int*>(a.ids)[j];
    int e = (int)(v < 0 ? 0 : (v >= a.E ? a.E - 1 : v));
    s_ids[j] = e;
    a.ws.ids32[j] = e;
    a.ws.wts[j] = a.w ? load_scalar(a.w, a.w_dt, j) : 0.f;
  }
  __syncthreads();
  build_routing_tables<4>(s_ids, P, a.E, a.K, a.ws, s_cnt, s_off, s_rank, s_wcnt, s_aidx);
  __syncthreads();
  // Optional copies of the tables for callers that inspect them.
  for (int e = threadIdx.x; e < a.E; e += 256) {
    if (a.counts_out) a.counts_out[e] = s_cnt[e];
    if (a.offsets_out) a.offsets_out[e] = s_off[e];
  }
  if (threadIdx.x == 0 && a.offsets_out) a.offsets_out[a.E] = P;
  if (a.perm_out || a.inverse_out) {
    __threadfence_block();
    __syncthreads();
    for (int j = threadIdx.x; j < P; j += 256) {
      if (a.perm_out) a.perm_out[j] = a.ws.perm[j];
      if (a.inverse_out) a.inverse_out[j] = a.ws.inverse[j];
    }
  }
}

// ---------------------------------------------------------------------------
// 2./3. Expert stage
// ---------------------------------------------------------------------------
struct ExpertArgs {
  const void* x;
  int x_dt;
  const void* gu;
  const void* dn;
  const void* sgu;
  const void* sdn;
  const void* sg;
  int sg_dt;
  int T, H, I, E, K;
  int has_shared;
  float* out;
  float* layer_out;
  MoeWs ws;
};

template <bool BFW, bool BFX, int NJ>
__global__ __launch_bounds__(256) void moe_gateup_kernel(ExpertArgs a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int chunks = a.I / kGateUpRows;
  int slot = blockIdx.x / chunks;
  const int chunk = blockIdx.x - slot * chunks;
  const int P = a.T * a.K;
  const size_t esz = BFW ? 2 : 4;

  const char* W;
  bool shared = false;
  int pos0, npairs, t = 0;  // t: token of the first pair
  if (a.has_shared && slot == 0) {
    W = reinterpret_cast<const char*>(a.sgu);
    shared = true;
    pos0 = P;
    npairs = a.T;
  } else {
    if (a.has_shared) slot -= 1;
    // The active count and this slot's record (slot < E) are loaded
    // together: one round trip before the weights can be fetched.
    const int na = a.ws.num_active[0];
    const int4 rec = a.ws.slots[slot];
    if (slot >= na) return;
    W = reinterpret_cast<const char*>(a.gu) + (size_t)rec.x * 2 * a.I * a.H * esz;
    pos0 = rec.y;
    npairs = rec.z;
    t = rec.w;
  }

  const int nch = a.H >> 3;
  const int i0 = chunk * kGateUpRows + wave * 2;  // this wave's two intermediates
  const size_t rows[4] = {(size_t)i0, (size_t)i0 + 1, (size_t)a.I + i0, (size_t)a.I + i0 + 1};

  // The first pair's token chunks are issued first (clamped in range), then
  // the four rows (gate i0, gate i0+1, up i0, up i0+1), streamed once: the
  // compiler converts the rows before the pair loop, and chunks issued
  // after them would wait for that.  Each later pair costs one round trip
  // (its chunks are loaded together while its token index is fetched).
  Raw8<BFX> xr[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) xr[j] = load_raw8<BFX>(a.x, (size_t)t * a.H + (size_t)min(lane + kWave * j, nch - 1) * 8);
  Raw8<BFW> wr[4][NJ];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int c = lane + kWave * j;
      if (c < nch) wr[r][j] = load_raw8_stream<BFW>(W, rows[r] * a.H + (size_t)c * 8);
    }
  }

  for (int pp = 0; pp < npairs; ++pp) {
    const int pos = pos0 + pp;
    int t_next = 0;
    if (pp + 1 < npairs) t_next = shared ? pp + 1 : a.ws.perm[pos + 1] / a.K;
    // The rows are converted to fp32 where they are used, once per pair:
    // hoisted out of this loop the converted rows would double the
    // registers the rows take and cost a wavefront per SIMD.
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int j = 0; j < NJ; ++j) asm volatile("" : "+v"(wr[r][j].a));
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int c = lane + kWave * j;
      if (c < nch) {
        float x8[8];
        raw8_to_f32<BFX>(xr[j], x8);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float w8[8];
          raw8_to_f32<BFW>(wr[r][j], w8);
#pragma unroll
          for (int q = 0; q < 8; ++q) acc[r] = fmaf(w8[q], x8[q], acc[r]);
        }
      }
    }
    // the four row sums at once (lanes 16r ..: row r), gathered in lane 0
    const float rs = rows4_sum(acc);
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(rs), 16 * r));
    if (lane == 0) {
      float2 v = make_float2(silu(acc[0]) * acc[2], silu(acc[1]) * acc[3]);
      *reinterpret_cast<float2*>(a.ws.act + (size_t)pos * a.I + i0) = v;
    }
    if (pp + 1 < npairs) {
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        xr[j] = load_raw8<BFX>(a.x, (size_t)t_next * a.H + (size_t)min(lane + kWave * j, nch - 1) * 8);
    }
  }

  // Shared-expert gate sigmoid(w_g . x_t), once per token.
  if (shared && chunk == 0 && a.sg) {
    // (a 16-byte aligned gate weight is read 8 elements per load)
    const bool sg_bf = a.sg_dt == FK_DTYPE_BF16, sg_vec = (reinterpret_cast<uintptr_t>(a.sg) & 15u) == 0;
    for (int t = wave; t < a.T; t += 4) {
      float d = 0.f;
      for (int c = lane; c < nch; c += kWave) {
        float x8[8], g8[8];
        load8_f32<BFX>(a.x, (size_t)t * a.H + (size_t)c * 8, x8);
        if (sg_vec && sg_bf) load8_f32<true>(a.sg, (size_t)c * 8, g8);
        else if (sg_vec) load8_f32<false>(a.sg, (size_t)c * 8, g8);
        else
#pragma unroll
          for (int q = 0; q < 8; ++q) g8[q] = load_scalar(a.sg, a.sg_dt, (size_t)c * 8 + q);
#pragma unroll
        for (int q = 0; q < 8; ++q) d = fmaf(x8[q], g8[q], d);
      }
      d = wave_sum(d);
      if (lane == 0) a.ws.sgate[t] = sigmoid(d);
    }
  }
}

// Down projection, expert-major.  Workgroup (slot, row chunk) streams 16
// contiguous rows of the slot's down matrix (4 per wavefront, one 16-byte
// load per lane per row at I=512, all issued before use) and, for every pair
// routed to the slot, writes y[pos, row] = W_d[e][row] . act[pos].
template <bool BFW, int NJI>
__global__ __launch_bounds__(256) void moe_down_kernel(ExpertArgs a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int chunks = (a.H + kDownRows - 1) / kDownRows;
  int slot = blockIdx.x / chunks;
  const int chunk = blockIdx.x - slot * chunks;
  const int P = a.T * a.K;
  const size_t esz = BFW ? 2 : 4;
  const char* W;
  int pos0, npairs;
  if (a.has_shared && slot == 0) {
    W = reinterpret_cast<const char*>(a.sdn);
    pos0 = P;
    npairs = a.T;
  } else {
    if (a.has_shared) slot -= 1;
    const int na = a.ws.num_active[0];  // loaded with the record (slot < E)
    const int4 rec = a.ws.slots[slot];
    if (slot >= na) return;
    W = reinterpret_cast<const char*>(a.dn) + (size_t)rec.x * a.H * a.I * esz;
    pos0 = rec.y;
    npairs = rec.z;
  }
  const int nci = a.I >> 3;
  const int r0 = chunk * kDownRows + wave * kDownRowsPerWave;
  constexpr int R = kDownRowsPerWave;

  // Activation rows: the first pair's is issued before the weights, each
  // later pair's is fetched while the previous pair is computed (chunks
  // clamped in range, out-of-range ones unused).
  float av[NJI][8];
#pragma unroll
  for (int j = 0; j < NJI; ++j) load8_act(a.ws.act, (size_t)pos0 * a.I + (size_t)min(lane + kWave * j, nci - 1) * 8, av[j]);
  Raw8<BFW> wr[R][NJI];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < NJI; ++j) {
      const int c = lane + kWave * j;
      if (c < nci && r0 + r < a.H) wr[r][j] = load_raw8_stream<BFW>(W, (size_t)(r0 + r) * a.I + (size_t)c * 8);
    }

  for (int pp = 0; pp < npairs; ++pp) {
    const int pos = pos0 + pp;
    // rows converted where used (as in the gate/up kernel).  Four rows per
    // wavefront keep it at 49 registers and eight wavefronts per SIMD: at
    // eight or sixteen rows per wavefront (fewer, longer streams, 4-6
    // wavefronts per SIMD) the T = 16 expert stage measured 2-12 us slower.
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int j = 0; j < NJI; ++j) asm volatile("" : "+v"(wr[r][j].a));
    float an[NJI][8];
    if (pp + 1 < npairs) {
#pragma unroll
      for (int j = 0; j < NJI; ++j)
        load8_act(a.ws.act, (size_t)(pos + 1) * a.I + (size_t)min(lane + kWave * j, nci - 1) * 8, an[j]);
    }
    float d[R];
#pragma unroll
    for (int r = 0; r < R; ++r) d[r] = 0.f;
#pragma unroll
    for (int j = 0; j < NJI; ++j) {
      const int c = lane + kWave * j;
      if (c < nci) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (r0 + r < a.H) {
            float w8[8];
            raw8_to_f32<BFW>(wr[r][j], w8);
#pragma unroll
            for (int q = 0; q < 8; ++q) d[r] = fmaf(w8[q], av[j][q], d[r]);
          }
        }
      }
    }
    if (pp + 1 < npairs) {
#pragma unroll
      for (int j = 0; j < NJI; ++j)
#pragma unroll
        for (int q = 0; q < 8; ++q) av[j][q] = an[j][q];
    }
    // the four row sums at once: lanes 16r .. 16r + 15 hold row r0 + r
    static_assert(R == 4, "rows4_sum sums four rows");
    const float v = rows4_sum(d);
    if ((lane & 15) == 0 && r0 + (lane >> 4) < a.H) a.ws.y[(size_t)pos * a.H + r0 + (lane >> 4)] = v;
  }
}

// out[t, h] = sum_k w[t,k] * y[pos(t,k), h]  (slot order k = 0..K-1)
//             + g_t * y[P + t, h]            (shared expert, g_t = sigmoid(w_g . x_t) or 1)
// layer_out = x + out (LO: layer_out is written).  BFX: bf16 hidden
// states.  Every load is issued
// before the first use, in two dependent rounds (slot positions, weights,
// gate and residual input; then the K + 1 rows of y), with indices clamped
// in range and unused values dropped: a loop over the slots would make
// each slot wait for its position and then for its y value.  While the
// workspace's error word is set (a wait of the router that built the
// tables ran out, now or in an earlier uncleared call) the outputs are NaN.
template <bool BFX, bool LO>
__global__ __launch_bounds__(256) void moe_combine_kernel(ExpertArgs a) {
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t total = (size_t)a.T * a.H;
  const bool bad = load_coherent(&a.ws.tickets[kTicketError]) != 0u;
  if (idx >= total) return;
  const int t = (int)(idx / a.H);
  const int h = (int)(idx - (size_t)t * a.H);
  const int K = a.K, P = a.T * K;  // K <= 8 (host checks)
  int inv[8];
  float wk[8], yv[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int pair = t * K + min(k, K - 1);
    inv[k] = a.ws.inverse[pair];
    wk[k] = a.ws.wts[pair];
  }
  const float g = a.ws.sgate[t];
  uint32_t xr[1];
  if constexpr (LO) gather_raw<BFX>(a.x, idx, 0, 1, xr);
#pragma unroll
  for (int k = 0; k < 8; ++k) yv[k] = a.ws.y[(size_t)inv[k] * a.H + h];
  const float ys = a.ws.y[(size_t)(P + (a.has_shared ? t : 0)) * a.H + h];
  float acc = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k)
    if (k < K) acc += wk[k] * yv[k];
  if (a.has_shared) acc += (a.sg ? g : 1.f) * ys;
  acc = poison_if(bad, acc);
  a.out[idx] = acc;
  if constexpr (LO) a.layer_out[idx] = raw_value<BFX>(xr[0]) + acc;
}

// ---------------------------------------------------------------------------
// Batched expert stage (T >= 44 tokens, bf16 weights and hidden states):
// MFMA grouped GEMM over the routing tables.
//
// Weight rows are loaded row-contiguously (a wavefront's K range of a row
// is LPR lanes x 16 B, RPI rows per load: the MFMA operand layout, 16 rows x
// 64 B per load, streams at half the rate) and each wavefront turns them
// into v_mfma_f32_16x16x32_bf16 A operands (lane l: row l % 16, k group
// l / 16 of each 32-wide step) once, through its own LDS area; the tokens of
// an expert then go through in tiles of 16 columns, each tile one MFMA per
// 32-wide step and row tile, and the wavefronts' partial tiles are summed
// in a fixed order through LDS.
//   gate/up: work item (slot, 16 intermediates) = 16 gate + 16 up rows, 512
//            threads, K = H split over the 8 wavefronts; the tokens are the
//            bf16 hidden states themselves (exact products).
//   down:    work item (slot, 32 or 64 output rows), 256 threads, K = I split over
//            the 4 wavefronts; fp32 activations enter as bf16 hi + lo
//            columns (8 pairs per tile, ~16 mantissa bits).
// ---------------------------------------------------------------------------
// From this many tokens the MFMA expert kernels replace the GEMV ones (model
// shapes: equal at 40 tokens, 1.2 us faster at 48, 3.3 at 56, 7.7 at 63).
constexpr int kMfmaMinTokens = 44;
constexpr int kGuMfmaRows = 16;   // intermediates per gate/up work item
// Output rows per down work item: 32 while the routed experts average at
// most kDnMfmaSmallPairs pairs (one tile of 8 pairs for most of them), else
// 64.  Smaller items stream their 32 KB sooner (T=64 76.6 -> 71.3 us, T=128
// 88.8 -> 85.7 us at the model's shapes); with more tiles per item the
// per-tile reduction and the activation reads, which grow with the number
// of items, cost more (T=256 99.8 -> 106.2 us), so 64 rows stay there.
constexpr int kDnMfmaRowsSmall = 32;
constexpr int kDnMfmaRows = 64;
constexpr int kDnMfmaSmallPairs = 4;
constexpr int kGuMfmaWaves = 8;
constexpr int kDnMfmaWaves = 4;

// Shapes the MFMA kernels take (powers of two, so lane splits are shifts).
static bool mfma_expert_shapes_ok(int H, int I) {
  return (H == 512 || H == 1024 || H == 2048) && (I == 256 || I == 512);
}

// Row-contiguous registers v[s] (instruction s: row s*RPI + lane/LPR, 16 B
// at k = (lane % LPR) * 8 of the wavefront's K range) -> MFMA A operands
// v[s] (step s: row lane % 16, k = s*32 + (lane / 16) * 8), through the
// wavefront's LDS area of 16 rows x pitch bytes.  The reads follow the
// writes in the same wavefront, so LDS order alone makes them see them.
// NS: MFMA steps of the wavefront's K range (= loads per 16 rows).
template <int NS>
__device__ __forceinline__ void rows_to_mfma_a(u32x4 (&v)[NS], char* area, int pitch, int lpr_sh, int lane) {
  const int rpi = kWave >> lpr_sh, lpr = 1 << lpr_sh;
#pragma unroll
  for (int s = 0; s < NS; ++s)
    *reinterpret_cast<u32x4*>(area + (s * rpi + (lane >> lpr_sh)) * pitch + ((lane & (lpr - 1)) << 4)) = v[s];
#pragma unroll
  for (int s = 0; s < NS; ++s) v[s] = *reinterpret_cast<const u32x4*>(area + (lane & 15) * pitch + s * 64 + (lane >> 4) * 16);
}

// Expert record of a slot (the shared expert in slot 0 when present):
// weights, first permuted position, pair count; false past the active ones.
__device__ __forceinline__ bool expert_slot(const ExpertArgs& a, int slot, const char* routed, const char* shared_w,
                                            size_t expert_bytes, const char*& W, int& pos0, int& npairs, bool& shared) {
  shared = false;
  if (a.has_shared && slot == 0) {
    W = shared_w;
    pos0 = a.T * a.K;
    npairs = a.T;
    shared = true;
    return true;
  }
  if (a.has_shared) slot -= 1;
  const int na = a.ws.num_active[0];  // loaded with the record (slot < E)
  const int4 rec = a.ws.slots[slot];
  if (slot >= na) return false;
  W = routed + (size_t)rec.x * expert_bytes;
  pos0 = rec.y;
  npairs = rec.z;
  return true;
}

// KS = H / 256: MFMA steps per wavefront (H = 512, 1024, 2048 -> 2, 4, 8).
template <int KS>
__global__ __launch_bounds__(512) void moe_gateup_mfma_kernel(ExpertArgs a) {
  extern __shared__ float4 s_gu_v[];
  char* s_lds = reinterpret_cast<char*>(s_gu_v);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int H = a.H, I = a.I, K = a.K;
  const int ipb = I / kGuMfmaRows;
  const int ib = blockIdx.x % ipb, i0 = ib * kGuMfmaRows;
  const char* W;
  int pos0, npairs;
  bool shared;
  if (!expert_slot(a, blockIdx.x / ipb, reinterpret_cast<const char*>(a.gu), reinterpret_cast<const char*>(a.sgu),
                   (size_t)2 * I * H * 2, W, pos0, npairs, shared))
    return;
  const int lh = 31 - __builtin_clz((unsigned)H);
  const int kw = H >> 3;                 // K range of a wavefront's MFMAs (KS steps of 32)
  const int pitch = 2 * H + 16;          // LDS tile row (16-byte pad: the 16 rows of an operand read hit distinct banks)
  // Whole-row loads: wavefront w reads gate rows i0 + 2w, i0 + 2w + 1 and the
  // same up rows, one 1 KiB piece per load (slot s: row 2w + s / (KS/2),
  // piece s % (KS/2)); reading its MFMA K range of all 16 rows instead
  // streams measurably slower on this part.  The gate rows, then the up
  // rows, meet in the workgroup's LDS tile, from which each wavefront reads
  // its operands.
  constexpr int PPR = KS / 2;  // 1 KiB pieces per row
  const uint32_t lane_off = (uint32_t)((wave << (lh + 2)) + (lane << 4));
  u32x4 av[2][KS];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int s = 0; s < KS; ++s)
      av[h][s] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
          W + ((size_t)(h * I + i0 + s / PPR) << (lh + 1)) + (size_t)(s % PPR) * 1024 + lane_off));
  const int n = lane & 15, g4 = lane >> 4;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (h > 0) __syncthreads();  // the gate operands are read
#pragma unroll
    for (int s = 0; s < KS; ++s)
      *reinterpret_cast<u32x4*>(s_lds + (2 * wave + s / PPR) * pitch + (s % PPR) * 1024 + lane * 16) = av[h][s];
    __syncthreads();
#pragma unroll
    for (int s = 0; s < KS; ++s)
      av[h][s] = *reinterpret_cast<const u32x4*>(s_lds + n * pitch + (wave * kw + s * 32 + g4 * 8) * 2);
  }
  __syncthreads();  // the partial tiles below overlap the LDS tile

  float* s_part = reinterpret_cast<float*>(s_lds);  // [wave][gate|up][16 rows][16 columns]
  for (int tile = 0; tile * 16 < npairs; ++tile) {
    // column n: pair tile*16 + n (clamped; columns past npairs are dropped)
    const int p = min(tile * 16 + n, npairs - 1);
    const int t = shared ? p : a.ws.perm[pos0 + p] / K;
    u32x4 bv[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s)
      bv[s] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(a.x) + (size_t)t * H + wave * kw + s * 32 +
                                              g4 * 8);
    f32x4_t accg = {0.f, 0.f, 0.f, 0.f}, accu = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      accg = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av[0][s]),
                                                     __builtin_bit_cast(bf16x8_t, bv[s]), accg, 0, 0, 0);
      accu = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av[1][s]),
                                                     __builtin_bit_cast(bf16x8_t, bv[s]), accu, 0, 0, 0);
    }
    if (tile > 0) __syncthreads();  // the previous tile's sums are read
    float* pw = s_part + (size_t)wave * 512;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      pw[(g4 * 4 + q) * 16 + n] = accg[q];
      pw[256 + (g4 * 4 + q) * 16 + n] = accu[q];
    }
    __syncthreads();
    if (tid < 256) {
      const int r = tid >> 4, c = tid & 15;
      float gs = 0.f, us = 0.f;
#pragma unroll
      for (int w = 0; w < kGuMfmaWaves; ++w) {
        gs += s_part[w * 512 + r * 16 + c];
        us += s_part[w * 512 + 256 + r * 16 + c];
      }
      if (tile * 16 + c < npairs) a.ws.act[(size_t)(pos0 + tile * 16 + c) * I + i0 + r] = silu(gs) * us;
    }
  }

  // Shared-expert gate sigmoid(w_g . x_t), once per token (bf16 gate weight
  // or per element otherwise).
  if (shared && ib == 0 && a.sg) {
    const int nch = H >> 3;
    const bool sg_vec = a.sg_dt == FK_DTYPE_BF16 && (reinterpret_cast<uintptr_t>(a.sg) & 15u) == 0;
    for (int t = wave; t < a.T; t += kGuMfmaWaves) {
      float d = 0.f;
      for (int c = lane; c < nch; c += kWave) {
        float x8[8], g8[8];
        load8_f32<true>(a.x, (size_t)t * H + (size_t)c * 8, x8);
        if (sg_vec) load8_f32<true>(a.sg, (size_t)c * 8, g8);
        else
#pragma unroll
          for (int q = 0; q < 8; ++q) g8[q] = load_scalar(a.sg, a.sg_dt, (size_t)c * 8 + q);
#pragma unroll
        for (int q = 0; q < 8; ++q) d = fmaf(x8[q], g8[q], d);
      }
      d = wave_sum(d);
      if (lane == 0) a.ws.sgate[t] = sigmoid(d);
    }
  }
}

// KS = I / 128: MFMA steps per wavefront (I = 256, 512 -> 2, 4); RT: row
// tiles of 16 output rows per work item.
template <int KS, int RT>
__global__ __launch_bounds__(256) void moe_down_mfma_kernel(ExpertArgs a) {
  extern __shared__ float4 s_dn_v[];
  char* s_lds = reinterpret_cast<char*>(s_dn_v);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int H = a.H, I = a.I;
  constexpr int NR = RT * 16;  // output rows per work item
  const int rbn = H / NR;
  const int rb = blockIdx.x % rbn, r0 = rb * NR;
  const char* W;
  int pos0, npairs;
  bool shared;
  if (!expert_slot(a, blockIdx.x / rbn, reinterpret_cast<const char*>(a.dn), reinterpret_cast<const char*>(a.sdn),
                   (size_t)H * I * 2, W, pos0, npairs, shared))
    return;
  const int li = 31 - __builtin_clz((unsigned)I);
  const int kw = I >> 2;                 // K range of a wavefront (KS steps of 32)
  const int lpr_sh = li - 5;             // LPR = kw / 8
  const int rpi = kWave >> lpr_sh;
  const int pitch = kw * 2 + 16;

  // The activations of a tile's pairs (column n: pair n/2, bf16 hi for even
  // n, lo for odd n) do not depend on the weights: the first tile's are
  // issued before the weight rows, each later tile's while the previous one
  // is computed.
  const int n = lane & 15, g4 = lane >> 4;
  float4 araw[KS][2];
  auto load_act = [&](int tile) {
    const int p = min(tile * 8 + (n >> 1), npairs - 1);
    const float* ar = a.ws.act + (size_t)(pos0 + p) * I + wave * kw + g4 * 8;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      araw[s][0] = *reinterpret_cast<const float4*>(ar + s * 32);
      araw[s][1] = *reinterpret_cast<const float4*>(ar + s * 32 + 4);
    }
  };
  load_act(0);

  // rows r0 + 16 rt .. of this wavefront's K range (RT row tiles)
  const uint32_t lane_off = (uint32_t)((((lane >> lpr_sh) << li) + wave * kw + ((lane & ((1 << lpr_sh) - 1)) << 3)) << 1);
  u32x4 av[RT][KS];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int s = 0; s < KS; ++s)
      av[rt][s] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4*>(W + ((size_t)(r0 + rt * 16 + s * rpi) << (li + 1)) + lane_off));
  char* area = s_lds + (size_t)wave * 16 * pitch;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) rows_to_mfma_a<KS>(av[rt], area, pitch, lpr_sh, lane);
  __syncthreads();  // the partial tiles below overlap other wavefronts' areas

  float* s_part = reinterpret_cast<float*>(s_lds);  // [wave][row tile][16 rows][16 columns]
  for (int tile = 0; tile * 8 < npairs; ++tile) {
    u32x4 bv[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const float4 lo4 = araw[s][0], hi4 = araw[s][1];
      const float v8[8] = {lo4.x, lo4.y, lo4.z, lo4.w, hi4.x, hi4.y, hi4.z, hi4.w};
      uint32_t h[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // hi = bf16(v), lo = bf16(v - hi), both rounded to nearest even
        const uint32_t hi = pack_bf16x2(v8[2 * e], v8[2 * e + 1]);
        const uint32_t lo = pack_bf16x2(v8[2 * e] - __uint_as_float(hi << 16), v8[2 * e + 1] - __uint_as_float(hi & 0xffff0000u));
        h[e] = (n & 1) ? lo : hi;
      }
      bv[s] = u32x4{h[0], h[1], h[2], h[3]};
    }
    if ((tile + 1) * 8 < npairs) load_act(tile + 1);
    f32x4_t acc[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      acc[rt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s)
        acc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av[rt][s]),
                                                          __builtin_bit_cast(bf16x8_t, bv[s]), acc[rt], 0, 0, 0);
    }
    if (tile > 0) __syncthreads();  // the previous tile's sums are read
    float* pw = s_part + (size_t)wave * RT * 256;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int q = 0; q < 4; ++q) pw[rt * 256 + (g4 * 4 + q) * 16 + n] = acc[rt][q];
    __syncthreads();
    // thread: output row R = tid % NR (tile R / 16, row R % 16), pairs
    // j = tid / NR + jj * (256 / NR) (NR = 16: threads past 128 idle)
    {
      constexpr int JS = 256 / NR < 8 ? 256 / NR : 8;
      const int R = tid % NR, rt = R >> 4, r = R & 15;
#pragma unroll
      for (int jj = 0; jj < 8 / JS; ++jj) {
        const int j = tid / NR + jj * JS;
        if (j >= 8) break;
        float y = 0.f;
#pragma unroll
        for (int w = 0; w < kDnMfmaWaves; ++w)
          y += s_part[w * RT * 256 + rt * 256 + r * 16 + 2 * j] + s_part[w * RT * 256 + rt * 256 + r * 16 + 2 * j + 1];
        if (tile * 8 + j < npairs) a.ws.y[(size_t)(pos0 + tile * 8 + j) * H + r0 + R] = y;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Single-launch MoE layer for one token (T = 1, H <= 2048 with H % 8 == 0,
// I <= 512 with I % 16 == 0, E <= 256, K <= 8, bf16 router and expert
// weights, shared expert present).  From two tokens on the tagged router and
// the expert kernels are faster.
//
// 512-thread workgroups, one per CU (grid G capped at the co-resident
// capacity).  Item q of P1 goes to wavefront q / G of workgroup q % G, so
// consecutive items land on different CUs.
//   P1  router logits (one expert row per item; every workgroup holds one
//       row, so the logits land one row's latency after the launch) and,
//       overlapped, the shared expert's gate/up + SwiGLU (one intermediate
//       per item) and its gate: routing-independent weights that stream
//       while the logits are handed off
//   P2  every workgroup polls the logits and selects the top-k itself
//       (topk_select_ranked, one wavefront), which writes the routing table
//       (expert of slot u, selection order) into LDS
//   P3  routed gate/up: workgroup b takes block b (16 consecutive
//       intermediates of one slot, two per wavefront); each intermediate
//       leaves as one tagged word.  Then its down item is issued: 64 rows of
//       one slot's down matrix (8 per wavefront, 64 KB), and one shared down
//       row per wavefront for its output rows 8 b .. 8 b + 7
//   P4  the workgroup polls its down item's slot activations (512 words, one
//       per thread: the 32 workgroups of that slot, not the whole grid) and
//       the shared ones, applies its 64 rows (lanes 8 j .. 8 j + 7 end with
//       row j) and publishes y[slot][row] as tagged words
//   P5  it polls the K slots' y of its 8 output rows (64 words) and writes
//       out = sum_k w_k y_k + g sh in the multi-launch combine's order
//       (routed slots in selection order, then the gated shared expert,
//       moe_combine_kernel) and layer_out = x + out.
// Every workgroup thus polls 512 + 512 + 64 words after its gate/up block
// instead of all 4,608 activations: polls that run while the weight stream
// is still in flight slow it down.
//
// Hand-offs carry a launch tag instead of using barriers: every value that
// crosses workgroups (logits, activations, shared gate) is written as a
// tagged word (store_tagged) and polled until it carries this launch's tag,
// so a consumer waits only for the values it reads.  The tag is
// epoch + 1, where the epoch is a workspace counter that every wavefront
// reads at its start; each workgroup posts a started record with its tag,
// and workgroup 0 advances the epoch once every record of this launch is
// there (so no wavefront can read the advanced epoch in the same launch).
// Tags are 32-bit: a word left untouched for exactly 2^32 launches on one
// workspace would read as current.
// ---------------------------------------------------------------------------
constexpr int kFusedMaxTokens = 1;  // from 2 tokens on, the tagged router + expert kernels are faster
constexpr int kFusedMaxPairs = kFusedMaxTokens * 8;
constexpr int kFusedWaves = 8;
constexpr int kFusedMaxExperts = 256;
constexpr int kFusedChunk = 16;  // routed items per workgroup block: 16 tagged words = one 128-byte line
static_assert(kFusedLogitWords >= (size_t)kFusedMaxTokens * kFusedMaxExperts, "fused logit region too small");
static_assert(kFusedActWords >= (size_t)(kFusedMaxPairs + kFusedMaxTokens) * 512, "fused activation region too small");
static_assert(kFusedGateWords >= (size_t)kFusedMaxTokens, "fused gate region too small");

struct FusedArgs {
  RouterArgs r;
  const void* gu;
  const void* dn;
  const void* sgu;
  const void* sdn;
  const void* sg;
  int sg_dt;
  int I;
  float* out;
  float* layer_out;
};

// Down-row chunk (8 bf16) of this lane against the activation row staged in LDS.
__device__ __forceinline__ float dot8_act_lds(const Raw8<true>& w, const float* act_row, int lane, int I) {
  float d = 0.f;
  if (lane * 8 < I) {
    float w8[8], a8[8];
    raw8_to_f32<true>(w, w8);
    const float4* p = reinterpret_cast<const float4*>(act_row + lane * 8);
    const float4 lo = p[0], hi = p[1];
    a8[0] = lo.x; a8[1] = lo.y; a8[2] = lo.z; a8[3] = lo.w;
    a8[4] = hi.x; a8[5] = hi.y; a8[6] = hi.z; a8[7] = hi.w;
#pragma unroll
    for (int q = 0; q < 8; ++q) d = fmaf(w8[q], a8[q], d);
  }
  return d;
}


// Gate/up rows of NI intermediates (bf16, H <= 2048: 4 chunks per lane)
// against the token's chunks xt; act[i] = silu(gate_i . x) * (up_i . x),
// the same in every lane.  Every row load is issued before the first
// product (addresses clamped in range, so no load is conditional);
// after_issue() runs right behind the loads.
template <bool BFX, int NI, class AfterIssue>
__device__ __forceinline__ void fused_gu_rows(const Raw8<BFX> (&xt)[4], const char* const (&gate)[NI],
                                              const char* const (&up)[NI], int nch, int lane, float (&act)[NI],
                                              AfterIssue after_issue) {
  Raw8<true> g[NI][4], u[NI][4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const size_t c8 = (size_t)min(lane + kWave * j, nch - 1) * 8;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      g[i][j] = load_raw8_stream<true>(gate[i], c8);
      u[i][j] = load_raw8_stream<true>(up[i], c8);
    }
  }
  after_issue();
  float acc[2 * NI];
#pragma unroll
  for (int i = 0; i < 2 * NI; ++i) acc[i] = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (lane + kWave * j < nch) {
      float x8[8], w8[8];
      raw8_to_f32<BFX>(xt[j], x8);
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        raw8_to_f32<true>(g[i][j], w8);
#pragma unroll
        for (int q = 0; q < 8; ++q) acc[2 * i] = fmaf(w8[q], x8[q], acc[2 * i]);
        raw8_to_f32<true>(u[i][j], w8);
#pragma unroll
        for (int q = 0; q < 8; ++q) acc[2 * i + 1] = fmaf(w8[q], x8[q], acc[2 * i + 1]);
      }
    }
  }
  // the 2 NI sums at once (rows4_sum: lanes 16 r hold sum r; rows8_sum:
  // lanes 8 r)
  if constexpr (NI <= 2) {
    float d[4] = {acc[0], acc[1], NI > 1 ? acc[2] : 0.f, NI > 1 ? acc[3] : 0.f};
    const float rs = rows4_sum(d);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const float gs = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(rs), 32 * i));
      const float us = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(rs), 32 * i + 16));
      act[i] = silu(gs) * us;
    }
  } else {
    static_assert(NI <= 4, "at most four intermediates per call");
    float d[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) d[i] = i < 2 * NI ? acc[i] : 0.f;
    const float rs = rows8_sum(d);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const float gs = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(rs), 16 * i));
      const float us = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(rs), 16 * i + 8));
      act[i] = silu(gs) * us;
    }
  }
}

// Eight down rows (one 16-byte chunk of each in this lane) against the
// lane's 8 activation columns, read once from LDS; d[j] is row j's partial.
__device__ __forceinline__ void dot8x8_act_lds(const Raw8<true> (&w)[8], const float* act_row, int lane, int I,
                                               float (&d)[8]) {
  float a8[8];
  const float4* p = reinterpret_cast<const float4*>(act_row + min(lane * 8, I - 8));
  const float4 lo = p[0], hi = p[1];
  a8[0] = lo.x; a8[1] = lo.y; a8[2] = lo.z; a8[3] = lo.w;
  a8[4] = hi.x; a8[5] = hi.y; a8[6] = hi.z; a8[7] = hi.w;
  const bool in = lane * 8 < I;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float w8[8];
    raw8_to_f32<true>(w[j], w8);
    float acc = 0.f;
#pragma unroll
    for (int q = 0; q < 8; ++q) acc = fmaf(w8[q], a8[q], acc);
    d[j] = in ? acc : 0.f;
  }
}

FK_TIMELINE_BUFFER(moe_fused)

// FAST: the host has checked that the grid has one workgroup per gate/up
// block, per down item and per output row group (the model's shape on a
// full MI355X): straight-line code for that case.
template <bool BFX, bool FAST>
__global__ __launch_bounds__(512) void moe_fused_kernel(FusedArgs f) {
  constexpr int RG = kFusedWaves;       // output rows per final row group (one per wavefront)
  constexpr int DR = RG * kFusedWaves;  // rows per down item (8 per wavefront)
  __shared__ int s_active[kFusedMaxPairs];  // routed experts, selection order
  __shared__ float s_wpos[kFusedMaxPairs];  // routing weight of each slot
  __shared__ int s_fail;
  __shared__ uint32_t s_wtag[kFusedWaves];
  __shared__ __align__(16) TopkLds s_topk;
  __shared__ __align__(16) float s_sha[512];  // shared activations
  __shared__ __align__(16) float s_ra[512];   // activations of the down item's slot
  __shared__ float s_sg;                      // shared gate
  __shared__ float s_yk[kFusedMaxPairs * RG];  // final: y[slot][row] of the row group
  __shared__ float s_act16[kFusedChunk];       // the gate/up block's activations
  __shared__ float s_ystage[DR];               // the down item's outputs
  __shared__ float s_sh[RG];                   // final: shared down rows of the row group
  const RouterArgs& a = f.r;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int G = gridDim.x, b = blockIdx.x;
  const int NW = G * kFusedWaves;
  const int q0 = wave * G + b;
  const int H = a.H, E = a.E, K = a.K, I = f.I, P = K;
  const int nch = H >> 3;
  uint32_t* err = &a.ws.tickets[kTicketError];
  // The launch tag (epoch + 1) is loaded after the wavefront's P1 weight
  // loads are issued: computed from a load issued first, it would make every
  // wavefront wait for that load before issuing anything else.
  uint32_t tag = 0, plim = 0;
  bool have_tag = false;
  if (tid == 0) s_fail = 0;
  __syncthreads();
  FK_TIMELINE_DECL;
  FK_MARK(0);  // (timeline markers: diagnostic builds only)
  // The fast path's item indices (block b: slot f_ub, intermediates f_i0..;
  // down item b: slot f_ud, rows f_rr0..), computed here, where the scalar
  // divisions overlap the first loads' latency instead of delaying the
  // routed gate/up rows.
  int f_ub = 0, f_i0 = 0, f_ud = 0, f_rr0 = 0;
  if constexpr (FAST) {
    const int bpe_ = I / kFusedChunk, cpe_ = (H + DR - 1) / DR;
    f_ub = b / bpe_;
    f_i0 = (b - f_ub * bpe_) * kFusedChunk;
    f_ud = b / cpe_;
    f_rr0 = (b - f_ud * cpe_) * DR;
    asm volatile("" : "+s"(f_ub), "+s"(f_i0), "+s"(f_ud), "+s"(f_rr0));
  }

  // ---------------- P1: router rows, shared gate/up, shared gate -----------
  // Item q: router rows 0..E-1, shared intermediates E..E+I-1, then the
  // shared gate.  Each wavefront publishes its result as one tagged word.
  const int nitems = E + I + 1;
  for (int q = q0; q < nitems; q += NW) {
    if (q < E) {
      const int e = q;
      // All loads of the row (weights, the token, the bf16 norm weight) are
      // issued before the first use: indices are clamped in range and
      // out-of-range chunks are zeroed afterwards, so there is no branch
      // between them (a load whose dtype is tested at run time would wait
      // for every load before it).
      Raw8<true> wr[4], nr[4];
      Raw8<BFX> xr[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int cc = min(lane + kWave * j, nch - 1);
        wr[j] = load_raw8<true>(a.W, (size_t)e * H + (size_t)cc * 8);
        xr[j] = load_raw8<BFX>(a.x, (size_t)cc * 8);
        nr[j] = load_raw8<true>(a.nw, (size_t)cc * 8);
      }
      {
        const WaitLimits wl = wait_limits(a.ws.tickets, kTicketEpoch);
        tag = wl.tag;
        plim = wl.poll;
      }
      have_tag = true;
      float wn[4][8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int c = lane + kWave * j;
        float w8[8], n8[8];
        raw8_to_f32<true>(nr[j], n8);
        raw8_to_f32<true>(wr[j], w8);
#pragma unroll
        for (int qq = 0; qq < 8; ++qq) wn[j][qq] = c < nch ? w8[qq] * (a.off + n8[qq]) : 0.f;
      }
      const float bias = a.bias ? load_scalar(a.bias, a.bias_dt, e) : 0.f;
      float ss = 0.f, d = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool in = lane + kWave * j < nch;
        float x8[8];
        raw8_to_f32<BFX>(xr[j], x8);
#pragma unroll
        for (int qq = 0; qq < 8; ++qq) {
          const float xv = in ? x8[qq] : 0.f;
          ss = fmaf(xv, xv, ss);
          d = fmaf(xv, wn[j][qq], d);
        }
      }
      ss = wave_sum(ss);
      d = wave_sum(d);
      const float v = d * rsqrtf(ss / (float)H + a.eps) + bias;
      if (lane == 0) {
        a.logits[e] = v;
        store_tagged(a.ws.f_logits + e, v, tag);
      }
    } else if (q < E + I) {
      const int i = q - E;
      Raw8<BFX> xt[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) xt[j] = load_raw8<BFX>(a.x, (size_t)min(lane + kWave * j, nch - 1) * 8);
      const char* sgu = reinterpret_cast<const char*>(f.sgu);
      const char* g[1] = {sgu + (size_t)i * H * 2};
      const char* u[1] = {sgu + (size_t)(I + i) * H * 2};
      float act[1];
      fused_gu_rows<BFX, 1>(xt, g, u, nch, lane, act, [&]() {
        const WaitLimits wl = wait_limits(a.ws.tickets, kTicketEpoch);
        tag = wl.tag;
        plim = wl.poll;
      });
      have_tag = true;
      if (lane == 0) store_tagged(a.ws.f_act + (size_t)P * I + i, act[0], tag);
    } else {
      // Shared-expert gate of the token: one row like the router's.  (The
      // gate weight is bf16 here; a NULL gate reads the norm weight, a valid
      // address, and the products are dropped.)
      Raw8<BFX> xr[4];
      Raw8<true> gr[4];
      const void* gsrc = f.sg ? f.sg : a.nw;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int cc = min(lane + kWave * j, nch - 1);
        xr[j] = load_raw8<BFX>(a.x, (size_t)cc * 8);
        gr[j] = load_raw8<true>(gsrc, (size_t)cc * 8);
      }
      {
        const WaitLimits wl = wait_limits(a.ws.tickets, kTicketEpoch);
        tag = wl.tag;
        plim = wl.poll;
      }
      have_tag = true;
      float d = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int c = lane + kWave * j;
        float x8[8], g8[8];
        raw8_to_f32<BFX>(xr[j], x8);
        raw8_to_f32<true>(gr[j], g8);
#pragma unroll
        for (int qq = 0; qq < 8; ++qq) d = fmaf(x8[qq], (f.sg && c < nch) ? g8[qq] : 0.f, d);
      }
      d = wave_sum(d);
      if (lane == 0) store_tagged(a.ws.f_sgate, f.sg ? sigmoid(d) : 1.f, tag);
    }
  }
  FK_MARK(1);
  if (!have_tag) {
    const WaitLimits wl = wait_limits(a.ws.tickets, kTicketEpoch);
    tag = wl.tag;
    plim = wl.poll;
  }
  // Fast path: wavefronts 1-7 fetch their shared down row (routing-
  // independent, used at the very end) while wavefront 0 selects the top-k,
  // when the HBM is otherwise nearly idle; wavefront 0 fetches its own after
  // the selection (before it, the row would sit ahead of the logit polls in
  // the wavefront's in-order load queue).
  Raw8<true> sdr_early;
  if constexpr (FAST) {
    if (wave != 0)
      sdr_early = load_raw8_stream<true>(f.sdn, (size_t)(uint32_t)((b * RG + wave) * I) + (size_t)min(lane * 8, I - 8));
  }
  // Started record of this workgroup: every wavefront has used the epoch it
  // read (its LDS write needs the loaded value), so the epoch may advance
  // once all records of this launch are there.
  if (lane == 0) s_wtag[wave] = tag;
  __syncthreads();
  if (tid == 0) store_tagged(a.ws.f_started + b, __uint_as_float(s_wtag[kFusedWaves - 1]), tag);

  // ---------------- P2: top-k, routing table in LDS ------------------------
  if (wave == 0) {
    constexpr int NJE = kFusedMaxExperts / kWave;
    uint64_t w[NJE];
    const uint64_t* srcs[NJE];
#pragma unroll
    for (int j = 0; j < NJE; ++j) {
      const int ex = lane + kWave * j;
      srcs[j] = ex < E ? a.ws.f_logits + ex : nullptr;
      w[j] = srcs[j] ? load_tagged(srcs[j]) : 0ull;
    }
    const bool ok = poll_tagged<NJE>(w, srcs, tag, plim);
    if (!ok) s_fail = 1;
    FK_MARK(2);
    float l[NJE];
#pragma unroll
    for (int j = 0; j < NJE; ++j) l[j] = value_of(w[j]);
    // One token: the K selections are distinct experts, so the routing
    // table is the selection itself (slot u = selection u) with no sort.
    // (After a failed wait the logits may be stale: the ids are in range
    // and every output of this workgroup is poisoned below.)
    topk_select_ranked(l, E, K, lane, &s_topk, s_active, s_wpos);
    FK_MARK(3);
  } else if (b == 0) {
    // Workgroup 0 checks that every wavefront of this launch has read the
    // epoch (its started record carries the tag) before advancing it.
    constexpr int kChunk = 4;
    const int nthr = (kFusedWaves - 1) * kWave;
    for (int base = tid - kWave; base < G; base += kChunk * nthr) {
      uint64_t w[kChunk];
      const uint64_t* srcs[kChunk];
#pragma unroll
      for (int j = 0; j < kChunk; ++j) {
        const int r = base + j * nthr;
        srcs[j] = r < G ? a.ws.f_started + r : nullptr;
        w[j] = srcs[j] ? load_tagged(srcs[j]) : 0ull;
      }
      if (!poll_tagged<kChunk>(w, srcs, tag, plim)) s_fail = 1;
    }
  }
  __syncthreads();
  // A failed wait poisons every later output of the workgroup.  Workgroup 0
  // advances the epoch only when every workgroup has read it (all started
  // records carry this launch's tag): otherwise a late workgroup would take
  // the next launch's tag and publish words that launch reads as its own.
  const bool bad = s_fail;
  if (b == 0 && tid == 0 && !bad) store_coherent(&a.ws.tickets[kTicketEpoch], tag);
  FK_MARK(4);
  if (b == 0 && tid < P) {
    a.ids_out[tid] = s_active[tid];
    a.w_out[tid] = poison_if(bad, s_wpos[tid]);
  }

  // ---------------- P3..P5 ------------------------------------------------
  const int bpe = I / kFusedChunk, nblk = K * bpe;
  const int cpe = (H + DR - 1) / DR, ndn = K * cpe;  // down items: (slot, 64-row chunk)
  const int ngrp = H / RG;                            // final row groups
  const int r0 = b * RG;  // this workgroup's first final row group (if b < ngrp)
  const size_t dcol = (size_t)min(lane * 8, I - 8);
  const char* gu = reinterpret_cast<const char*>(f.gu);
  const size_t rowb = (size_t)H * 2, expb = (size_t)2 * I * rowb;
  // The residual input of the workgroup's rows (raw bits; converted where
  // used, since a conversion here would wait for it).
  uint32_t x_raw[1];
  gather_raw<BFX>(a.x, (size_t)min(r0 + lane, H - 1), 0, 1, x_raw);
  if constexpr (FAST) {
    // The model's shape on a full grid: workgroup b takes gate/up block b,
    // down item b and output rows r0 .. r0 + 7, in straight-line code with
    // unconditional (clamped) loads, so the compiler's waits are exact.
    // Stores go out through one wavefront (7) and the polls through others:
    // a wavefront's loads retire in order behind its stores, so a poll
    // behind a store would wait for the store's acknowledgement.
    const int ub = f_ub, i0 = f_i0, ia = i0 + 2 * wave;
    const int ud = f_ud, rr0 = f_rr0, rw = rr0 + wave * RG;
    const char* we = gu + (size_t)s_active[ub] * expb;
    const char* g2[2] = {we + (size_t)ia * rowb, we + (size_t)(ia + 1) * rowb};
    const char* u2[2] = {we + (size_t)(I + ia) * rowb, we + (size_t)(I + ia + 1) * rowb};
    const uint16_t* dnb = reinterpret_cast<const uint16_t*>(f.dn) + (size_t)s_active[ud] * H * I;
    const uint16_t* sdb = reinterpret_cast<const uint16_t*>(f.sdn);
    const uint64_t* sh_src = a.ws.f_act + (size_t)P * I + min(tid, I - 1);
    const uint64_t* ra_src0 = a.ws.f_act + (size_t)ud * I + min(tid, I - 1);
    const uint64_t* ra_src1 = a.ws.f_act + (size_t)ud * I + min(tid + 256, I - 1);
    const uint64_t* y_src = a.ws.f_y + (size_t)min(lane >> 3, K - 1) * H + r0 + (lane & 7);
    Raw8<BFX> xt[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) xt[j] = load_raw8<BFX>(a.x, (size_t)min(lane + kWave * j, nch - 1) * 8);
    uint64_t shw = 0, sgw = 0;
    float act[2];
    // gate/up rows, then the shared activation word and gate (stored in P1)
    FK_MARK(9);
    fused_gu_rows<BFX, 2>(xt, g2, u2, nch, lane, act, [&]() {
      shw = load_tagged(sh_src);
      sgw = load_tagged(a.ws.f_sgate);
      FK_MARK(10);
    });
    FK_MARK(11);
    if (lane == 0) {
      s_act16[2 * wave] = act[0];
      s_act16[2 * wave + 1] = act[1];
    }
    // Down rows of the item and the shared down row, issued only now: loads
    // in flight together are served interleaved whatever their issue order,
    // and the hand-off waits for the gate/up rows, not for these.
    Raw8<true> dr[RG];
#pragma unroll
    for (int j = 0; j < RG; ++j) dr[j] = load_raw8_stream<true>(dnb, (size_t)(uint32_t)(min(rw + j, H - 1) * I) + dcol);
    Raw8<true> sdr = sdr_early;
    if (wave == 0) sdr = load_raw8_stream<true>(sdb, (size_t)(uint32_t)((r0 + wave) * I) + dcol);
    // the slot's activations: 512 words over wavefronts 0-3, two per lane
    uint64_t raw0 = 0, raw1 = 0;
    if (wave < 4) {
      raw0 = load_tagged(ra_src0);
      raw1 = load_tagged(ra_src1);
    }
    bool ok = true;
    const float shv = settle_tagged(shw, sh_src, tag, plim, ok);
    const float sgv = settle_tagged(sgw, a.ws.f_sgate, tag, plim, ok);
    if (tid < I) s_sha[tid] = shv;
    if (tid == 0) s_sg = sgv;
    lds_barrier();
    FK_MARK(5);
    if (wave == kFusedWaves - 1 && lane < kFusedChunk)
      store_tagged(a.ws.f_act + (size_t)ub * I + i0 + lane, poison_if(bad, s_act16[lane]), tag);
    if (wave < 4) {
      const float v0 = settle_tagged(raw0, ra_src0, tag, plim, ok);
      const float v1 = settle_tagged(raw1, ra_src1, tag, plim, ok);
      if (tid < I) s_ra[tid] = v0;
      if (tid + 256 < I) s_ra[tid + 256] = v1;
    }
    if (!ok) s_fail = 1;
    lds_barrier();
    FK_MARK(6);
    // down: 8 rows per wavefront (lanes 8 j .. 8 j + 7 end with row j), and
    // one shared row
    {
      float dd[RG];
      dot8x8_act_lds(dr, s_ra, lane, I, dd);
      const float v = rows8_sum(dd);
      if ((lane & 7) == 0) s_ystage[wave * RG + (lane >> 3)] = v;
    }
    {
      const float sh = wave_sum(dot8_act_lds(sdr, s_sha, lane, I));
      if (lane == 0) s_sh[wave] = sh;
    }
    uint64_t yw = 0;
    if (wave == 0) yw = load_tagged(y_src);
    lds_barrier();
    if (wave == kFusedWaves - 1 && rr0 + lane < H)
      store_tagged(a.ws.f_y + (size_t)ud * H + rr0 + lane, poison_if(s_fail, s_ystage[lane]), tag);
    FK_MARK(7);
    if (wave == 0) {
      bool yok = true;
      const float yv = settle_tagged(yw, y_src, tag, plim, yok);
      s_yk[lane] = yv;
      if (!yok) s_fail = 1;
    }
    lds_barrier();
    if (wave == 0 && lane < RG) {
      const bool bad_out = s_fail;
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < kFusedMaxPairs; ++k)
        if (k < K) acc += s_wpos[k] * s_yk[k * RG + lane];
      acc += s_sg * s_sh[lane];
      const float o = poison_if(bad_out, acc);
      f.out[r0 + lane] = o;
      if (f.layer_out) f.layer_out[r0 + lane] = raw_value<BFX>(x_raw[0]) + o;
    }
  } else {
    // The shared activations and gate, one word per thread: stored in P1, so
    // the first read finds them; issued behind the first gate/up rows.
    uint64_t shw[2];
    const uint64_t* shs[2] = {tid < I ? a.ws.f_act + (size_t)P * I + tid : nullptr, tid == 0 ? a.ws.f_sgate : nullptr};
    {
      Raw8<BFX> xt[4];
  #pragma unroll
      for (int j = 0; j < 4; ++j) xt[j] = load_raw8<BFX>(a.x, (size_t)min(lane + kWave * j, nch - 1) * 8);
      bool first = true;
      auto issue_shared = [&]() {
        if (first) {
  #pragma unroll
          for (int j = 0; j < 2; ++j) shw[j] = shs[j] ? load_tagged(shs[j]) : 0ull;
        }
      };
      if (b >= nblk) {
        issue_shared();
      }
      for (int blk = b; blk < nblk; blk += G) {
        // intermediates ia, ia + 1 of slot u in this wavefront
        const int u_ = blk / bpe, ia = (blk - u_ * bpe) * kFusedChunk + 2 * wave;
        const char* we = gu + (size_t)s_active[u_] * expb;
        const char* g[2] = {we + (size_t)ia * rowb, we + (size_t)(ia + 1) * rowb};
        const char* u[2] = {we + (size_t)(I + ia) * rowb, we + (size_t)(I + ia + 1) * rowb};
        float act[2];
        fused_gu_rows<BFX, 2>(xt, g, u, nch, lane, act, issue_shared);
        first = false;
        if (lane < 2) store_tagged(a.ws.f_act + (size_t)u_ * I + ia + lane, poison_if(bad, lane ? act[1] : act[0]), tag);
      }
    }
    // The first down item's rows and the shared down row of the first row
    // group, issued only now: loads in flight together are served interleaved
    // whatever their issue order, and the hand-off waits for the gate/up rows,
    // not for these.  (wave-uniform: the down code reduces across lanes with
    // lane swaps, which read inactive lanes' stale registers)
    const bool dn0 = b < ndn, grp0 = r0 < H;
    Raw8<true> dr[RG], sdr;
    auto issue_down = [&](int d, Raw8<true> (&w)[RG]) {
      const int u_ = d / cpe, rr = (d - u_ * cpe) * DR + wave * RG;
      const size_t ex = (size_t)s_active[u_];
  #pragma unroll
      for (int j = 0; j < RG; ++j) w[j] = load_raw8_stream<true>(f.dn, (ex * H + min(rr + j, H - 1)) * I + dcol);
    };
    if (dn0) issue_down(b, dr);
    if (grp0) sdr = load_raw8_stream<true>(f.sdn, (size_t)(r0 + wave) * I + dcol);
    // the shared words
    if (!poll_tagged<2>(shw, shs, tag, plim)) s_fail = 1;
    if (tid < I) s_sha[tid] = value_of(shw[0]);
    if (tid == 0) s_sg = value_of(shw[1]);
    lds_barrier();
    FK_MARK(5);

    // ---------------- P4: down items -----------------------------------------
    // The item's slot activations, one word per thread, then its 64 rows.
    auto down_item = [&](int d, const Raw8<true> (&w)[RG]) {
      const int u_ = d / cpe, rr = (d - u_ * cpe) * DR + wave * RG;
      {
        uint64_t aw[1];
        const uint64_t* as[1] = {tid < I ? a.ws.f_act + (size_t)u_ * I + tid : nullptr};
        aw[0] = as[0] ? load_tagged(as[0]) : 0ull;
        if (!poll_tagged<1>(aw, as, tag, plim)) s_fail = 1;
        if (tid < I) s_ra[tid] = value_of(aw[0]);
      }
      lds_barrier();
      float dd[RG];
  #pragma unroll
      for (int j = 0; j < RG; ++j) dd[j] = dot8_act_lds(w[j], s_ra, lane, I);
      const float v = rows8_sum(dd);
      const int row = rr + (lane >> 3);
      if ((lane & 7) == 0 && row < H) store_tagged(a.ws.f_y + (size_t)u_ * H + row, poison_if(s_fail, v), tag);
      lds_barrier();  // s_ra is rewritten by the next item
    };
    if (dn0) down_item(b, dr);
    for (int d = b + G; d < ndn; d += G) {
      Raw8<true> w[RG];
      issue_down(d, w);
      down_item(d, w);
    }
    FK_MARK(6);

    // ---------------- P5: combine of the workgroup's output rows -------------
    auto final_group = [&](int rg0, const Raw8<true>& ws) {
      const float sh = wave_sum(dot8_act_lds(ws, s_sha, lane, I));
      if (lane == 0) s_sh[wave] = sh;
      if (wave == 0) {
        // lane (k, j) = (l / 8, l % 8): y of slot k at row rg0 + j
        const int k = lane >> 3, j = lane & 7;
        uint64_t yw[1];
        const uint64_t* ys[1] = {k < K ? a.ws.f_y + (size_t)k * H + rg0 + j : nullptr};
        yw[0] = ys[0] ? load_tagged(ys[0]) : 0ull;
        if (!poll_tagged<1>(yw, ys, tag, plim)) s_fail = 1;
        s_yk[lane] = value_of(yw[0]);
      }
      lds_barrier();
      if (wave == 0 && lane < RG) {
        const bool bad_out = s_fail;
        float acc = 0.f;
  #pragma unroll
        for (int k = 0; k < kFusedMaxPairs; ++k)
          if (k < K) acc += s_wpos[k] * s_yk[k * RG + lane];
        acc += s_sg * s_sh[lane];
        const float o = poison_if(bad_out, acc);
        const int r = rg0 + lane;
        f.out[r] = o;
        if (f.layer_out)
          f.layer_out[r] = (rg0 == r0 ? raw_value<BFX>(x_raw[0]) : load_scalar(a.x, BFX ? FK_DTYPE_BF16 : FK_DTYPE_F32, r)) + o;
      }
      lds_barrier();
    };
    if (grp0) {
      FK_MARK(7);
      final_group(r0, sdr);
    }
    for (int grp = b + G; grp < ngrp; grp += G) {
      const int rg0 = grp * RG;
      const Raw8<true> ws = load_raw8_stream<true>(f.sdn, (size_t)(rg0 + wave) * I + dcol);
      final_group(rg0, ws);
    }
  }
  // A failed wait anywhere in the workgroup sets the workspace's error word.
  lds_barrier();
  if (tid == 0 && s_fail) __hip_atomic_fetch_or(err, FK_DEVICE_ERR_BARRIER, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  FK_MARK(8);
  FK_TIMELINE_COMMIT(moe_fused, blockIdx.x);
}

// ---------------------------------------------------------------------------
// Router without grid barrier (T <= 256, E <= 256, H <= 2048).
//
// Workgroup (ub, tb) computes the logits of expert rows 8ub.. (one per
// wavefront) for tokens tu*tb .. tu*tb + tu - 1 (tu from 2 to 32, the
// smallest whose grid is co-resident), in tiles of TU tokens (2 when a
// workgroup has 2, else 4): the row and the first tile's tokens are loaded
// together, each later tile is fetched while the previous one is computed,
// and every tile leaves as one tagged run per token (the launch-tag protocol
// of the single-launch layer, same epoch counter).
// Up to 8 tokens, workgroup 0 then polls every logit and selects every
// token itself (one token per wavefront).  From 9 tokens on, workgroup b
// polls the logits of tokens b, b + grid, .. and computes each top-k with
// one wavefront (a selection is issue-bound, so the tokens go to different
// CUs), writes the token's ids and weights, and publishes the ids as tagged
// words; workgroup 0 polls the T*K ids.  Either way workgroup 0 then
// advances the epoch (the words it polled carry this launch's tag, so every
// workgroup has written logits with it and has read the epoch) and builds
// the routing tables for the expert stage.  The logits are moe_router_kernel's
// (same arithmetic); the selection is the ranked one of the single-launch
// layer (topk_select_ranked): the same ids, weights equal to rounding.
// ---------------------------------------------------------------------------
constexpr int kTagRouterMaxTokens = 256;
constexpr int kTagRouterTile = 4;       // tokens per tile of the logits loop
constexpr int kTagRouterMaxPerWg = 32;  // most tokens per workgroup
// Up to this many tokens workgroup 0 selects them all, one token per
// wavefront.  (Two per wavefront, up to 16 tokens, measured 0.4-0.8 us
// slower at 12-16 tokens than the selections spread over one workgroup per
// token: a selection is VALU-bound, and eight wavefronts share one CU's
// four SIMDs.)
constexpr int kTagRouterSelfTokens = kFusedWaves;
constexpr int kMaskWords = kTagRouterMaxTokens / 32;
// From this many tokens on the tagged router computes its logits on MFMA
// (moe_router_tagged_kernel<.., MF = true>) when the shapes allow: at the
// model's shapes 11.4-11.6 us from 33 to 48 tokens, where the register tiles
// take 11.0 us at 33 tokens and 12.0-12.3 us from 36 on (18.4 against
// 12.6 us at 128).
constexpr int kRouterMfmaMinTokens = 36;
static_assert(kFusedSelWords >= (size_t)kTagRouterMaxTokens * 8, "router selection region too small");
static_assert(kFusedLogitWords >= (size_t)kTagRouterMaxTokens * kFusedMaxExperts, "router logit region too small");

// Routing tables for T <= 256 tokens and E <= 512 experts (one expert per
// thread of a 512-thread workgroup) from s_mask[e * ceil(T/32) + t / 32],
// whose bit t % 32 says that token t chose expert e (a token chooses an
// expert at most once).  Counts are popcounts, offsets their exclusive
// prefix, and pair j = t*K + k goes to offsets[e] + (earlier tokens that
// chose e): the stable order by expert of a counting sort, as
// build_routing_tables gives (records in ws.slots included).
__device__ void build_routing_tables_masks(const int* s_ids, const uint32_t* s_mask, int T, int K, int E, MoeWs ws,
                                           int* s_off) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  __shared__ int s_wtot[kFusedWaves][2];
  const int nw = (T + 31) >> 5;
  int c = 0, first = -1;
  if (tid < E) {
    for (int w = nw - 1; w >= 0; --w) {
      const uint32_t m = s_mask[tid * nw + w];
      c += __popc(m);
      if (m) first = w * 32 + __ffs(m) - 1;
    }
  }
  const int nz = c > 0 ? 1 : 0;
  const int isum = wave_incl_scan(c, lane), inz = wave_incl_scan(nz, lane);
  if (lane == kWave - 1) {
    s_wtot[wave][0] = isum;
    s_wtot[wave][1] = inz;
  }
  __syncthreads();
  int psum = 0, pnz = 0;
  for (int w = 0; w < wave; ++w) {
    psum += s_wtot[w][0];
    pnz += s_wtot[w][1];
  }
  if (tid < E) {
    const int off = psum + isum - c;
    s_off[tid] = off;
    ws.offsets[tid] = off;
    ws.counts[tid] = c;
    if (nz) {
      ws.active[pnz + inz - 1] = tid;
      ws.slots[pnz + inz - 1] = make_int4(tid, off, c, first);  // first pair: lowest token
    }
  }
  const int P = T * K;
  if (tid == 0) {
    int na = 0;
    for (int w = 0; w < kFusedWaves; ++w) na += s_wtot[w][1];
    ws.offsets[E] = P;
    ws.num_active[0] = na;
  }
  __syncthreads();
  for (int j = tid; j < P; j += kFusedWaves * kWave) {
    const int t = j / K, e = s_ids[j];
    const uint32_t* m = s_mask + e * nw;
    int pos = s_off[e] + __popc(m[t >> 5] & ((1u << (t & 31)) - 1u));
    for (int w = 0; w < (t >> 5); ++w) pos += __popc(m[w]);
    ws.perm[pos] = j;
    ws.inverse[j] = pos;
  }
}

// TILED: a workgroup takes more than one tile of tokens (tu > 4).  The
// single-tile variant keeps no prefetch registers (two workgroups per CU)
// and every wavefront sums its tokens' squares beside its dot products; the
// tiled one, VALU-bound, has wavefront t sum token t's squares once for all
// rows and the storing threads apply the scale (same expression, so both
// give the same logits).  Dynamic LDS: workgroup 0's ids [T*K] and token
// masks [E * ceil(T/32)] (sized by the host for this T).
FK_TIMELINE_BUFFER(moe_router)

// MF: the logits as v_mfma_f32_16x16x32_bf16 tiles instead (bf16 router
// weight, H a multiple of 256 up to 2048, E a multiple of 16; the host picks
// it from kRouterMfmaMinTokens tokens on).  Workgroup (ue, ut) takes experts
// 16 ue .. + 15 and tokens 16 ut .. + 15; wavefront w multiplies the K range
// w H/8 .. + H/8: A = the 16 weight rows, B = the tokens x * (off + w_norm)
// as bf16 hi + lo columns (~16 mantissa bits, as the expert stage's
// activations), accumulated in fp32; each lane also sums its x^2 for the
// token's RMSNorm.  The eight partial tiles and sums meet in LDS in wave
// order; the logit is sum * rsqrt(mean(x^2) + eps) + bias.
template <bool BFW, bool BFX, bool BFN, bool TILED, int TU, bool MF = false>
__global__ __launch_bounds__(512) void moe_router_tagged_kernel(RouterArgs a) {
  static_assert(TU <= kTagRouterTile && (!TILED || TU == kTagRouterTile), "tile of tokens");
  extern __shared__ int s_dyn_ids[];
  __shared__ int s_off[kFusedMaxExperts];
  __shared__ float s_chunk[TU][8];
  __shared__ float s_ss[TU];
  __shared__ int s_fail;
  __shared__ __align__(16) TopkLds s_topk[kFusedWaves];
  __shared__ float s_selw[kTagRouterSelfTokens * 8];  // selected weights (ids: s_ids, or s_sel_id)
  __shared__ int s_sel_id[8];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int T = a.T, H = a.H, E = a.E, K = a.K, nch = H >> 3;
  const int nrb = (E + 7) / 8, tu = a.tu;
  const int ub = blockIdx.x % nrb, tb = blockIdx.x / nrb;
  const int e = ub * 8 + wave, t0 = tb * tu, ntok = max(0, min(tu, T - t0));
  WaitHeader hdr = load_wait_header(a.ws.tickets, kTicketEpoch);  // (limits taken after the first loads)
  if (tid == 0) s_fail = 0;
  FK_TIMELINE_DECL;
  FK_MARK(0);  // (timeline markers: diagnostic builds only)

  WaitLimits wl{};
  uint32_t tag = 0;
  if constexpr (MF) {
    static_assert(BFW, "the MFMA logits take a bf16 router weight");
    __shared__ float s_macc[kFusedWaves][16][17];
    __shared__ float s_mss[kFusedWaves][16];
    const int nue = E >> 4, ue = blockIdx.x % nue, ut = blockIdx.x / nue;
    const int e0 = ue * 16, tm0 = ut * 16;
    const int kw = H >> 3, ks = kw >> 5;  // K range per wavefront, its 32-wide steps (<= 8)
    const int n = lane & 15, g4 = lane >> 4;
    const int tok = min(tm0 + n, T - 1);  // (columns past the last token repeat it; not stored)
    // every load first: the weight rows (A operands), the token chunks and
    // the norm weight of this lane's k groups, then the bias word
    u32x4 wa[8];
    Raw8<BFX> xb[8];
    Raw8<BFN> nb[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      if (s < ks) {
        const int k = wave * kw + s * 32 + g4 * 8;
        wa[s] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(a.W) + (size_t)(e0 + n) * H + k);
        xb[s] = load_raw8<BFX>(a.x, (size_t)tok * H + k);
        nb[s] = load_raw8<BFN>(a.nw, (size_t)k);
      }
    }
    const int brow = min(e0 + (tid & 15), E - 1);
    const void* bsrc = a.bias ? a.bias : a.W;
    const int bdt = a.bias ? a.bias_dt : FK_DTYPE_F32;
    const uint32_t bias_word = elem_word(bsrc, bdt, brow);
    wl = hdr.limits();
    tag = wl.tag;
    f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float ss = 0.f;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      if (s < ks) {
        float x8[8], n8[8], y[8];
        raw8_to_f32<BFX>(xb[s], x8);
        raw8_to_f32<BFN>(nb[s], n8);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          ss = fmaf(x8[q], x8[q], ss);
          y[q] = x8[q] * (a.off + n8[q]);
        }
        u32x4 vh, vl;
        split_hi_lo8(y, vh, vl);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, wa[s]), __builtin_bit_cast(bf16x8_t, vh), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, wa[s]), __builtin_bit_cast(bf16x8_t, vl), acc, 0, 0, 0);
      }
    }
    // lanes n, n + 16, n + 32, n + 48 hold token n's k groups
    ss += __shfl_xor(ss, 16);
    ss += __shfl_xor(ss, 32);
    if (g4 == 0) s_mss[wave][n] = ss;
#pragma unroll
    for (int q = 0; q < 4; ++q) s_macc[wave][g4 * 4 + q][n] = acc[q];  // row (expert) g4*4+q, column (token) n
    __syncthreads();
    if (tid < 256) {
      const int r = tid & 15, c = tid >> 4, t = tm0 + c, ee = e0 + r;
      float d = 0.f, st = 0.f;
#pragma unroll
      for (int w = 0; w < kFusedWaves; ++w) {
        d += s_macc[w][r][c];
        st += s_mss[w][c];
      }
      const float bias = a.bias ? elem_value(bias_word, bsrc, bdt, brow) : 0.f;
      const float v = d * rsqrtf(st / (float)H + a.eps) + bias;
      if (t < T && ee < E) {
        const size_t o = (size_t)t * E + ee;
        a.logits[o] = v;
        store_tagged(a.ws.f_logits + o, v, tag);
      }
    }
    FK_MARK(1);
  } else {
    // ---- logits of rows 8ub.. for tokens t0 .. t0 + ntok - 1 ----------------
    // Every load of the row is issued with the first tile's tokens, before the
    // first use (the norm weight with a compile-time dtype: a run-time dtype
    // test would wait for every load before it); token indices past this
    // workgroup's last token repeat it (cache hits, not other tokens' lines).
    const int tlast = t0 + ntok - 1;
    const bool row = e < E;
    const int erow = row ? e : 0;
    Raw8<BFX> xr[TU][4];
    float wn[4][8];
    // bias of the row whose logits this thread applies it to: the wavefront's
    // row, or (tiled) the row this thread stores (thread t*8 + l: row 8ub + l);
    // its word is loaded after the rows (unconditionally: a missing bias reads
    // the router weight and is dropped), decoded where it is added
    const int brow = TILED ? min(ub * 8 + (tid & 7), E - 1) : erow;
    const void* bsrc = a.bias ? a.bias : a.W;
    const int bdt = a.bias ? a.bias_dt : FK_DTYPE_F32;
    uint32_t bias_word;
    {
      Raw8<BFW> wr[4];
      Raw8<BFN> nr[4];
  #pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int cc = min(lane + kWave * j, nch - 1);
        wr[j] = load_raw8<BFW>(a.W, (size_t)erow * H + (size_t)cc * 8);
  #pragma unroll
        for (int t = 0; t < TU; ++t)
          xr[t][j] = load_raw8<BFX>(a.x, (size_t)min(t0 + t, tlast) * H + (size_t)cc * 8);
        nr[j] = load_raw8<BFN>(a.nw, (size_t)cc * 8);
      }
      bias_word = elem_word(bsrc, bdt, brow);
  #pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int c = lane + kWave * j;
        float w8[8], n8[8];
        raw8_to_f32<BFN>(nr[j], n8);
        raw8_to_f32<BFW>(wr[j], w8);
  #pragma unroll
        for (int q = 0; q < 8; ++q) wn[j][q] = c < nch ? w8[q] * (a.off + n8[q]) : 0.f;
      }
    }
    const bool bias_on = a.bias && (TILED ? tid < 8 * TU && ub * 8 + (tid & 7) < E : row);
    const float bias = bias_on ? elem_value(bias_word, bsrc, bdt, brow) : 0.f;
    wl = hdr.limits();
    tag = wl.tag;
    for (int tt = 0; tt < ntok; tt += TU) {
      const int nt = min(TU, ntok - tt);
      // next tile's tokens, fetched while this tile is computed (bf16 tokens;
      // fp32 ones are fetched after it, which keeps the registers in budget)
      constexpr bool PF = BFX && TILED;
      Raw8<BFX> xn[PF ? TU : 1][4];
      const bool more = TILED && tt + TU < ntok;
      if (PF && more) {
  #pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int cc = min(lane + kWave * j, nch - 1);
  #pragma unroll
          for (int t = 0; t < (PF ? TU : 1); ++t)
            xn[t][j] = load_raw8<BFX>(a.x, (size_t)min(t0 + tt + TU + t, tlast) * H + (size_t)cc * 8);
        }
      }
      // Wavefront t < TU also sums the squares of token t (the RMSNorm scale
      // is shared by every row); the storing threads apply it.
      float mine = 0.f;  // lane t < nt: dot of token t0 + tt + t with the row
  #pragma unroll
      for (int t = 0; t < TU; ++t) {
        if (t < nt) {
          if constexpr (!TILED) {
            float ss = 0.f, d = 0.f;
  #pragma unroll
            for (int j = 0; j < 4; ++j) {
              const bool in = lane + kWave * j < nch;
              float x8[8];
              raw8_to_f32<BFX>(xr[t][j], x8);
  #pragma unroll
              for (int q = 0; q < 8; ++q) {
                const float xv = in ? x8[q] : 0.f;
                ss = fmaf(xv, xv, ss);
                d = fmaf(xv, wn[j][q], d);
              }
            }
            ss = wave_sum(ss);
            d = wave_sum(d);
            mine = lane == t ? d * rsqrtf(ss / (float)H + a.eps) + bias : mine;
            continue;
          }
          float d = 0.f;
  #pragma unroll
          for (int j = 0; j < 4; ++j) {
            const bool in = lane + kWave * j < nch;
            float x8[8];
            raw8_to_f32<BFX>(xr[t][j], x8);
  #pragma unroll
            for (int q = 0; q < 8; ++q) d = fmaf(in ? x8[q] : 0.f, wn[j][q], d);
          }
          d = wave_sum(d);
          mine = lane == t ? d : mine;
          if (wave == t) {  // (a branch of its own: a per-element test costs every wavefront)
            float ss = 0.f;
  #pragma unroll
            for (int j = 0; j < 4; ++j) {
              const bool in = lane + kWave * j < nch;
              float x8[8];
              raw8_to_f32<BFX>(xr[t][j], x8);
  #pragma unroll
              for (int q = 0; q < 8; ++q) {
                const float xv = in ? x8[q] : 0.f;
                ss = fmaf(xv, xv, ss);
              }
            }
            ss = wave_sum(ss);
            if (lane == 0) s_ss[t] = ss;
          }
        }
      }
      if (lane < nt) s_chunk[lane][wave] = mine;
      __syncthreads();
      if (tid < 8 * nt) {
        const int t = tid >> 3, l = tid & 7, ee = ub * 8 + l;
        if (ee < E) {
          const float v = TILED ? s_chunk[t][l] * rsqrtf(s_ss[t] / (float)H + a.eps) + bias : s_chunk[t][l];
          const size_t o = (size_t)(t0 + tt + t) * E + ee;
          a.logits[o] = v;
          store_tagged(a.ws.f_logits + o, v, tag);
        }
      }
      __syncthreads();  // s_chunk is rewritten by the next tile
      if (tt == 0) FK_MARK(1);
      if (more) {
  #pragma unroll
        for (int t = 0; t < TU; ++t)
  #pragma unroll
          for (int j = 0; j < 4; ++j) {
            if constexpr (PF) xr[t][j] = xn[t][j];
            else xr[t][j] = load_raw8<BFX>(a.x, (size_t)min(t0 + tt + TU + t, tlast) * H +
                                                    (size_t)min(lane + kWave * j, nch - 1) * 8);
          }
      }
    }
  
  }

  FK_MARK(2);
  const int nmw = (T + 31) >> 5;
  int* s_ids = s_dyn_ids;
  uint32_t* s_mask = reinterpret_cast<uint32_t*>(s_dyn_ids + T * K);  // [E][nmw]
  if (T <= kTagRouterSelfTokens) {
    // ---- few tokens: workgroup 0 selects every token itself ----------------
    // (wavefront w: token w), with no hand-off of the ids through memory.  Its logits polls cover every workgroup's logits, so they also
    // show that every workgroup has read the epoch.
    if (blockIdx.x != 0) {
      if (tid == 0 && s_fail)
        __hip_atomic_fetch_or(&a.ws.tickets[kTicketError], FK_DEVICE_ERR_BARRIER, __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
      FK_MARK(3);
      FK_TIMELINE_COMMIT(moe_router, blockIdx.x);
      return;
    }
    for (int i = tid; i < E * nmw; i += kFusedWaves * kWave) s_mask[i] = 0u;
    // Wavefront w: token w (tokens w + 8 s with more per wavefront); the
    // ranked selections write ids and weights to LDS.
    constexpr int S = kTagRouterSelfTokens / kFusedWaves;
    uint64_t w[S * 4];
    const uint64_t* srcs[S * 4];
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = wave + kFusedWaves * s, ex = lane + kWave * j;
        srcs[s * 4 + j] = t < T && ex < E ? a.ws.f_logits + (size_t)t * E + ex : nullptr;
        w[s * 4 + j] = srcs[s * 4 + j] ? load_tagged(srcs[s * 4 + j]) : 0ull;
      }
    const bool ok = poll_tagged<S * 4>(w, srcs, tag, wl.poll);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int t = wave + kFusedWaves * s;
      if (t < T) {
        float l[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) l[j] = srcs[s * 4 + j] ? value_of(w[s * 4 + j]) : -INFINITY;
        topk_select_ranked(l, E, K, lane, &s_topk[wave], s_ids + t * K, s_selw + t * K);
      }
    }
    if (!ok) s_fail = 1;
    __syncthreads();  // s_mask cleared, selections and s_fail in LDS
    const bool bad = s_fail != 0;
    for (int j = tid; j < T * K; j += kFusedWaves * kWave) {
      // (after a failed wait: stale logits, ids in range, weights poisoned)
      const int sid = s_ids[j], t = j / K;
      const float swt = poison_if(bad, s_selw[j]);
      a.ids_out[j] = sid;
      a.w_out[j] = swt;
      a.ws.ids32[j] = sid;
      a.ws.wts[j] = swt;
      atomicOr(&s_mask[sid * nmw + (t >> 5)], 1u << (t & 31));
    }
    __syncthreads();
    if (tid == 0) {
      if (!s_fail) store_coherent(&a.ws.tickets[kTicketEpoch], tag);
      else __hip_atomic_fetch_or(&a.ws.tickets[kTicketError], FK_DEVICE_ERR_BARRIER, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
    }
    FK_MARK(4);
    build_routing_tables_masks(s_ids, s_mask, T, K, E, a.ws, s_off);
    FK_MARK(5);
    FK_TIMELINE_COMMIT(moe_router, blockIdx.x);
    return;
  }
  // ---- top-k of tokens blockIdx.x, blockIdx.x + grid, .. ------------------
  if (wave == 0) {
    constexpr int NJE = kFusedMaxExperts / kWave;
    for (int t = blockIdx.x; t < T; t += gridDim.x) {
      uint64_t w[NJE];
      const uint64_t* srcs[NJE];
#pragma unroll
      for (int j = 0; j < NJE; ++j) {
        const int ex = lane + kWave * j;
        srcs[j] = ex < E ? a.ws.f_logits + (size_t)t * E + ex : nullptr;
        w[j] = srcs[j] ? load_tagged(srcs[j]) : 0ull;
      }
      const bool ok = poll_tagged<NJE>(w, srcs, tag, wl.poll);
      if (!ok) s_fail = 1;
      float l[NJE];
#pragma unroll
      for (int j = 0; j < NJE; ++j) l[j] = srcs[j] ? value_of(w[j]) : -INFINITY;
      topk_select_ranked(l, E, K, lane, &s_topk[0], s_sel_id, s_selw);
      // (one wavefront: its LDS writes are done once the count drains)
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (lane < K) {
        // (stale logits after a failed wait: ids in range, weights poisoned)
        const int id = s_sel_id[lane];
        const float wt = poison_if(!ok, s_selw[lane]);
        const int j = t * K + lane;
        a.ids_out[j] = id;
        a.w_out[j] = wt;
        a.ws.ids32[j] = id;
        a.ws.wts[j] = wt;
        store_tagged(a.ws.f_sel + j, __int_as_float(id), tag);
      }
    }
  }
  if (blockIdx.x != 0) {
    if (tid == 0 && s_fail)
      __hip_atomic_fetch_or(&a.ws.tickets[kTicketError], FK_DEVICE_ERR_BARRIER, __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
    FK_MARK(3);
    FK_TIMELINE_COMMIT(moe_router, blockIdx.x);
    return;
  }

  // ---- workgroup 0: every token's ids, epoch, routing tables --------------
  for (int i = tid; i < E * nmw; i += kFusedWaves * kWave) s_mask[i] = 0u;
  __syncthreads();
  const int P = T * K;  // <= 2048: up to 4 ids per thread
  {
    constexpr int NP = kTagRouterMaxTokens * 8 / (kFusedWaves * kWave);
    uint64_t w[NP];
    const uint64_t* srcs[NP];
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int j = tid + i * kFusedWaves * kWave;
      srcs[i] = j < P ? a.ws.f_sel + j : nullptr;
      w[i] = srcs[i] ? load_tagged(srcs[i]) : 0ull;
    }
    if (!poll_tagged<NP>(w, srcs, tag, wl.poll)) s_fail = 1;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int j = tid + i * kFusedWaves * kWave;
      if (j < P) {
        // (clamped: after a failed poll the word may come from another launch)
        const int id = min(max(__float_as_int(value_of(w[i])), 0), E - 1);
        const int t = j / K;
        s_ids[j] = id;
        atomicOr(&s_mask[id * nmw + (t >> 5)], 1u << (t & 31));
      }
    }
  }
  __syncthreads();
  if (tid == 0) {
    // (not after a failed wait: a workgroup that has not read the epoch yet
    // would take the next launch's tag; the error word, which the expert
    // stage and every later launch on this workspace read, poisons them)
    if (!s_fail) store_coherent(&a.ws.tickets[kTicketEpoch], tag);
    else __hip_atomic_fetch_or(&a.ws.tickets[kTicketError], FK_DEVICE_ERR_BARRIER, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
  }
  FK_MARK(4);
  build_routing_tables_masks(s_ids, s_mask, T, K, E, a.ws, s_off);
  FK_MARK(5);
  FK_TIMELINE_COMMIT(moe_router, blockIdx.x);
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
static int check_ws(void* ws, size_t bytes, int T, int K, int E, int I, int H, MoeWs* out) {
  size_t need = moe_ws_layout(T, K, E, I, H, nullptr, out);
  if (!ws) return fail(FK_ERR_WORKSPACE, "workspace is NULL (need %zu bytes)", need);
  if (bytes < need) return fail(FK_ERR_WORKSPACE, "workspace has %zu bytes, need %zu", bytes, need);
  if (!aligned16(ws)) return fail(FK_ERR_ALIGNMENT, "workspace must be 16-byte aligned");
  moe_ws_layout(T, K, E, I, H, reinterpret_cast<char*>(ws), out);
  return FK_OK;
}

#define FK_DISPATCH_BOOL(cond, NAME, ...) \
  if (cond) {                             \
    constexpr bool NAME = true;           \
    __VA_ARGS__                           \
  } else {                                \
    constexpr bool NAME = false;          \
    __VA_ARGS__                           \
  }

// norm_dt / gate_dt: the router's norm weight and the shared-expert gate
// weight, which the single-launch kernel reads as bf16 (gate_dt is ignored
// when there is no gate weight).
static bool fused_eligible(int T, int H, int I, int E, int K, int router_dt, int expert_dt, bool has_shared, int norm_dt,
                           bool has_gate, int gate_dt) {
  return T >= 1 && T <= kFusedMaxTokens && H <= 2048 && H % 8 == 0 && I <= 512 && I % kFusedChunk == 0 && E <= kFusedMaxExperts && K <= 8 &&
         router_dt == FK_DTYPE_BF16 && expert_dt == FK_DTYPE_BF16 && has_shared && norm_dt == FK_DTYPE_BF16 &&
         (!has_gate || gate_dt == FK_DTYPE_BF16);
}

template <bool BX>
static int launch_fused_t(const FusedArgs& fa, hipStream_t stream) {
  static int cap_cache[64] = {0};
  const int cap = resident_capacity(moe_fused_kernel<BX, false>, 512, 0, cap_cache);
  const int cus = device_cus();
  const int G = cap < cus ? cap : cus;  // one workgroup per CU
  if (G < 1) return fail(FK_ERR_UNSUPPORTED, "fused MoE kernel does not fit on this device");
  if (G > kFusedMaxGrid) return fail(FK_ERR_UNSUPPORTED, "fused MoE grid %d exceeds %d workgroups", G, kFusedMaxGrid);
  // one workgroup per gate/up block (16 intermediates of a slot), per down
  // item (64 rows of a slot) and per row group (8 output rows)
  const int K = fa.r.K, H = fa.r.H, I = fa.I;
  const bool fast = G == K * (I / kFusedChunk) && G == K * ((H + 63) / 64) && G * 8 == H;
  if (fast) hipLaunchKernelGGL((moe_fused_kernel<BX, true>), dim3(G), dim3(512), 0, stream, fa);
  else hipLaunchKernelGGL((moe_fused_kernel<BX, false>), dim3(G), dim3(512), 0, stream, fa);
  return check_launch("moe_fused_kernel");
}

template <bool BW, bool BX, int NJ, int NJE>
static int launch_router_t(const RouterArgs& ra, hipStream_t stream) {
  static int cap_cache[64] = {0};
  auto kernel = moe_router_kernel<BW, BX, NJ, NJE>;
  const int cap = resident_capacity(kernel, 256, 0, cap_cache);
  const int gx = (ra.E + 3) / 4;
  if (cap < gx) return fail(FK_ERR_UNSUPPORTED, "router grid %d exceeds co-resident capacity %d", gx, cap);
  int gy = (ra.T + 15) / 16;
  if (gy > cap / gx) gy = cap / gx;
  if (gy < 1) gy = 1;
  hipLaunchKernelGGL(kernel, dim3(gx, gy), dim3(256), 0, stream, ra);
  return check_launch("moe_router_kernel");
}

static bool tagged_router_eligible(const RouterArgs& ra) {
  return ra.T <= kTagRouterMaxTokens && ra.E <= kFusedMaxExperts && ra.H <= 2048 && ra.K <= 8;
}

template <bool BW, bool BX, bool BN>
static int launch_router_tagged_t(const RouterArgs& ra_in, hipStream_t stream) {
  static int cap_cache[3][64] = {{0}};
  constexpr size_t kMaxShmAll = ((size_t)kTagRouterMaxTokens * 8 + (size_t)kFusedMaxExperts * kMaskWords) * 4;
  if constexpr (BW) {
    // MFMA logits: one workgroup per 16 experts x 16 tokens
    if (ra_in.T >= kRouterMfmaMinTokens && ra_in.H % 256 == 0 && ra_in.H <= 2048 && ra_in.E % 16 == 0) {
      auto kernel = moe_router_tagged_kernel<true, BX, BN, false, 2, true>;
      const int units = (ra_in.E / 16) * ((ra_in.T + 15) / 16);
      const int cap = resident_capacity(kernel, 512, kMaxShmAll, cap_cache[2]);
      if (units <= cap) {
        const size_t shm = ((size_t)ra_in.T * ra_in.K + (size_t)ra_in.E * ((ra_in.T + 31) / 32)) * 4;
        hipLaunchKernelGGL(kernel, dim3(units), dim3(512), shm, stream, ra_in);
        return check_launch("moe_router_tagged_kernel");
      }
    }
  }
  // Workgroup 0 waits for every other workgroup's logits: all must be
  // resident.  The fewest tokens per workgroup (2, 4, 8, .. 32) whose grid
  // is co-resident; one tile per workgroup (tu <= 4) takes the single-tile
  // variant, whose smaller register budget fits more workgroups.
  const int nrb = (ra_in.E + 7) / 8;
  RouterArgs ra = ra_in;
  auto pick = [&](int cap) {
    int tu = 2;
    while (tu < kTagRouterMaxPerWg && nrb * ((ra.T + tu - 1) / tu) > cap) tu *= 2;
    return tu;
  };
  // (capacities are taken at the largest dynamic LDS, T = 256)
  constexpr size_t kMaxShm = ((size_t)kTagRouterMaxTokens * 8 + (size_t)kFusedMaxExperts * kMaskWords) * 4;
  const int cap1 = resident_capacity(moe_router_tagged_kernel<BW, BX, BN, false, kTagRouterTile>, 512, kMaxShm, cap_cache[0]);
  ra.tu = pick(cap1);
  int cap = cap1;
  // (a two-token tile issues only two tokens' loads; its register budget is
  // within the four-token tile's, so cap1 holds for it)
  auto kernel = ra.tu <= 2 ? moe_router_tagged_kernel<BW, BX, BN, false, 2>
                           : moe_router_tagged_kernel<BW, BX, BN, false, kTagRouterTile>;
  if (ra.tu > kTagRouterTile) {
    kernel = moe_router_tagged_kernel<BW, BX, BN, true, kTagRouterTile>;
    cap = resident_capacity(kernel, 512, kMaxShm, cap_cache[1]);
    ra.tu = pick(cap);
  }
  const int units = nrb * ((ra.T + ra.tu - 1) / ra.tu);
  if (units > cap) return fail(FK_ERR_UNSUPPORTED, "router grid %d exceeds co-resident capacity %d", units, cap);
  const size_t shm = ((size_t)ra.T * ra.K + (size_t)ra.E * ((ra.T + 31) / 32)) * 4;
  hipLaunchKernelGGL(kernel, dim3(units), dim3(512), shm, stream, ra);
  return check_launch("moe_router_tagged_kernel");
}

static int launch_router(const RouterArgs& ra, int router_dt, int hidden_dt, hipStream_t stream) {
  const bool bfw = router_dt == FK_DTYPE_BF16, bfx = hidden_dt == FK_DTYPE_BF16;
  if (tagged_router_eligible(ra)) {
    int st = FK_OK;
    const bool bfn = ra.nw_dt == FK_DTYPE_BF16;
    FK_DISPATCH_BOOL(bfw, BW, FK_DISPATCH_BOOL(bfx, BX, FK_DISPATCH_BOOL(bfn, BN, {
      st = launch_router_tagged_t<BW, BX, BN>(ra, stream);
    })))
    return st;
  }
  const bool wide = ra.H > 2048, many = ra.E > 256;
  int st = FK_OK;
  FK_DISPATCH_BOOL(bfw, BW, FK_DISPATCH_BOOL(bfx, BX, {
    if (wide) st = many ? launch_router_t<BW, BX, 8, 16>(ra, stream) : launch_router_t<BW, BX, 8, 4>(ra, stream);
    else st = many ? launch_router_t<BW, BX, 4, 16>(ra, stream) : launch_router_t<BW, BX, 4, 4>(ra, stream);
  }))
  return st;
}

// Batched expert stage on MFMA: gate/up then down (see moe_gateup_mfma_kernel).
static int launch_experts_mfma(const ExpertArgs& ea, int slots, hipStream_t stream) {
  static bool attr_set[64] = {false};
  const size_t gu_shm = std::max((size_t)16 * ((size_t)ea.H * 2 + 16), (size_t)kGuMfmaWaves * 512 * sizeof(float));
  const bool dn_small = (long long)ea.T * ea.K <= (long long)kDnMfmaSmallPairs * ea.E;
  const int dn_rows = dn_small ? kDnMfmaRowsSmall : kDnMfmaRows;
  const size_t dn_shm = std::max((size_t)16 * kDnMfmaWaves * ((size_t)ea.I / kDnMfmaWaves * 2 + 16),
                                 (size_t)kDnMfmaWaves * dn_rows * 16 * sizeof(float));
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return fail(FK_ERR_LAUNCH, "no current HIP device");
  if (!attr_set[dev]) {
    // (the largest need, H = 2048: 65,792 bytes)
    const int max_gu = 16 * (2048 * 2 + 16);
    for (const void* k : {reinterpret_cast<const void*>(moe_gateup_mfma_kernel<2>),
                          reinterpret_cast<const void*>(moe_gateup_mfma_kernel<4>),
                          reinterpret_cast<const void*>(moe_gateup_mfma_kernel<8>)})
      if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, max_gu) != hipSuccess)
        return fail(FK_ERR_LAUNCH, "cannot reserve %d bytes of LDS for the MFMA gate/up kernel", max_gu);
    attr_set[dev] = true;
  }
  const dim3 gu_grid(slots * (ea.I / kGuMfmaRows)), gu_block(kGuMfmaWaves * kWave);
  if (ea.H == 2048) hipLaunchKernelGGL(moe_gateup_mfma_kernel<8>, gu_grid, gu_block, gu_shm, stream, ea);
  else if (ea.H == 1024) hipLaunchKernelGGL(moe_gateup_mfma_kernel<4>, gu_grid, gu_block, gu_shm, stream, ea);
  else hipLaunchKernelGGL(moe_gateup_mfma_kernel<2>, gu_grid, gu_block, gu_shm, stream, ea);
  int st = check_launch("moe_gateup_mfma_kernel");
  if (st) return st;
  const dim3 dn_grid(slots * (ea.H / dn_rows)), dn_block(kDnMfmaWaves * kWave);
  if (dn_small) {
    if (ea.I == 512) hipLaunchKernelGGL((moe_down_mfma_kernel<4, kDnMfmaRowsSmall / 16>), dn_grid, dn_block, dn_shm, stream, ea);
    else hipLaunchKernelGGL((moe_down_mfma_kernel<2, kDnMfmaRowsSmall / 16>), dn_grid, dn_block, dn_shm, stream, ea);
  } else {
    if (ea.I == 512) hipLaunchKernelGGL((moe_down_mfma_kernel<4, kDnMfmaRows / 16>), dn_grid, dn_block, dn_shm, stream, ea);
    else hipLaunchKernelGGL((moe_down_mfma_kernel<2, kDnMfmaRows / 16>), dn_grid, dn_block, dn_shm, stream, ea);
  }
  return check_launch("moe_down_mfma_kernel");
}

static int launch_experts(const ExpertArgs& ea, int expert_dt, hipStream_t stream) {
  const bool bfw = expert_dt == FK_DTYPE_BF16, bfx = ea.x_dt == FK_DTYPE_BF16;
  const bool wide = ea.H > 2048;
  const int max_active = ea.T * ea.K < ea.E ? ea.T * ea.K : ea.E;
  const int slots = max_active + (ea.has_shared ? 1 : 0);
  int st = FK_OK;
  if (ea.T >= kMfmaMinTokens && bfw && bfx && mfma_expert_shapes_ok(ea.H, ea.I)) {
    st = launch_experts_mfma(ea, slots, stream);
    if (st) return st;
  } else {
    const int gu_grid = slots * (ea.I / kGateUpRows);
    FK_DISPATCH_BOOL(bfw, BW, FK_DISPATCH_BOOL(bfx, BX, {
      if (wide) {
        hipLaunchKernelGGL((moe_gateup_kernel<BW, BX, 8>), dim3(gu_grid), dim3(256), 0, stream, ea);
      } else {
        hipLaunchKernelGGL((moe_gateup_kernel<BW, BX, 4>), dim3(gu_grid), dim3(256), 0, stream, ea);
      }
    }))
    st = check_launch("moe_gateup_kernel");
    if (st) return st;

    const int dn_grid = slots * ((ea.H + kDownRows - 1) / kDownRows);
    const bool wide_i = ea.I > 512;
    FK_DISPATCH_BOOL(bfw, BW, {
      if (wide_i) hipLaunchKernelGGL((moe_down_kernel<BW, 2>), dim3(dn_grid), dim3(256), 0, stream, ea);
      else hipLaunchKernelGGL((moe_down_kernel<BW, 1>), dim3(dn_grid), dim3(256), 0, stream, ea);
    })
    st = check_launch("moe_down_kernel");
    if (st) return st;
  }
  const size_t total = (size_t)ea.T * ea.H;
  const bool lo = ea.layer_out != nullptr;
  const dim3 cgrid((unsigned)((total + 255) / 256));
  FK_DISPATCH_BOOL(bfx, BX, FK_DISPATCH_BOOL(lo, LO, {
    hipLaunchKernelGGL((moe_combine_kernel<BX, LO>), cgrid, dim3(256), 0, stream, ea);
  }))
  return check_launch("moe_combine_kernel");
}

static int validate_common(int T, int H, int E, int K) {
  if (T < 1) return fail(FK_ERR_INVALID, "tokens must be positive (got %d)", T);
  if (H < 8 || H % 8) return fail(FK_ERR_ALIGNMENT, "hidden_size must be a positive multiple of 8 (got %d)", H);
  if (H > 4096) return fail(FK_ERR_UNSUPPORTED, "hidden_size must be <= 4096 (got %d)", H);
  if (E < 1 || E > kMaxExperts) return fail(FK_ERR_UNSUPPORTED, "num_experts must be in [1, %d] (got %d)", kMaxExperts, E);
  if (K < 1 || K > 8 || K > E) return fail(FK_ERR_INVALID, "top_k must be in [1, min(8, num_experts)] (got %d)", K);
  if ((long long)T * K > kMaxPairs) return fail(FK_ERR_UNSUPPORTED, "tokens * top_k must be <= %d", kMaxPairs);
  return FK_OK;
}

static int validate_experts(const void* hidden, int hidden_dt, const void* gu, const void* dn, int expert_dt,
                            const void* sgu, const void* sdn, const void* sg, int sg_dt, int T, int H, int I,
                            int E, int K) {
  int st = validate_common(T, H, E, K);
  if (st) return st;
  if (!is_float_dtype(hidden_dt) || !is_float_dtype(expert_dt)) return fail(FK_ERR_DTYPE, "hidden/expert dtype must be f32 or bf16");
  if (sg && !is_float_dtype(sg_dt)) return fail(FK_ERR_DTYPE, "shared_gate dtype must be f32 or bf16");
  if (I < 8 || I % 8) return fail(FK_ERR_ALIGNMENT, "intermediate must be a positive multiple of 8 (got %d)", I);
  if (I > 1024) return fail(FK_ERR_UNSUPPORTED, "intermediate must be <= 1024 (got %d)", I);
  if (!hidden || !gu || !dn) return fail(FK_ERR_INVALID, "hidden and expert weights must be non-NULL");
  if ((sgu == nullptr) != (sdn == nullptr)) return fail(FK_ERR_INVALID, "shared_gate_up and shared_down must both be set or both NULL");
  if (!aligned16(hidden) || !aligned16(gu) || !aligned16(dn) || (sgu && !aligned16(sgu)) || (sdn && !aligned16(sdn)))
    return fail(FK_ERR_ALIGNMENT, "hidden and expert weights must be 16-byte aligned");
  return FK_OK;
}

static ExpertArgs make_expert_args(const void* hidden, int hidden_dt, const void* gu, const void* dn,
                                   const void* sgu, const void* sdn, const void* sg, int sg_dt, int T, int H,
                                   int I, int E, int K, float* out, float* layer_out, const MoeWs& ws) {
  ExpertArgs ea;
  ea.x = hidden;
  ea.x_dt = hidden_dt;
  ea.gu = gu;
  ea.dn = dn;
  ea.sgu = sgu;
  ea.sdn = sdn;
  ea.sg = sgu ? sg : nullptr;
  ea.sg_dt = sg_dt;
  ea.T = T;
  ea.H = H;
  ea.I = I;
  ea.E = E;
  ea.K = K;
  ea.has_shared = sgu != nullptr;
  ea.out = out;
  ea.layer_out = layer_out;
  ea.ws = ws;
  return ea;
}

// ---------------------------------------------------------------------------
// Allocation-free MoE layer: the workspace of fk_moe_layer lives in a
// file-scope device array instead of caller memory.  Each GPU the library
// runs on holds its own copy (kNoAllocScratchBytes) until the process ends;
// every call on that GPU shares it.
// ---------------------------------------------------------------------------
constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[64] = {nullptr};

__global__ __launch_bounds__(256) void zero_fill_kernel(u32x4* p, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256)
    p[i] = u32x4{0u, 0u, 0u, 0u};
}

// Device address of this GPU's scratch array.  On the first call on a
// device (with that device current) the address is taken with
// hipGetSymbolAddress -- the array's name is only a host-side stand-in --
// and the array is zero-filled on `stream` (the workspace contract: zero
// once, then self-resetting), and waited for.  That first call must not be
// under graph capture: a captured fill would re-zero the launch epoch on
// every replay.
static int noalloc_scratch(hipStream_t stream, void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return fail(FK_ERR_LAUNCH, "no current HIP device");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) != hipSuccess) return fail(FK_ERR_LAUNCH, "hipStreamIsCapturing failed");
    if (cs != hipStreamCaptureStatusNone)
      return fail(FK_ERR_UNSUPPORTED,
                  "the first fk_moe_layer_noalloc call on a device clears its scratch and must not be captured");
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return fail(FK_ERR_LAUNCH, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    hipLaunchKernelGGL(zero_fill_kernel, dim3(1024), dim3(256), 0, stream, reinterpret_cast<u32x4*>(p),
                       kNoAllocScratchBytes / 16);
    const int st = check_launch("zero_fill_kernel");
    if (st) return st;
    // Wait for the fill: a first call from another stream (or thread, once
    // the lock is released) must find the array cleared.
    const hipError_t se = hipStreamSynchronize(stream);
    if (se != hipSuccess) return fail(FK_ERR_LAUNCH, "clearing the scratch array: %s", hipGetErrorString(se));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return FK_OK;
}

}  // namespace fk

using namespace fk;

extern "C" {

size_t fk_moe_workspace_bytes(int tokens, int top_k, int num_experts, int intermediate, int hidden_size) {
  if (tokens < 1 || top_k < 1 || num_experts < 1 || intermediate < 1 || hidden_size < 1) return 0;
  MoeWs ws;
  return moe_ws_layout(tokens, top_k, num_experts, intermediate, hidden_size, nullptr, &ws);
}

int fk_moe_router(const void* hidden, int hidden_dtype, const void* norm_weight, int norm_dtype,
                  const void* router_weight, int router_dtype, const void* router_bias, int bias_dtype,
                  int tokens, int hidden_size, int num_experts, int top_k, float eps, float norm_offset,
                  float* logits, int64_t* topk_ids, float* topk_weights, void* workspace,
                  size_t workspace_bytes, void* stream) {
  int st = validate_common(tokens, hidden_size, num_experts, top_k);
  if (st) return st;
  if (!is_float_dtype(hidden_dtype) || !is_float_dtype(norm_dtype) || !is_float_dtype(router_dtype) ||
      (router_bias && !is_float_dtype(bias_dtype)))
    return fail(FK_ERR_DTYPE, "router inputs must be f32 or bf16");
  if (!hidden || !norm_weight || !router_weight || !logits || !topk_ids || !topk_weights)
    return fail(FK_ERR_INVALID, "router pointers must be non-NULL");
  if (!aligned16(hidden) || !aligned16(router_weight) || !aligned16(norm_weight))
    return fail(FK_ERR_ALIGNMENT, "hidden, norm_weight and router_weight must be 16-byte aligned");
  MoeWs ws;
  // The router only needs the routing tables, which precede the
  // size-dependent activation buffers in every layout.
  st = check_ws(workspace, workspace_bytes, tokens, top_k, num_experts, 0, 0, &ws);
  if (st) return st;
  RouterArgs ra;
  ra.x = hidden;
  ra.nw = norm_weight;
  ra.W = router_weight;
  ra.bias = router_bias;
  ra.nw_dt = norm_dtype;
  ra.bias_dt = bias_dtype;
  ra.T = tokens;
  ra.H = hidden_size;
  ra.E = num_experts;
  ra.K = top_k;
  ra.tu = 2;
  ra.eps = eps;
  ra.off = norm_offset;
  ra.logits = logits;
  ra.ids_out = topk_ids;
  ra.w_out = topk_weights;
  ra.ws = ws;
  return launch_router(ra, router_dtype, hidden_dtype, as_stream(stream));
}

int fk_moe_align(const void* topk_ids, int ids_dtype, const void* topk_weights, int weights_dtype, int tokens,
                 int top_k, int num_experts, void* workspace, size_t workspace_bytes, int32_t* counts_out,
                 int32_t* offsets_out, int32_t* perm_out, int32_t* inverse_out, void* stream) {
  if (tokens < 1 || top_k < 1 || top_k > 8) return fail(FK_ERR_INVALID, "need tokens >= 1 and 1 <= top_k <= 8");
  if (num_experts < 1 || num_experts > kMaxExperts) return fail(FK_ERR_UNSUPPORTED, "num_experts must be in [1, %d]", kMaxExperts);
  if ((long long)tokens * top_k > kMaxPairs) return fail(FK_ERR_UNSUPPORTED, "tokens * top_k must be <= %d", kMaxPairs);
  if (!is_index_dtype(ids_dtype)) return fail(FK_ERR_DTYPE, "topk_ids must be int32 or int64");
  if (topk_weights && !is_float_dtype(weights_dtype)) return fail(FK_ERR_DTYPE, "topk_weights must be f32 or bf16");
  if (!topk_ids) return fail(FK_ERR_INVALID, "topk_ids must be non-NULL");
  MoeWs ws;
  int st = check_ws(workspace, workspace_bytes, tokens, top_k, num_experts, 0, 0, &ws);
  if (st) return st;
  AlignArgs aa;
  aa.ids = topk_ids;
  aa.ids_dt = ids_dtype;
  aa.w = topk_weights;
  aa.w_dt = weights_dtype;
  aa.T = tokens;
  aa.K = top_k;
  aa.E = num_experts;
  aa.ws = ws;
  aa.counts_out = counts_out;
  aa.offsets_out = offsets_out;
  aa.perm_out = perm_out;
  aa.inverse_out = inverse_out;
  hipLaunchKernelGGL(moe_align_kernel, dim3(1), dim3(256), 0, as_stream(stream), aa);
  return check_launch("moe_align_kernel");
}

int fk_moe_experts(const void* hidden, int hidden_dtype, const void* gate_up, const void* down, int expert_dtype,
                   const void* shared_gate_up, const void* shared_down, const void* shared_gate,
                   int shared_gate_dtype, int tokens, int hidden_size, int intermediate, int num_experts,
                   int top_k, float* out, float* layer_out, void* workspace, size_t workspace_bytes,
                   void* stream) {
  int st = validate_experts(hidden, hidden_dtype, gate_up, down, expert_dtype, shared_gate_up, shared_down,
                            shared_gate, shared_gate_dtype, tokens, hidden_size, intermediate, num_experts, top_k);
  if (st) return st;
  if (!out) return fail(FK_ERR_INVALID, "out must be non-NULL");
  MoeWs ws;
  st = check_ws(workspace, workspace_bytes, tokens, top_k, num_experts, intermediate, hidden_size, &ws);
  if (st) return st;
  ExpertArgs ea = make_expert_args(hidden, hidden_dtype, gate_up, down, shared_gate_up, shared_down, shared_gate,
                                   shared_gate_dtype, tokens, hidden_size, intermediate, num_experts, top_k, out,
                                   layer_out, ws);
  return launch_experts(ea, expert_dtype, as_stream(stream));
}

int fk_moe_layer(const void* hidden, int hidden_dtype, const void* norm_weight, int norm_dtype,
                 const void* router_weight, int router_dtype, const void* router_bias, int bias_dtype,
                 const void* gate_up, const void* down, int expert_dtype, const void* shared_gate_up,
                 const void* shared_down, const void* shared_gate, int shared_gate_dtype, int tokens,
                 int hidden_size, int intermediate, int num_experts, int top_k, float eps, float norm_offset,
                 float* logits, int64_t* topk_ids, float* topk_weights, float* moe_out, float* layer_out,
                 void* workspace, size_t workspace_bytes, void* stream) {
  int st = validate_experts(hidden, hidden_dtype, gate_up, down, expert_dtype, shared_gate_up, shared_down,
                            shared_gate, shared_gate_dtype, tokens, hidden_size, intermediate, num_experts, top_k);
  if (st) return st;
  if (!moe_out) return fail(FK_ERR_INVALID, "moe_out must be non-NULL");
  MoeWs ws;
  st = check_ws(workspace, workspace_bytes, tokens, top_k, num_experts, intermediate, hidden_size, &ws);
  if (st) return st;
  if (fused_eligible(tokens, hidden_size, intermediate, num_experts, top_k, router_dtype, expert_dtype,
                     shared_gate_up != nullptr, norm_dtype, shared_gate != nullptr, shared_gate_dtype) &&
      (!shared_gate || aligned16(shared_gate))) {
    if (!is_float_dtype(norm_dtype) || (router_bias && !is_float_dtype(bias_dtype)))
      return fail(FK_ERR_DTYPE, "router inputs must be f32 or bf16");
    if (!norm_weight || !router_weight || !logits || !topk_ids || !topk_weights)
      return fail(FK_ERR_INVALID, "router pointers must be non-NULL");
    if (!aligned16(norm_weight) || !aligned16(router_weight))
      return fail(FK_ERR_ALIGNMENT, "norm_weight and router_weight must be 16-byte aligned");
    FusedArgs fa;
    fa.r.x = hidden;
    fa.r.nw = norm_weight;
    fa.r.W = router_weight;
    fa.r.bias = router_bias;
    fa.r.nw_dt = norm_dtype;
    fa.r.bias_dt = bias_dtype;
    fa.r.T = tokens;
    fa.r.H = hidden_size;
    fa.r.E = num_experts;
    fa.r.K = top_k;
    fa.r.tu = 1;
    fa.r.eps = eps;
    fa.r.off = norm_offset;
    fa.r.logits = logits;
    fa.r.ids_out = topk_ids;
    fa.r.w_out = topk_weights;
    fa.r.ws = ws;
    fa.gu = gate_up;
    fa.dn = down;
    fa.sgu = shared_gate_up;
    fa.sdn = shared_down;
    fa.sg = shared_gate;
    fa.sg_dt = shared_gate_dtype;
    fa.I = intermediate;
    fa.out = moe_out;
    fa.layer_out = layer_out;
    if (hidden_dtype == FK_DTYPE_BF16) return launch_fused_t<true>(fa, as_stream(stream));
    return launch_fused_t<false>(fa, as_stream(stream));
  }
  st = fk_moe_router(hidden, hidden_dtype, norm_weight, norm_dtype, router_weight, router_dtype, router_bias,
                     bias_dtype, tokens, hidden_size, num_experts, top_k, eps, norm_offset, logits, topk_ids,
                     topk_weights, workspace, workspace_bytes, stream);
  if (st) return st;
  ExpertArgs ea = make_expert_args(hidden, hidden_dtype, gate_up, down, shared_gate_up, shared_down, shared_gate,
                                   shared_gate_dtype, tokens, hidden_size, intermediate, num_experts, top_k,
                                   moe_out, layer_out, ws);
  return launch_experts(ea, expert_dtype, as_stream(stream));
}

int fk_moe_layer_noalloc(const void* hidden, int hidden_dtype, const void* norm_weight, int norm_dtype,
                         const void* router_weight, int router_dtype, const void* router_bias, int bias_dtype,
                         const void* gate_up, const void* down, int expert_dtype, const void* shared_gate_up,
                         const void* shared_down, const void* shared_gate, int shared_gate_dtype, int tokens,
                         int hidden_size, int intermediate, int num_experts, int top_k, float eps,
                         float norm_offset, float* logits, int64_t* topk_ids, float* topk_weights, float* moe_out,
                         float* layer_out, void* stream) {
  int st = validate_experts(hidden, hidden_dtype, gate_up, down, expert_dtype, shared_gate_up, shared_down,
                            shared_gate, shared_gate_dtype, tokens, hidden_size, intermediate, num_experts, top_k);
  if (st) return st;
  MoeWs ws;
  const size_t need = moe_ws_layout(tokens, top_k, num_experts, intermediate, hidden_size, nullptr, &ws);
  if (need > kNoAllocScratchBytes)
    return fail(FK_ERR_UNSUPPORTED,
                "fk_moe_layer_noalloc: this problem needs %zu bytes of scratch, more than the %zu bytes each GPU "
                "holds (use fk_moe_layer with a workspace of fk_moe_workspace_bytes)",
                need, kNoAllocScratchBytes);
  void* ptr = nullptr;
  st = noalloc_scratch(as_stream(stream), &ptr);
  if (st) return st;
  return fk_moe_layer(hidden, hidden_dtype, norm_weight, norm_dtype, router_weight, router_dtype, router_bias,
                      bias_dtype, gate_up, down, expert_dtype, shared_gate_up, shared_down, shared_gate,
                      shared_gate_dtype, tokens, hidden_size, intermediate, num_experts, top_k, eps, norm_offset,
                      logits, topk_ids, topk_weights, moe_out, layer_out, ptr, kNoAllocScratchBytes, stream);
}

int fk_moe_noalloc_workspace(void** workspace, size_t* workspace_bytes, void* stream) {
  if (!workspace || !workspace_bytes) return fail(FK_ERR_INVALID, "workspace and workspace_bytes must be non-NULL");
  void* p = nullptr;
  const int st = noalloc_scratch(as_stream(stream), &p);
  if (st) return st;
  *workspace = p;
  *workspace_bytes = kNoAllocScratchBytes;
  return FK_OK;
}

}  // extern "C"
