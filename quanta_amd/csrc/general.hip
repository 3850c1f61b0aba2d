// The block for inputs outside the fast path's formats: float32 activations, float32 scale/bias
// triplets, group sizes 32/64/128 at any hidden size, code widths 2-8, dense float32 or bf16
// expert stacks. It follows the reference's dtype flow exactly:
//   logits = f32(x) @ f32(gate)^T                                  (src/quanta/qwen35/moe.py:47)
//   gu = qmm(x_T, experts_gate_up) in T, the experts' dtype: the scale/bias dtype of a packed
//        triplet ("the qmm output follows the baked scale dtype", :98-104) or the dtype of a
//        dense stack (x cast to it, :77)
//   h = silu(g) * u in T; d = qmm(h, experts_down) in T               (:59-63, :121-123)
//   routed = sum_s f32(d) * w                                          (:191)
//   shared = f32(down(silu(xd Wg^T) * (xd Wu^T))) * sigmoid(f32(x) . f32(g)), xd = x cast to the
//            shared weights' dtype                                     (:145-151)
//   y = cast_x(routed + shared)                                        (:201-202)
// as the reference's own float32 parity gates run it (parity/qwen35_forward_test.py:213-271:
// hidden 32, group size 32, float32 throughout). Every matrix-vector product is one wavefront per
// output (lanes stride K, a fixed-order wavefront sum, fp32 accumulation); the affine weight
// s*q + b is evaluated in fp32 per element from the LSB-first packed code stream. These shapes are
// small (the parity configs); the fast path serves the bf16 g64 production formats.
#include <math.h>

#include "qmoe_internal.h"
#include "route_common.h"
#include "../../include/quanta_moe.h"

namespace qmoe {

__device__ __forceinline__ float gen_ld(const void* p, int64_t i, int dt) {
  return dt == QMOE_DT_F32 ? static_cast<const float*>(p)[i]
                           : bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
}
__device__ __forceinline__ float gen_round(float v, int dt) {
  return dt == QMOE_DT_F32 ? v : bf16_to_f32(f32_to_bf16(v));
}
__device__ __forceinline__ void gen_st(void* p, int64_t i, float v, int dt) {
  if (dt == QMOE_DT_F32) static_cast<float*>(p)[i] = v;
  else static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
}

// out[r][col0 + o] = sum_k a(r, k) * W_e(r)[o][k]: a = the activation row r / row_div, rounded to
// act_round when that differs from its dtype (the reference's cast to the weights' dtype); W a
// dense [E][n_out][K] stack or affine codes (bits, group gs, scale/bias [E][n_out][K/gs]).
struct GenMv {
  const void* act;
  int act_dt, act_round;     // QMOE_DT_*; act_round: the dtype the activation is cast to first
  int64_t act_rows;
  int K;
  const int32_t* row_expert;  // [rows] expert of each output row (nullable: expert 0)
  int row_div;
  int64_t rows;
  int n_out;
  const uint32_t* packed;     // affine codes (nullable: dense)
  const void* scale;
  const void* bias;
  int bits, gs, sb_dt;
  const void* dense;
  int dense_dt;
  void* out;
  int out_dt;
  int64_t ld_out;
  int col0;
};

__global__ void __launch_bounds__(256) gen_matvec_kernel(GenMv a) {
  const int lane = threadIdx.x & 63;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (gid >= a.rows * a.n_out) return;   // whole wavefronts exit together; no barriers below
  const int64_t r = gid / a.n_out;
  const int o = static_cast<int>(gid - r * a.n_out);
  const int e = a.row_expert ? a.row_expert[r] : 0;
  const int64_t ar = r / a.row_div;
  float acc = 0.f;
  if (ar < a.act_rows && e >= 0) {
    const int64_t wrow = static_cast<int64_t>(e) * a.n_out + o;
    const int64_t abase = ar * a.K;
    const int64_t words = static_cast<int64_t>(a.K) * a.bits / 32;
    const uint32_t mask = (1u << a.bits) - 1u;
    for (int k = lane; k < a.K; k += 64) {
      float xv = gen_ld(a.act, abase + k, a.act_dt);
      if (a.act_round != a.act_dt) xv = gen_round(xv, a.act_round);
      float wv;
      if (a.packed) {
        const int64_t bit = static_cast<int64_t>(k) * a.bits;
        const uint32_t* p = a.packed + wrow * words + bit / 32;
        const int sh = static_cast<int>(bit & 31);
        uint32_t c = p[0] >> sh;
        if (sh + a.bits > 32) c |= p[1] << (32 - sh);
        const int64_t g = wrow * (a.K / a.gs) + k / a.gs;
        wv = fmaf(gen_ld(a.scale, g, a.sb_dt), static_cast<float>(c & mask), gen_ld(a.bias, g, a.sb_dt));
      } else {
        wv = gen_ld(a.dense, wrow * a.K + k, a.dense_dt);
      }
      acc = fmaf(xv, wv, acc);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
  if (lane == 0) gen_st(a.out, r * a.ld_out + a.col0 + o, acc, a.out_dt);
}

static int gen_matvec(const GenMv& a, hipStream_t stream) {
  const int64_t waves = a.rows * a.n_out;
  if (waves <= 0) return 0;
  if ((waves + 3) / 4 > 0x7fffffff) return fail("general: product too large");
  gen_matvec_kernel<<<dim3(static_cast<unsigned>((waves + 3) / 4)), 256, 0, stream>>>(a);
  return check_launch("general matvec");
}

// h[r][i] = glu(gu[r][i], gu[r][n + i]) in dtype dt (fp32 math, one rounding)
__global__ void __launch_bounds__(256) gen_glu_kernel(const void* gu, void* h, int64_t rows, int n,
                                                      int dt, int act, float alpha, float limit) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= rows * n) return;
  const int64_t r = i / n, c = i - r * n;
  const float g = gen_ld(gu, r * 2 * n + c, dt), u = gen_ld(gu, r * 2 * n + n + c, dt);
  gen_st(h, i, glu_f(g, u, act, alpha, limit), dt);
}

// y[t][j] = cast_x(sum_s f32(d[t*k+s][j]) * w[t][s] + f32(sh[t][j]) * sg[t])
__global__ void __launch_bounds__(256) gen_combine_kernel(const void* d, int d_dt, const float* w,
                                                          int N, int k, int H, const void* sh,
                                                          int sh_dt, const float* sg, void* y,
                                                          int y_dt) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<int64_t>(N) * H) return;
  const int64_t t = i / H, j = i - t * H;
  float acc = 0.f;
  for (int s = 0; s < k; ++s)
    acc += gen_ld(d, (t * k + s) * H + j, d_dt) * w[t * k + s];
  if (sh) acc += gen_ld(sh, t * H + j, sh_dt) * (sg ? sg[t] : 1.0f);
  gen_st(y, i, acc, y_dt);
}

// The run-every-expert form (the reference's sparse=False oracle, moe.py:127-142): every token
// runs every expert e (idx_all[t][e] = e) and the combine weights are the routing weights
// scattered onto the chosen experts, zero elsewhere.
__global__ void __launch_bounds__(256) gen_scatter_kernel(const int32_t* idx, const float* w, int N,
                                                          int k, int E, int32_t* idx_all,
                                                          float* w_all) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= N) return;
  for (int e = 0; e < E; ++e) {
    idx_all[static_cast<int64_t>(t) * E + e] = e;
    w_all[static_cast<int64_t>(t) * E + e] = 0.f;
  }
  for (int s = 0; s < k; ++s) {
    const int e = idx[static_cast<int64_t>(t) * k + s];
    if (e >= 0 && e < E) w_all[static_cast<int64_t>(t) * E + e] = w[static_cast<int64_t>(t) * k + s];
  }
}

struct GenLayout {
  size_t logits, idx, w, sg, idx_all, w_all, gu, h, d, sgu, sh, so, total;
};
static int dt_bytes(int dt) { return dt == QMOE_DT_F32 ? 4 : 2; }
// The routed experts' compute dtype: a dense stack's own dtype (x is cast to it, moe.py:77); for
// packed codes the promotion of x's and the scales' dtypes (mx.gather_qmm's result type).
static int routed_dtype(const qmoe_general_config_t& c) {
  if (!c.experts_packed) return c.expert_dtype;
  return (c.x_dtype == QMOE_DT_F32 || c.expert_dtype == QMOE_DT_F32) ? QMOE_DT_F32 : QMOE_DT_BF16;
}
// Slots per token of the routed stage: top_k, or every expert for the run-every-expert form.
static int routed_slots(const qmoe_general_config_t& c) { return c.dense_all ? c.n_experts : c.top_k; }
static GenLayout gen_layout(const qmoe_general_config_t& c, int64_t N) {
  GenLayout L{};
  size_t o = 0;
  auto take = [&](size_t b) {
    const size_t at = o;
    o = align256(o + b);
    return at;
  };
  const int64_t mc = N * routed_slots(c);
  const int te = dt_bytes(routed_dtype(c)), ts = dt_bytes(c.shared_dtype);
  L.logits = take(static_cast<size_t>(N) * (c.n_experts + 1) * 4);
  L.idx = take(static_cast<size_t>(N) * c.top_k * 4);
  L.w = take(static_cast<size_t>(N) * c.top_k * 4);
  L.sg = take(static_cast<size_t>(N) * 4);
  L.idx_all = take(c.dense_all ? static_cast<size_t>(mc) * 4 : 0);
  L.w_all = take(c.dense_all ? static_cast<size_t>(mc) * 4 : 0);
  L.gu = take(static_cast<size_t>(mc) * 2 * c.inter * te);
  L.h = take(static_cast<size_t>(mc) * c.inter * te);
  L.d = take(static_cast<size_t>(mc) * c.hidden * te);
  L.sgu = take(static_cast<size_t>(N) * 2 * c.shared_inter * ts);
  L.sh = take(static_cast<size_t>(N) * c.shared_inter * ts);
  L.so = take(static_cast<size_t>(N) * c.hidden * ts);
  L.total = o;
  return L;
}

int validate_routing(int N, int H, int E, int k, int scoring, int n_group, int topk_group);

static bool dt_ok(int dt) { return dt == QMOE_DT_BF16 || dt == QMOE_DT_F32; }

static int gen_validate(const qmoe_general_config_t& c) {
  int rc = validate_routing(1, c.hidden, c.n_experts, c.top_k, c.scoring, c.n_group, c.topk_group);
  if (rc) return rc;
  if (c.top_k > 64) return fail("general: top_k <= 64 required");
  if (!dt_ok(c.x_dtype) || !dt_ok(c.gate_dtype) || !dt_ok(c.expert_dtype) || !dt_ok(c.shared_dtype) ||
      !dt_ok(c.shared_gate_dtype))
    return fail("general: dtypes must be QMOE_DT_BF16 or QMOE_DT_F32");
  if (c.inter <= 0 || c.shared_inter < 0) return fail("general: inter > 0, shared_inter >= 0 required");
  if (c.norm_topk < QMOE_NORM_NONE || c.norm_topk > QMOE_NORM_MULTI) return fail("general: bad norm_topk");
  if (c.act < QMOE_ACT_SILU || c.act > QMOE_ACT_SWIGLU_OAI) return fail("general: unknown act");
  if (c.act != QMOE_ACT_SILU && !(c.act_limit > 0.f)) return fail("general: act_limit must be > 0");
  if (c.experts_packed) {
    if (c.bits < 2 || c.bits > 8 || c.bits == 7) return fail("general: bits must be 2, 3, 4, 5, 6 or 8");
    if (c.group_size != 32 && c.group_size != 64 && c.group_size != 128)
      return fail("general: group_size must be 32, 64 or 128");
    if (c.hidden % c.group_size || c.inter % c.group_size)
      return fail("general: hidden and inter must be multiples of group_size");
    if ((static_cast<int64_t>(c.hidden) * c.bits) % 32 || (static_cast<int64_t>(c.inter) * c.bits) % 32)
      return fail("general: packed rows must fill whole 32-bit words");
  } else if (c.experts_packed != 0) {
    return fail("general: experts_packed must be 0 or 1");
  }
  if (c.dense_all != 0 && c.dense_all != 1) return fail("general: dense_all must be 0 or 1");
  if (c.shared_gated != 0 && c.shared_gated != 1) return fail("general: shared_gated must be 0 or 1");
  return 0;
}

}  // namespace qmoe

using namespace qmoe;

extern "C" size_t qmoe_forward_general_workspace(const qmoe_general_config_t* cfg, int64_t N) {
  if (!cfg || N <= 0) return 0;
  return gen_layout(*cfg, N).total;
}

extern "C" int qmoe_forward_general(const qmoe_general_config_t* cfg, const qmoe_general_weights_t* wts,
                                    const void* x, int64_t N, void* y, void* ws, size_t ws_bytes,
                                    void* stream_) {
  if (!cfg || !wts || !x || !y || !ws) return fail("qmoe_forward_general: null pointer");
  const qmoe_general_config_t& c = *cfg;
  int rc = gen_validate(c);
  if (rc) return rc;
  if (N <= 0 || N > 65535) return fail("qmoe_forward_general: 0 < N <= 65535 tokens per call");
  const GenLayout L = gen_layout(c, N);
  if (ws_bytes < L.total) return fail("qmoe_forward_general: workspace too small");
  if (!wts->gate || !wts->gu || !wts->dn) return fail("qmoe_forward_general: missing weights");
  if (c.experts_packed && (!wts->gu_scale || !wts->gu_bias || !wts->dn_scale || !wts->dn_bias))
    return fail("qmoe_forward_general: packed experts need scale and bias");
  const bool shared = c.shared_inter > 0;
  if (shared && (!wts->sh_gate || !wts->sh_up || !wts->sh_down))
    return fail("qmoe_forward_general: missing shared expert");
  if (shared && c.shared_gated && !wts->sh_expert_gate)
    return fail("qmoe_forward_general: a gated shared expert needs sh_expert_gate");
  hipStream_t st = static_cast<hipStream_t>(stream_);
  char* base = static_cast<char*>(ws);
  float* logits = reinterpret_cast<float*>(base + L.logits);
  int32_t* idx = reinterpret_cast<int32_t*>(base + L.idx);
  float* wv = reinterpret_cast<float*>(base + L.w);
  float* sg = reinterpret_cast<float*>(base + L.sg);
  const int n = static_cast<int>(N), H = c.hidden, E = c.n_experts, I = c.inter, Is = c.shared_inter;
  if (c.dense_all && c.experts_packed)
    return fail("qmoe_forward_general: the run-every-expert form takes dense stacks only");
  const int has_sg = (shared && c.shared_gated) ? 1 : 0;
  const int ld = E + 1;

  // router logits in f32 (column E: the shared expert's gate logit)
  GenMv r{};
  r.act = x; r.act_dt = c.x_dtype; r.act_round = c.x_dtype; r.act_rows = N; r.K = H;
  r.row_div = 1; r.rows = N; r.n_out = E; r.dense = wts->gate; r.dense_dt = c.gate_dtype;
  r.out = logits; r.out_dt = QMOE_DT_F32; r.ld_out = ld;
  if ((rc = gen_matvec(r, st))) return rc;
  if (has_sg) {
    GenMv g = r;
    g.n_out = 1; g.dense = wts->sh_expert_gate; g.dense_dt = c.shared_gate_dtype; g.col0 = E;
    if ((rc = gen_matvec(g, st))) return rc;
  }
  rc = launch_topk(logits, ld, wts->router_bias, n, E, c.top_k, c.scoring, c.n_group, c.topk_group,
                   c.norm_topk, c.routed_scale, has_sg, idx, wv, sg, st);
  if (rc) return rc;

  // routed experts in their dtype T
  const int T = routed_dtype(c);
  const int ks = routed_slots(c);
  const int64_t mc = N * ks;
  const int32_t* ridx = idx;
  const float* rw = wv;
  if (c.dense_all) {
    int32_t* ia = reinterpret_cast<int32_t*>(base + L.idx_all);
    float* wa = reinterpret_cast<float*>(base + L.w_all);
    gen_scatter_kernel<<<dim3((n + 255) / 256), 256, 0, st>>>(idx, wv, n, c.top_k, E, ia, wa);
    if ((rc = check_launch("general scatter"))) return rc;
    ridx = ia;
    rw = wa;
  }
  void* gu = base + L.gu;
  void* h = base + L.h;
  void* d = base + L.d;
  GenMv e{};
  e.act = x; e.act_dt = c.x_dtype; e.act_round = T; e.act_rows = N; e.K = H;
  e.row_expert = ridx; e.row_div = ks; e.rows = mc; e.n_out = 2 * I;
  e.bits = c.bits; e.gs = c.group_size; e.sb_dt = c.expert_dtype; e.dense_dt = c.expert_dtype;
  if (c.experts_packed) {
    e.packed = static_cast<const uint32_t*>(wts->gu); e.scale = wts->gu_scale; e.bias = wts->gu_bias;
  } else {
    e.dense = wts->gu;
  }
  e.out = gu; e.out_dt = T; e.ld_out = 2 * I;
  if ((rc = gen_matvec(e, st))) return rc;
  const int64_t hn = mc * I;
  gen_glu_kernel<<<dim3(static_cast<unsigned>((hn + 255) / 256)), 256, 0, st>>>(
      gu, h, mc, I, T, c.act, c.act_alpha, c.act_limit);
  if ((rc = check_launch("general glu"))) return rc;
  GenMv dn = e;
  dn.act = h; dn.act_dt = T; dn.act_round = T; dn.act_rows = mc; dn.K = I; dn.row_div = 1;
  dn.n_out = H; dn.out = d; dn.ld_out = H;
  if (c.experts_packed) {
    dn.packed = static_cast<const uint32_t*>(wts->dn); dn.scale = wts->dn_scale; dn.bias = wts->dn_bias;
  } else {
    dn.dense = wts->dn;
  }
  if ((rc = gen_matvec(dn, st))) return rc;

  // shared expert in its weights' dtype S
  void* so = nullptr;
  if (shared) {
    const int S = c.shared_dtype;
    void* sgu = base + L.sgu;
    void* sh = base + L.sh;
    so = base + L.so;
    GenMv s{};
    s.act = x; s.act_dt = c.x_dtype; s.act_round = S; s.act_rows = N; s.K = H; s.row_div = 1;
    s.rows = N; s.n_out = Is; s.dense = wts->sh_gate; s.dense_dt = S; s.out = sgu; s.out_dt = S;
    s.ld_out = 2 * Is;
    if ((rc = gen_matvec(s, st))) return rc;
    s.dense = wts->sh_up; s.col0 = Is;
    if ((rc = gen_matvec(s, st))) return rc;
    const int64_t sn = N * Is;
    gen_glu_kernel<<<dim3(static_cast<unsigned>((sn + 255) / 256)), 256, 0, st>>>(
        sgu, sh, N, Is, S, c.act, c.act_alpha, c.act_limit);
    if ((rc = check_launch("general shared glu"))) return rc;
    GenMv sd{};
    sd.act = sh; sd.act_dt = S; sd.act_round = S; sd.act_rows = N; sd.K = Is; sd.row_div = 1;
    sd.rows = N; sd.n_out = H; sd.dense = wts->sh_down; sd.dense_dt = S; sd.out = so; sd.out_dt = S;
    sd.ld_out = H;
    if ((rc = gen_matvec(sd, st))) return rc;
  }
  const int64_t yn = N * H;
  gen_combine_kernel<<<dim3(static_cast<unsigned>((yn + 255) / 256)), 256, 0, st>>>(
      d, T, rw, n, ks, H, so, c.shared_dtype, has_sg ? sg : nullptr, y, c.x_dtype);
  return check_launch("general combine");
}
