/*
 * CPU oracle for the gated-delta verify hot path.  TEST INFRASTRUCTURE ONLY:
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it as
 * a checker or a timed CPU baseline; the product library never links it.
 *
 * A plain-C restatement of the reference's recurrence, in the op order of the
 * reference's own CPU loop and Metal kernel:
 *   dflash_mlx/custom_qwen35_model.py:129-139 (advance_gated_delta_states,
 *   pure-op path) and :54-74 (gated_delta_state_update):
 *     S  = S * g_t                       (:59 / :135)
 *     kv = sum_dk S[dv,dk] * k_t[dk]     (:60-62 / :136)
 *     d  = (v_t[dv] - kv) * beta_t       (:64 / :137)
 *     S += k_t[dk] * d                   (:67 / :138)
 * plus the output the reference takes from mlx_lm's gated_delta_kernel
 * (called at custom_qwen35_model.py:457-466; mlx-lm 0.31.2 is not vendored):
 *     out_t[dv] = sum_dk S[dv,dk] * q_t[dk]   after the update
 * (the gated delta rule of Yang, Kautz & Hatamizadeh, "Gated Delta Networks",
 * ICLR 2025: o_t = S_t q_t), and the per-token state tape tape[t] = S.
 * GQA: value head hv uses key head hv / (Hv/Hk), as the reference's
 * mx.repeat(keys, repeat_factor, axis=2) implies (:1054-1057).
 *
 * Inputs are fp32 (bf16 inputs are widened exactly by the caller).  acc64 = 1
 * accumulates everything in double (the brute-force reference); acc64 = 0
 * keeps fp32 state and sums like the reference kernel.
 *
 * Build: oracle/Makefile (gcc -O2 -fopenmp -shared).
 */
#include <stdint.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

int oracle_abi_version(void) { return 1; }

int oracle_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void oracle_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* One (b, hv) head, fp32 state. */
static void scan_head_f32(const float* q, const float* k, const float* v,
                          const float* g, const float* beta, float* S, float* out,
                          float* tape, int n, int T, int B, int b, int hv, int hk,
                          int Hk, int Hv, int Dk, int Dv, int64_t tape_tstride) {
  for (int t = 0; t < n; ++t) {
    const float* kt = k + (((int64_t)b * T + t) * Hk + hk) * Dk;
    const float* vt = v + (((int64_t)b * T + t) * Hv + hv) * Dv;
    const float gt = g[((int64_t)b * T + t) * Hv + hv];
    const float bt = beta[((int64_t)b * T + t) * Hv + hv];
    for (int dv = 0; dv < Dv; ++dv) {
      float* row = S + (int64_t)dv * Dk;
      float kv = 0.0f;
      for (int dk = 0; dk < Dk; ++dk) {
        row[dk] = row[dk] * gt;
        kv += row[dk] * kt[dk];
      }
      const float d = (vt[dv] - kv) * bt;
      for (int dk = 0; dk < Dk; ++dk) row[dk] = row[dk] + kt[dk] * d;
      if (q != NULL && out != NULL) {
        const float* qt = q + (((int64_t)b * T + t) * Hk + hk) * Dk;
        float o = 0.0f;
        for (int dk = 0; dk < Dk; ++dk) o += row[dk] * qt[dk];
        out[(((int64_t)b * T + t) * Hv + hv) * Dv + dv] = o;
      }
    }
    if (tape != NULL)
      memcpy(tape + (int64_t)t * tape_tstride + ((int64_t)b * Hv + hv) * Dv * Dk, S,
             sizeof(float) * (size_t)Dv * Dk);
  }
  (void)B;
}

/* One (b, hv) head, double accumulation; S is a double scratch of Dv*Dk. */
static void scan_head_f64(const float* q, const float* k, const float* v,
                          const float* g, const float* beta, double* S, double* out,
                          double* tape, int n, int T, int b, int hv, int hk, int Hk,
                          int Hv, int Dk, int Dv, int64_t tape_tstride) {
  for (int t = 0; t < n; ++t) {
    const float* kt = k + (((int64_t)b * T + t) * Hk + hk) * Dk;
    const float* vt = v + (((int64_t)b * T + t) * Hv + hv) * Dv;
    const double gt = g[((int64_t)b * T + t) * Hv + hv];
    const double bt = beta[((int64_t)b * T + t) * Hv + hv];
    for (int dv = 0; dv < Dv; ++dv) {
      double* row = S + (int64_t)dv * Dk;
      double kv = 0.0;
      for (int dk = 0; dk < Dk; ++dk) {
        row[dk] *= gt;
        kv += row[dk] * (double)kt[dk];
      }
      const double d = ((double)vt[dv] - kv) * bt;
      for (int dk = 0; dk < Dk; ++dk) row[dk] += (double)kt[dk] * d;
      if (q != NULL && out != NULL) {
        const float* qt = q + (((int64_t)b * T + t) * Hk + hk) * Dk;
        double o = 0.0;
        for (int dk = 0; dk < Dk; ++dk) o += row[dk] * (double)qt[dk];
        out[(((int64_t)b * T + t) * Hv + hv) * Dv + dv] = o;
      }
    }
    if (tape != NULL)
      memcpy(tape + (int64_t)t * tape_tstride + ((int64_t)b * Hv + hv) * Dv * Dk, S,
             sizeof(double) * (size_t)Dv * Dk);
  }
}

/*
 * Scan with out and tape, contiguous tensors:
 *   q, k [B,T,Hk,Dk]; v [B,T,Hv,Dv]; g, beta [B,T,Hv]; state_in [B,Hv,Dv,Dk]
 *   out [B,T,Hv,Dv] (or NULL); final_state [B,Hv,Dv,Dk]; tape [T,B,Hv,Dv,Dk]
 *   (or NULL); lengths [B] (or NULL: all T).
 * fp32 mode: outputs are float*.  Returns 0, or -2 on a bad shape.
 */
int oracle_gdn_scan_f32(const float* q, const float* k, const float* v, const float* g,
                        const float* beta, const float* state_in, float* out,
                        float* final_state, float* tape, const int32_t* lengths, int B,
                        int T, int Hk, int Hv, int Dk, int Dv) {
  if (B < 0 || T < 0 || Hk <= 0 || Hv <= 0 || Hv % Hk != 0 || Dk <= 0 || Dv <= 0) return -2;
  const int rep = Hv / Hk;
  const int64_t hs = (int64_t)Dv * Dk;
  const int64_t tape_tstride = (int64_t)B * Hv * hs;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t bh = 0; bh < (int64_t)B * Hv; ++bh) {
    const int b = (int)(bh / Hv), hv = (int)(bh % Hv);
    float* S = final_state + bh * hs;
    if (S != state_in + bh * hs) memcpy(S, state_in + bh * hs, sizeof(float) * (size_t)hs);
    int n = T;
    if (lengths != NULL) n = lengths[b] < 0 ? 0 : (lengths[b] > T ? T : lengths[b]);
    scan_head_f32(q, k, v, g, beta, S, out, tape, n, T, B, b, hv, hv / rep, Hk, Hv, Dk, Dv,
                  tape_tstride);
  }
  return 0;
}

/* Same contract, double accumulation and double outputs. */
int oracle_gdn_scan_f64(const float* q, const float* k, const float* v, const float* g,
                        const float* beta, const float* state_in, double* out,
                        double* final_state, double* tape, const int32_t* lengths, int B,
                        int T, int Hk, int Hv, int Dk, int Dv) {
  if (B < 0 || T < 0 || Hk <= 0 || Hv <= 0 || Hv % Hk != 0 || Dk <= 0 || Dv <= 0) return -2;
  const int rep = Hv / Hk;
  const int64_t hs = (int64_t)Dv * Dk;
  const int64_t tape_tstride = (int64_t)B * Hv * hs;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t bh = 0; bh < (int64_t)B * Hv; ++bh) {
    const int b = (int)(bh / Hv), hv = (int)(bh % Hv);
    double* S = final_state + bh * hs;
    for (int64_t i = 0; i < hs; ++i) S[i] = (double)state_in[bh * hs + i];
    int n = T;
    if (lengths != NULL) n = lengths[b] < 0 ? 0 : (lengths[b] > T ? T : lengths[b]);
    scan_head_f64(q, k, v, g, beta, S, out, tape, n, T, b, hv, hv / rep, Hk, Hv, Dk, Dv,
                  tape_tstride);
  }
  return 0;
}

/*
 * Greedy accept on fp32 logits [B, N, V]: posterior = first index of the
 * maximum (NaN above every number, the first NaN wins, -0 == +0), then the
 * longest agreeing draft prefix (dflash_mlx/runtime.py:41-47) and the bonus
 * posterior[matched] (runtime.py:145-147, :163), -1 when matched == N.
 */
static int key_gt(float a, float b) {
  /* 1 if a ranks strictly above b in argmax order. */
  const int an = a != a, bn = b != b;
  if (an || bn) return an && !bn;
  return a > b;
}

int oracle_greedy_accept_f32(const float* logits, const int32_t* draft, int n_draft,
                             int32_t* posterior, int32_t* matched, int32_t* bonus, int B,
                             int N, int V) {
  if (B < 0 || N <= 0 || V <= 0 || n_draft < 0) return -2;
  for (int b = 0; b < B; ++b) {
    for (int i = 0; i < N; ++i) {
      const float* row = logits + ((int64_t)b * N + i) * V;
      int best = 0;
      for (int j = 1; j < V; ++j)
        if (key_gt(row[j], row[best])) best = j;
      posterior[(int64_t)b * N + i] = best;
    }
    const int m = n_draft < N ? n_draft : N;
    int mt = 0;
    while (mt < m && draft[(int64_t)b * n_draft + mt] == posterior[(int64_t)b * N + mt]) ++mt;
    matched[b] = mt;
    bonus[b] = mt < N ? posterior[(int64_t)b * N + mt] : -1;
  }
  return 0;
}
