// ttc_lqr_host.cpp -- host (CPU) solver of the same batched LQR problems, for CPU tensors.
//
// The reference's pure-PyTorch solvers `riccati` (direct_lqr_solve, ttc/solvers/torch_lqr.py:93-118)
// and `kkt` (kkt_lqr_solve, torch_lqr.py:120-140) run on any device; TTCLayer on the CPU
// (solver_impl="riccati" / "kkt") uses them.  This file is that CPU path of libttc_lqr.so:
// no GPU involved, fp64 arithmetic on fp32 arrays in host memory, one problem at a time per
// thread (whole tokens per thread, so the head sums of grad_B / grad_Q are formed in a fixed
// order by one thread: deterministic, no atomics).
//
// Forward: the backward-in-time Riccati sweep (lin_solver_lqr.py:155-185) with the gain solve
// done by LU with partial pivoting, V symmetrised every step, u_0 = K_0 h_0.
// Backward: implicit differentiation of the KKT system (torch_lqr.py:34-63): the sweep again
// with every gain kept, closed-loop rollouts of the primal (from h_0) and of the adjoint problem
// (from 0, feed-forward w_0 = -Quu_0^{-1} d_u at t = 0), costates swept back with the
// closed-loop recursion lambda_k = Qc_k h_k + A_k lambda_{k+1} + K_k'(R u_k + B_k' lambda_{k+1})
// (the open-loop recursion of lin_solver_lqr.py:82-98 plus a term that vanishes at the optimum;
// it does not amplify rounding by prod A_k), gradients as outer products chained through the
// discount expansion of torch_lqr.py:65-91.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <thread>
#include <vector>

#include "ttc_lqr.h"

namespace {

struct Problem {  // views of one (token, head) problem; B and Q are the token's
  const float *a, *B, *Q, *r, *Qf, *lgA, *lgB, *lgQ, *h0;
};

struct Sizes {
  int d, du, T;
};

// Per-thread scratch.
struct Scratch {
  std::vector<double> V, W, Quu, X, Qs, Bd, Qfs;
  std::vector<double> K;        // gains K_t [T][du][d] (backward)
  std::vector<double> LU0;      // LU of Quu_0 [du][du]
  std::vector<int> piv, piv0;
  std::vector<double> h, hb, u, w, lam, lamb, tmp, tmp2, qv;
  void init(const Sizes& s, bool backward) {
    const size_t d = s.d, du = s.du, T = s.T;
    V.assign(d * d, 0.0); W.assign(d * du, 0.0); Quu.assign(du * du, 0.0); X.assign(du * d, 0.0);
    Qs.assign(d * d, 0.0); Bd.assign(d * du, 0.0); Qfs.assign(d * d, 0.0);
    piv.assign(du, 0); piv0.assign(du, 0); LU0.assign(du * du, 0.0);
    tmp.assign(std::max(d, du), 0.0); tmp2.assign(std::max(d, du), 0.0); qv.assign(d, 0.0);
    if (backward) {
      K.assign(T * du * d, 0.0);
      h.assign((T + 1) * d, 0.0); hb.assign((T + 1) * d, 0.0);
      u.assign(T * du, 0.0); w.assign(T * du, 0.0);
      lam.assign(d, 0.0); lamb.assign(d, 0.0);
    }
  }
};

// In-place LU with partial pivoting of the n x n row-major matrix M.  Returns false when a
// pivot is zero or not finite.
bool lu_factor(double* M, int n, int* piv) {
  for (int k = 0; k < n; ++k) {
    int p = k;
    double best = fabs(M[k * n + k]);
    for (int i = k + 1; i < n; ++i) {
      const double v = fabs(M[i * n + k]);
      if (v > best) { best = v; p = i; }
    }
    piv[k] = p;
    if (!(best > 0.0) || !std::isfinite(best)) return false;
    if (p != k)
      for (int j = 0; j < n; ++j) std::swap(M[k * n + j], M[p * n + j]);
    const double inv = 1.0 / M[k * n + k];
    for (int i = k + 1; i < n; ++i) {
      const double f = M[i * n + k] * inv;
      M[i * n + k] = f;
      if (f != 0.0)
        for (int j = k + 1; j < n; ++j) M[i * n + j] -= f * M[k * n + j];
    }
  }
  return true;
}

// Solve (LU) X = Y in place for `m` right-hand-side columns of the n x m row-major Y.
void lu_solve(const double* LU, int n, const int* piv, double* Y, int m) {
  for (int k = 0; k < n; ++k)
    if (piv[k] != k)
      for (int j = 0; j < m; ++j) std::swap(Y[k * m + j], Y[piv[k] * m + j]);
  for (int i = 1; i < n; ++i)
    for (int k = 0; k < i; ++k) {
      const double f = LU[i * n + k];
      if (f != 0.0)
        for (int j = 0; j < m; ++j) Y[i * m + j] -= f * Y[k * m + j];
    }
  for (int i = n - 1; i >= 0; --i) {
    for (int k = i + 1; k < n; ++k) {
      const double f = LU[i * n + k];
      if (f != 0.0)
        for (int j = 0; j < m; ++j) Y[i * m + j] -= f * Y[k * m + j];
    }
    const double inv = 1.0 / LU[i * n + i];
    for (int j = 0; j < m; ++j) Y[i * m + j] *= inv;
  }
}

// One Riccati step k of problem `pb`: V (= V_{k+1} on entry) -> V_k; the gain K_k = -X
// leaves in S.X ([du][d]).  At k == 0 the LU of Quu_0 is kept in S.LU0 / S.piv0 and V is
// not updated.  Returns false when Quu is singular or not finite.
bool riccati_step(const Problem& pb, const Sizes& s, int k, Scratch& S) {
  const int d = s.d, du = s.du;
  const double eA = exp((double)pb.lgA[0] * (k + 1));
  double* al = S.tmp.data();   // alpha (d)
  double* be = S.tmp2.data();  // beta (du)
  for (int i = 0; i < d; ++i) al[i] = 1.0 + (double)pb.a[i] * eA;
  for (int j = 0; j < du; ++j) be[j] = exp((double)pb.lgB[j] * (k + 1));
  // W = V B_k
  for (int i = 0; i < d; ++i) {
    double* wr = &S.W[(size_t)i * du];
    for (int j = 0; j < du; ++j) wr[j] = 0.0;
    for (int m = 0; m < d; ++m) {
      const double v = S.V[(size_t)i * d + m];
      const double* br = &S.Bd[(size_t)m * du];
      for (int j = 0; j < du; ++j) wr[j] += v * br[j];
    }
    for (int j = 0; j < du; ++j) wr[j] *= be[j];
  }
  // Quu = R + B_k' W ;  X = Qux = W' A_k  (du x d, solved in place below)
  for (int j = 0; j < du; ++j) {
    for (int l = 0; l < du; ++l) {
      double acc = 0.0;
      for (int m = 0; m < d; ++m) acc += S.Bd[(size_t)m * du + j] * S.W[(size_t)m * du + l];
      S.Quu[(size_t)j * du + l] = acc * be[j];
    }
    S.Quu[(size_t)j * du + j] += 1.0 / (double)pb.r[j];
    for (int i = 0; i < d; ++i) S.X[(size_t)j * d + i] = S.W[(size_t)i * du + j] * al[i];
  }
  for (int j = 0; j < du; ++j)  // exact symmetry, as the QP sees it
    for (int l = j + 1; l < du; ++l) {
      const double m = 0.5 * (S.Quu[(size_t)j * du + l] + S.Quu[(size_t)l * du + j]);
      S.Quu[(size_t)j * du + l] = m;
      S.Quu[(size_t)l * du + j] = m;
    }
  double* LU = (k == 0) ? S.LU0.data() : S.Quu.data();
  int* piv = (k == 0) ? S.piv0.data() : S.piv.data();
  if (k == 0) std::copy(S.Quu.begin(), S.Quu.end(), S.LU0.begin());
  if (!lu_factor(LU, du, piv)) return false;
  if (k == 0) {
    lu_solve(LU, du, piv, S.X.data(), d);
    return true;
  }
  // V_k = A V A - Qux' X + Qc_k, with Qux' X = (A W) X: scale W's rows by alpha
  for (int i = 0; i < d; ++i)
    for (int j = 0; j < du; ++j) S.W[(size_t)i * du + j] *= al[i];
  lu_solve(LU, du, piv, S.X.data(), d);
  double* q = S.qv.data();
  for (int i = 0; i < d; ++i) q[i] = exp((double)pb.lgQ[i] * k);
  for (int i = 0; i < d; ++i) {
    const double qi = q[i];
    for (int m = i; m < d; ++m) {
      double acc = 0.0;
      for (int j = 0; j < du; ++j) acc += S.W[(size_t)i * du + j] * S.X[(size_t)j * d + m];
      const double qm = q[m];
      const double vim = 0.5 * (S.V[(size_t)i * d + m] + S.V[(size_t)m * d + i]);
      const double val = al[i] * al[m] * vim - acc + qi * qm * S.Qs[(size_t)i * d + m];
      S.V[(size_t)i * d + m] = val;
      S.V[(size_t)m * d + i] = val;
    }
  }
  return true;
}

// Stage a problem's token-shared B and sym(Q), and V = sym(Q_f).
void stage(const Problem& pb, const Sizes& s, Scratch& S) {
  const int d = s.d, du = s.du;
  for (int i = 0; i < d * du; ++i) S.Bd[i] = pb.B[i];
  for (int i = 0; i < d; ++i)
    for (int m = 0; m < d; ++m) {
      S.Qs[(size_t)i * d + m] = 0.5 * ((double)pb.Q[i * d + m] + (double)pb.Q[m * d + i]);
      S.Qfs[(size_t)i * d + m] = 0.5 * ((double)pb.Qf[i * d + m] + (double)pb.Qf[m * d + i]);
    }
  std::copy(S.Qfs.begin(), S.Qfs.end(), S.V.begin());
}

bool forward_one(const Problem& pb, const Sizes& s, Scratch& S, float* u, bool keep_gains) {
  stage(pb, s, S);
  const int d = s.d, du = s.du;
  for (int k = s.T - 1; k >= 0; --k) {
    if (!riccati_step(pb, s, k, S)) return false;
    if (keep_gains)
      for (int e = 0; e < du * d; ++e) S.K[(size_t)k * du * d + e] = -S.X[e];
  }
  if (u != nullptr)
    for (int j = 0; j < du; ++j) {
      double acc = 0.0;
      for (int i = 0; i < d; ++i) acc -= S.X[(size_t)j * d + i] * (double)pb.h0[i];
      u[j] = (float)acc;
    }
  return true;
}

struct Grads {  // per-problem outputs (B / Q: accumulated into the token's head sums)
  float *gA, *gR, *gQf, *glA, *glB, *glQ, *gh0;
  double *gB, *gQ;  // token accumulators [d][du], [d][d]
};

bool backward_one(const Problem& pb, const Sizes& s, Scratch& S, const float* dU, const Grads& g) {
  const int d = s.d, du = s.du, T = s.T;
  if (!forward_one(pb, s, S, nullptr, true)) return false;
  // adjoint feed-forward w_0 = -Quu_0^{-1} d_u
  std::vector<double>& t1 = S.tmp;
  for (int j = 0; j < du; ++j) t1[j] = dU[j];
  lu_solve(S.LU0.data(), du, S.piv0.data(), t1.data(), 1);
  // closed-loop rollouts
  std::vector<double> be(du), q(d);
  for (int i = 0; i < d; ++i) { S.h[i] = pb.h0[i]; S.hb[i] = 0.0; }
  for (int k = 0; k < T; ++k) {
    const double* K = &S.K[(size_t)k * du * d];
    const double* hk = &S.h[(size_t)k * d];
    const double* hbk = &S.hb[(size_t)k * d];
    double* uk = &S.u[(size_t)k * du];
    double* wk = &S.w[(size_t)k * du];
    for (int j = 0; j < du; ++j) {
      double a1 = 0.0, a2 = (k == 0) ? -t1[j] : 0.0;
      for (int i = 0; i < d; ++i) { a1 += K[(size_t)j * d + i] * hk[i]; a2 += K[(size_t)j * d + i] * hbk[i]; }
      uk[j] = a1;
      wk[j] = a2;
    }
    const double eA = exp((double)pb.lgA[0] * (k + 1));
    for (int j = 0; j < du; ++j) be[j] = exp((double)pb.lgB[j] * (k + 1));
    for (int i = 0; i < d; ++i) {
      const double al = 1.0 + (double)pb.a[i] * eA;
      double a1 = al * hk[i], a2 = al * hbk[i];
      for (int j = 0; j < du; ++j) {
        const double bij = S.Bd[(size_t)i * du + j] * be[j];
        a1 += bij * uk[j];
        a2 += bij * wk[j];
      }
      S.h[(size_t)(k + 1) * d + i] = a1;
      S.hb[(size_t)(k + 1) * d + i] = a2;
    }
  }
  // costates and gradients, k = T-1 .. 0 (lam / lamb hold lambda_{k+1})
  double* lam = S.lam.data();
  double* lamb = S.lamb.data();
  {
    const double* hT = &S.h[(size_t)T * d];
    const double* hbT = &S.hb[(size_t)T * d];
    for (int i = 0; i < d; ++i) {
      double a1 = 0.0, a2 = 0.0;
      for (int m = 0; m < d; ++m) { a1 += S.Qfs[(size_t)i * d + m] * hT[m]; a2 += S.Qfs[(size_t)i * d + m] * hbT[m]; }
      lam[i] = a1;
      lamb[i] = a2;
    }
    for (int i = 0; i < d; ++i)
      for (int m = 0; m < d; ++m) g.gQf[i * d + m] = (float)(0.5 * (hbT[i] * hT[m] + hT[i] * hbT[m]));
  }
  std::vector<double> gA(d, 0.0), glB(du, 0.0), gR(du, 0.0), glQ(d, 0.0), cu(du), cw(du), nl(d), nlb(d);
  double glA = 0.0;
  for (int k = T - 1; k >= 0; --k) {
    const double* hk = &S.h[(size_t)k * d];
    const double* hbk = &S.hb[(size_t)k * d];
    const double* uk = &S.u[(size_t)k * du];
    const double* wk = &S.w[(size_t)k * du];
    const double eA = exp((double)pb.lgA[0] * (k + 1));
    for (int j = 0; j < du; ++j) be[j] = exp((double)pb.lgB[j] * (k + 1));
    for (int i = 0; i < d; ++i) q[i] = exp((double)pb.lgQ[i] * k);
    // A_diag / log_gamma_A: d/dalpha_k = h_k lamb_{k+1} + hb_k lam_{k+1}  (torch_lqr.py:51)
    for (int i = 0; i < d; ++i) {
      const double ga = hk[i] * lamb[i] + hbk[i] * lam[i];
      gA[i] += ga * eA;
      glA += ga * (double)pb.a[i] * (k + 1) * eA;
    }
    // B / log_gamma_B: lamb u' + lam w'  (torch_lqr.py:53), through B_k = B diag(beta_k)
    for (int j = 0; j < du; ++j) {
      double sb = 0.0;
      for (int i = 0; i < d; ++i) {
        const double gb = lamb[i] * uk[j] + lam[i] * wk[j];
        g.gB[(size_t)i * du + j] += gb * be[j];
        sb += gb * (double)pb.B[i * du + j];
      }
      glB[j] += sb * (k + 1) * be[j];
      // R_inv: d/dR = u w (torch_lqr.py:59), R = 1 / R_inv
      const double rj = (double)pb.r[j];
      gR[j] -= uk[j] * wk[j] / (rj * rj);
    }
    if (k == 0) {
      const double eA0 = exp((double)pb.lgA[0]);
      for (int i = 0; i < d; ++i) g.gh0[i] = (float)((1.0 + (double)pb.a[i] * eA0) * lamb[i]);  // torch_lqr.py:61
      break;
    }
    // state cost on h_k (k >= 1): Q / log_gamma_Q through Qc_k = D_k Q D_k  (torch_lqr.py:55)
    for (int i = 0; i < d; ++i) {
      const double qi = q[i];
      double sq = 0.0;
      for (int m = 0; m < d; ++m) {
        const double qm = q[m];
        const double G = 0.5 * (hbk[i] * hk[m] + hk[i] * hbk[m]);
        g.gQ[(size_t)i * d + m] += qi * G * qm;
        sq += G * qi * qm * S.Qs[(size_t)i * d + m];
      }
      glQ[i] += 2.0 * sq * k;
    }
    // closed-loop costate step: lambda_k = Qc_k h_k + A_k lambda_{k+1} + K_k'(R u_k + B_k' lambda_{k+1})
    const double* K = &S.K[(size_t)k * du * d];
    for (int j = 0; j < du; ++j) {
      double b1 = 0.0, b2 = 0.0;
      for (int i = 0; i < d; ++i) { b1 += S.Bd[(size_t)i * du + j] * lam[i]; b2 += S.Bd[(size_t)i * du + j] * lamb[i]; }
      const double rr = 1.0 / (double)pb.r[j];
      cu[j] = rr * uk[j] + be[j] * b1;
      cw[j] = rr * wk[j] + be[j] * b2;
    }
    for (int i = 0; i < d; ++i) {
      const double qi = q[i];
      double a1 = 0.0, a2 = 0.0;
      for (int m = 0; m < d; ++m) {
        const double qc = qi * q[m] * S.Qs[(size_t)i * d + m];
        a1 += qc * hk[m];
        a2 += qc * hbk[m];
      }
      const double al = 1.0 + (double)pb.a[i] * eA;
      double k1 = 0.0, k2 = 0.0;
      for (int j = 0; j < du; ++j) { k1 += K[(size_t)j * d + i] * cu[j]; k2 += K[(size_t)j * d + i] * cw[j]; }
      nl[i] = a1 + al * lam[i] + k1;
      nlb[i] = a2 + al * lamb[i] + k2;
    }
    for (int i = 0; i < d; ++i) { lam[i] = nl[i]; lamb[i] = nlb[i]; }
  }
  for (int i = 0; i < d; ++i) { g.gA[i] = (float)gA[i]; g.glQ[i] = (float)glQ[i]; }
  for (int j = 0; j < du; ++j) { g.glB[j] = (float)glB[j]; g.gR[j] = (float)gR[j]; }
  g.glA[0] = (float)glA;
  return true;
}

int n_workers(int32_t n_threads, int64_t n_tokens) {
  int n = n_threads > 0 ? n_threads : (int)std::thread::hardware_concurrency();
  if (n < 1) n = 1;
  if ((int64_t)n > n_tokens) n = (int)std::max<int64_t>(n_tokens, 1);
  return n;
}

// Run fn(token, scratch) over all tokens on n workers (dynamic token assignment).
template <typename F>
void parallel_tokens(int64_t n_tokens, int workers, const Sizes& s, bool backward, F fn) {
  std::atomic<int64_t> next{0};
  auto body = [&]() {
    Scratch S;
    S.init(s, backward);
    for (;;) {
      const int64_t n = next.fetch_add(1);
      if (n >= n_tokens) break;
      fn(n, S);
    }
  };
  if (workers == 1) {
    body();
    return;
  }
  std::vector<std::thread> pool;
  pool.reserve(workers);
  for (int t = 0; t < workers; ++t) pool.emplace_back(body);
  for (auto& th : pool) th.join();
}

bool args_ok(int64_t n_tokens, int32_t heads, int32_t d, int32_t du, int32_t T) {
  return n_tokens >= 0 && heads > 0 && d > 0 && du > 0 && T > 0 && d <= 4096 && du <= 4096;
}

Problem problem_at(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                   const float* lA, const float* lB, const float* lQ, const float* h0, int64_t n, int h, int H,
                   int d, int du) {
  const int64_t p = n * H + h;
  return Problem{A + p * d, B + n * (int64_t)d * du, Q + n * (int64_t)d * d, R + p * du, Qf + p * (int64_t)d * d,
                 lA + p, lB + p * du, lQ + p * d, h0 + p * d};
}

}  // namespace

extern "C" {

int ttc_lqr_forward_host(const float* A_diag, const float* B, const float* Q, const float* R_inv, const float* Q_f,
                         const float* log_gamma_A, const float* log_gamma_B, const float* log_gamma_Q,
                         const float* h0, int64_t n_tokens, int32_t heads, int32_t d, int32_t du, int32_t T,
                         float* u, int32_t* status, int32_t n_threads) {
  if (!args_ok(n_tokens, heads, d, du, T)) return TTC_LQR_EINVAL;
  if (status) *status = 0;
  if (n_tokens == 0) return TTC_LQR_OK;
  if (!A_diag || !B || !Q || !R_inv || !Q_f || !log_gamma_A || !log_gamma_B || !log_gamma_Q || !h0 || !u)
    return TTC_LQR_EINVAL;
  const Sizes s{d, du, T};
  std::atomic<int> flags{0};
  parallel_tokens(n_tokens, n_workers(n_threads, n_tokens), s, false, [&](int64_t n, Scratch& S) {
    for (int h = 0; h < heads; ++h) {
      const Problem pb = problem_at(A_diag, B, Q, R_inv, Q_f, log_gamma_A, log_gamma_B, log_gamma_Q, h0, n, h,
                                    heads, d, du);
      float* up = u + (n * heads + h) * du;
      bool ok = forward_one(pb, s, S, up, false);
      for (int j = 0; j < du && ok; ++j) ok = std::isfinite(up[j]);
      if (!ok) {
        for (int j = 0; j < du; ++j) up[j] = NAN;
        flags.fetch_or(TTC_LQR_STATUS_NONFINITE);
      }
    }
  });
  if (status) *status = flags.load();
  return TTC_LQR_OK;
}

int ttc_lqr_backward_host(const float* A_diag, const float* B, const float* Q, const float* R_inv,
                          const float* Q_f, const float* log_gamma_A, const float* log_gamma_B,
                          const float* log_gamma_Q, const float* h0, const float* d_u, int64_t n_tokens,
                          int32_t heads, int32_t d, int32_t du, int32_t T, float* grad_A_diag, float* grad_B,
                          float* grad_Q, float* grad_R_inv, float* grad_Q_f, float* grad_log_gamma_A,
                          float* grad_log_gamma_B, float* grad_log_gamma_Q, float* grad_h0, float grad_limit,
                          int32_t* status, int32_t n_threads) {
  if (!args_ok(n_tokens, heads, d, du, T)) return TTC_LQR_EINVAL;
  if (status) *status = 0;
  if (n_tokens == 0) return TTC_LQR_OK;
  if (!A_diag || !B || !Q || !R_inv || !Q_f || !log_gamma_A || !log_gamma_B || !log_gamma_Q || !h0 || !d_u ||
      !grad_A_diag || !grad_B || !grad_Q || !grad_R_inv || !grad_Q_f || !grad_log_gamma_A || !grad_log_gamma_B ||
      !grad_log_gamma_Q || !grad_h0)
    return TTC_LQR_EINVAL;
  const Sizes s{d, du, T};
  std::atomic<int> flags{0};
  // the reference's guard (fused_lqr.py:243-246): non-finite or |g| >= limit in the gradients
  // of A_diag, B, Q, R_inv, Q_f and h0
  auto check = [&](const float* v, int64_t n, int& f) {
    for (int64_t e = 0; e < n; ++e) {
      if (!std::isfinite(v[e])) f |= TTC_LQR_STATUS_NONFINITE;
      else if (fabsf(v[e]) >= grad_limit) f |= TTC_LQR_STATUS_LARGE;
    }
  };
  parallel_tokens(n_tokens, n_workers(n_threads, n_tokens), s, true, [&](int64_t n, Scratch& S) {
    std::vector<double> gB((size_t)d * du, 0.0), gQ((size_t)d * d, 0.0);
    int f = 0;
    for (int h = 0; h < heads; ++h) {
      const int64_t p = n * heads + h;
      const Problem pb = problem_at(A_diag, B, Q, R_inv, Q_f, log_gamma_A, log_gamma_B, log_gamma_Q, h0, n, h,
                                    heads, d, du);
      Grads g{grad_A_diag + p * d, grad_R_inv + p * du, grad_Q_f + p * (int64_t)d * d, grad_log_gamma_A + p,
              grad_log_gamma_B + p * du, grad_log_gamma_Q + p * d, grad_h0 + p * d, gB.data(), gQ.data()};
      if (!backward_one(pb, s, S, d_u + p * du, g)) {
        // singular or non-finite gain solve: NaN gradients, reported through the status word
        for (int i = 0; i < d; ++i) g.gA[i] = g.glQ[i] = g.gh0[i] = NAN;
        for (int j = 0; j < du; ++j) g.gR[j] = g.glB[j] = NAN;
        for (int e = 0; e < d * d; ++e) g.gQf[e] = NAN;
        g.glA[0] = NAN;
        for (auto& v : gB) v = NAN;
        for (auto& v : gQ) v = NAN;
      }
      check(g.gA, d, f);
      check(g.gR, du, f);
      check(g.gQf, (int64_t)d * d, f);
      check(g.gh0, d, f);
    }
    float* ob = grad_B + n * (int64_t)d * du;
    float* oq = grad_Q + n * (int64_t)d * d;
    for (size_t e = 0; e < gB.size(); ++e) ob[e] = (float)gB[e];
    for (size_t e = 0; e < gQ.size(); ++e) oq[e] = (float)gQ[e];
    check(ob, (int64_t)d * du, f);
    check(oq, (int64_t)d * d, f);
    if (f) flags.fetch_or(f);
  });
  if (status) *status = flags.load();
  return TTC_LQR_OK;
}

}  // extern "C"
