/*
 * Float64 token-by-token Mamba-2 SSD recurrence: forward and adjoint backward.
 *
 * Test infrastructure only (an independent pin for the torch restatement in
 * oracle/ssd_reference.py); nothing in the product links it.
 *
 * Forward (mamba_torch/ssd_reference.py:10-77,
 * mamba_ascendc/csrc/ops/mamba2_ssd_fwd/design.md:10-20):
 *   u_t = dt_t + bias ; q_t = clamp(softplus(u_t) or u_t, lo, hi)
 *   S_t = exp(A q_t) S_{t-1} + (x_t q_t) (x) B_t
 *   ypre_t = S_t . C_t + D x_t ; out_t = ypre_t * silu(z_t)
 *
 * Backward is the reverse-time adjoint of that recurrence
 * (mamba_ascendc/csrc/ops/mamba2_ssd_bwd/design.md:73-107 states the same
 * equations; mamba_ascendc/csrc/ops/mamba2_ssd_dt_bwd/design.md gives the
 * clamp/softplus chain: the clamp passes the gradient where lo <= q_pre <= hi).
 *
 * Layouts (all contiguous, row-major): x, z, out [b,l,h,p]; dt [b,l,h];
 * A, bias [h]; B, C [b,l,g,n]; D [h] (d_mode 1) or [h,p] (d_mode 2);
 * init, final [b,h,p,n].  Optional pointers may be NULL.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

static double softplus(double u) { return u > 20.0 ? u : log1p(exp(u)); }
static double sigmoid(double u) { return 1.0 / (1.0 + exp(-u)); }

typedef struct {
    long b, l, h, p, g, n;
} dims_t;

static void discretize(const double *dt, const double *bias, long h_idx, int softplus_on,
                       double lo, double hi, double *q, double *dq_du)
{
    double u = *dt + (bias ? bias[h_idx] : 0.0);
    double pre = softplus_on ? softplus(u) : u;
    double grad = (pre >= lo && pre <= hi) ? 1.0 : 0.0;
    if (softplus_on) grad *= sigmoid(u);
    *q = pre < lo ? lo : (pre > hi ? hi : pre);
    *dq_du = grad;
}

int ssd_seq_fwd(long b, long l, long h, long p, long g, long n,
                int softplus_on, double lo, double hi, int d_mode,
                const double *x, const double *dt, const double *A,
                const double *B, const double *C, const double *D,
                const double *z, const double *bias, const double *init,
                double *out, double *final_state)
{
    if (h % g) return -1;
    long r = h / g;
    double *S = (double *)malloc(sizeof(double) * (size_t)(p * n));
    if (!S) return -2;
    for (long bi = 0; bi < b; ++bi)
        for (long hi_ = 0; hi_ < h; ++hi_) {
            long gi = hi_ / r;
            if (init)
                memcpy(S, init + (bi * h + hi_) * p * n, sizeof(double) * (size_t)(p * n));
            else
                memset(S, 0, sizeof(double) * (size_t)(p * n));
            for (long t = 0; t < l; ++t) {
                double q, dqdu;
                discretize(dt + (bi * l + t) * h + hi_, bias, hi_, softplus_on, lo, hi, &q, &dqdu);
                double a = exp(A[hi_] * q);
                const double *xt = x + ((bi * l + t) * h + hi_) * p;
                const double *Bt = B + ((bi * l + t) * g + gi) * n;
                const double *Ct = C + ((bi * l + t) * g + gi) * n;
                double *ot = out + ((bi * l + t) * h + hi_) * p;
                for (long pi = 0; pi < p; ++pi) {
                    double v = xt[pi] * q, acc = 0.0;
                    double *Sp = S + pi * n;
                    for (long ni = 0; ni < n; ++ni) {
                        Sp[ni] = a * Sp[ni] + v * Bt[ni];
                        acc += Sp[ni] * Ct[ni];
                    }
                    if (d_mode == 1) acc += D[hi_] * xt[pi];
                    if (d_mode == 2) acc += D[hi_ * p + pi] * xt[pi];
                    if (z) {
                        double zz = z[((bi * l + t) * h + hi_) * p + pi];
                        acc *= zz * sigmoid(zz);
                    }
                    ot[pi] = acc;
                }
            }
            if (final_state)
                memcpy(final_state + (bi * h + hi_) * p * n, S, sizeof(double) * (size_t)(p * n));
        }
    free(S);
    return 0;
}

/* Gradients are accumulated into the outputs, which the caller zero-fills.
 * dout or dfinal may be NULL (treated as zero). */
int ssd_seq_bwd(long b, long l, long h, long p, long g, long n,
                int softplus_on, double lo, double hi, int d_mode,
                const double *x, const double *dt, const double *A,
                const double *B, const double *C, const double *D,
                const double *z, const double *bias, const double *init,
                const double *dout, const double *dfinal,
                double *dx, double *ddt, double *dA, double *dB, double *dC,
                double *dD, double *dz, double *dbias, double *dinit)
{
    if (h % g) return -1;
    long r = h / g;
    size_t pn = (size_t)(p * n);
    double *Sall = (double *)malloc(sizeof(double) * pn * (size_t)(l + 1));
    double *gS = (double *)malloc(sizeof(double) * pn);
    double *qs = (double *)malloc(sizeof(double) * (size_t)l * 2);
    double *gy = (double *)malloc(sizeof(double) * (size_t)p);
    double *dv = (double *)malloc(sizeof(double) * (size_t)p);
    if (!Sall || !gS || !qs || !gy || !dv) {
        free(Sall); free(gS); free(qs); free(gy); free(dv);
        return -2;
    }
    for (long bi = 0; bi < b; ++bi)
        for (long hh = 0; hh < h; ++hh) {
            long gi = hh / r;
            /* forward sweep keeping every state: Sall[t+1] = S_t, Sall[0] = S_{-1} */
            if (init)
                memcpy(Sall, init + (bi * h + hh) * pn, sizeof(double) * pn);
            else
                memset(Sall, 0, sizeof(double) * pn);
            for (long t = 0; t < l; ++t) {
                double q, dqdu;
                discretize(dt + (bi * l + t) * h + hh, bias, hh, softplus_on, lo, hi, &q, &dqdu);
                qs[2 * t] = q;
                qs[2 * t + 1] = dqdu;
                double a = exp(A[hh] * q);
                const double *xt = x + ((bi * l + t) * h + hh) * p;
                const double *Bt = B + ((bi * l + t) * g + gi) * n;
                const double *Sp = Sall + (size_t)t * pn;
                double *Sn = Sall + (size_t)(t + 1) * pn;
                for (long pi = 0; pi < p; ++pi)
                    for (long ni = 0; ni < n; ++ni)
                        Sn[pi * n + ni] = a * Sp[pi * n + ni] + xt[pi] * q * Bt[ni];
            }
            if (dfinal)
                memcpy(gS, dfinal + (bi * h + hh) * pn, sizeof(double) * pn);
            else
                memset(gS, 0, sizeof(double) * pn);
            for (long t = l - 1; t >= 0; --t) {
                double q = qs[2 * t], dqdu = qs[2 * t + 1];
                double a = exp(A[hh] * q);
                long xo = ((bi * l + t) * h + hh) * p;
                const double *xt = x + xo;
                const double *Bt = B + ((bi * l + t) * g + gi) * n;
                const double *Ct = C + ((bi * l + t) * g + gi) * n;
                const double *St = Sall + (size_t)(t + 1) * pn;
                const double *Sprev = Sall + (size_t)t * pn;
                for (long pi = 0; pi < p; ++pi) {
                    double go = dout ? dout[xo + pi] : 0.0;
                    double dcoef = d_mode == 1 ? D[hh] : (d_mode == 2 ? D[hh * p + pi] : 0.0);
                    if (z) {
                        double zz = z[xo + pi], sg = sigmoid(zz);
                        double ypre = dcoef * xt[pi];
                        for (long ni = 0; ni < n; ++ni) ypre += St[pi * n + ni] * Ct[ni];
                        gy[pi] = go * zz * sg;
                        dz[xo + pi] += go * ypre * sg * (1.0 + zz * (1.0 - sg));
                    } else {
                        gy[pi] = go;
                    }
                    if (d_mode == 1) dD[hh] += gy[pi] * xt[pi];
                    if (d_mode == 2) dD[hh * p + pi] += gy[pi] * xt[pi];
                }
                double *dCt = dC + ((bi * l + t) * g + gi) * n;
                double *dBt = dB + ((bi * l + t) * g + gi) * n;
                double da = 0.0;
                for (long pi = 0; pi < p; ++pi) {
                    double acc_dv = 0.0, v = xt[pi] * q;
                    for (long ni = 0; ni < n; ++ni) {
                        double gs = gS[pi * n + ni] + gy[pi] * Ct[ni];
                        gS[pi * n + ni] = gs;
                        dCt[ni] += gy[pi] * St[pi * n + ni];
                        da += gs * a * Sprev[pi * n + ni];
                        dBt[ni] += gs * v;
                        acc_dv += gs * Bt[ni];
                    }
                    dv[pi] = acc_dv;
                }
                for (long k = 0; k < (long)pn; ++k) gS[k] *= a;
                double dq = A[hh] * da;
                for (long pi = 0; pi < p; ++pi) {
                    double dcoef = d_mode == 1 ? D[hh] : (d_mode == 2 ? D[hh * p + pi] : 0.0);
                    dx[xo + pi] += q * dv[pi] + gy[pi] * dcoef;
                    dq += dv[pi] * xt[pi];
                }
                dA[hh] += da * q;
                double dd = dq * dqdu;
                ddt[(bi * l + t) * h + hh] += dd;
                if (dbias) dbias[hh] += dd;
            }
            if (dinit)
                for (size_t k = 0; k < pn; ++k) dinit[(bi * h + hh) * pn + k] += gS[k];
        }
    free(Sall); free(gS); free(qs); free(gy); free(dv);
    return 0;
}
