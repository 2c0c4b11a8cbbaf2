/*
 * CPU oracle for the Flash-EKV LUT CIMLinear. TEST INFRASTRUCTURE ONLY: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and
 * only as the checker. The product path (isa-_amd/) never calls it.
 *
 * Restates the reference algorithm with an fp32 table:
 *   - table: src/isa/approximations/delta_lut.py:25-34 (evaluated in fp64, rounded once
 *     to fp32; the reference's final bf16 cast at :35 is the separate bf16 mode),
 *   - lookup: src/isa/kernels/transformer_ffn/cuda/ekv_cuda.cu:19-36 (clamp with
 *     fminf/fmaxf, so a NaN coordinate reads entry 0; trunc; i1 = min(i0+1, N-1);
 *     fmaf(alpha, q1 - q0, q0)), scale as ekv_cuda.cu:371,
 *   - forward: src/isa/kernels/transformer_ffn/ekv_lut_triton.py:52-61,
 *   - backward: ekv_cuda.cu:224-250 (dX) and :324-339 (dVth+-).
 * Every per-cell quantity is computed in fp32 as the reference does; only the sums
 * over k, o or m are carried in double, so the oracle is the reference's arithmetic
 * without its accumulation-order rounding.
 *
 * Pinned (tests/test_oracle.py): the table against the closed form and the reference's
 * own test grid (tests/test_flash_formula.py:56-84), forward and backward against the
 * exact formula and its autograd gradients as N grows, and the invariants
 * vth_pos == vth_neg -> 0, swap -> negation, additivity over K, linearity in G.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>

static double softplus_ref(double u) { return u > 20.0 ? u : log1p(exp(u)); }

static double sig_from_sp(double sp) { return sp > 20.0 ? 1.0 : -expm1(-sp); }

/* delta_lut.py:25-34 on the grid linspace(delta_min, delta_max, n_entries) */
void oracle_lut_build(double n, double u_t, double i_s, double v_d, double delta_min, double delta_max,
                      int n_entries, float* table_i, float* table_ddelta) {
    const double inv_2nut = 1.0 / (2.0 * n * u_t);
    for (int j = 0; j < n_entries; ++j) {
        const double delta =
            n_entries > 1 ? delta_min + (double)j * ((delta_max - delta_min) / (double)(n_entries - 1)) : delta_min;
        const double sp1 = softplus_ref(delta * inv_2nut);
        const double sp2 = softplus_ref((delta - v_d) * inv_2nut);
        table_i[j] = (float)(i_s * (sp1 * sp1 - sp2 * sp2));
        table_ddelta[j] = (float)(i_s * 2.0 * inv_2nut * (sp1 * sig_from_sp(sp1) - sp2 * sig_from_sp(sp2)));
    }
}

/* ekv_cuda.cu:19-36 */
static inline float lut_lookup(const float* table, float delta, float delta_min, float scale, int size) {
    float c = (delta - delta_min) * scale;
    c = fminf(fmaxf(c, 0.0f), (float)(size - 1));
    const int i0 = (int)c;
    const int i1 = i0 + 1 < size - 1 ? i0 + 1 : size - 1;
    const float alpha = c - (float)i0;
    const float q0 = table[i0];
    const float q1 = table[i1];
    return fmaf(alpha, q1 - q0, q0);
}

static inline float lut_scale(int size, double delta_min, double delta_max) {
    return (float)((double)(size - 1) / (delta_max - delta_min));
}

/* out[m,o] = clamp(sum_k (L(x-wp) - L(x-wn)) / (1 + x/v_sat), out_min, out_max)
 * (ekv_lut_triton.py:52-61); sum in double. */
void oracle_forward(const float* x, const float* wp, const float* wn, const float* table_i, int64_t M, int64_t K,
                    int64_t O, int size, double delta_min, double delta_max, float v_sat, double out_min,
                    double out_max, double* out) {
    const float scale = lut_scale(size, delta_min, delta_max);
    const float dmin = (float)delta_min;
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m) {
        const float* xr = x + m * K;
        for (int64_t o = 0; o < O; ++o) {
            const float* pr = wp + o * K;
            const float* nr = wn + o * K;
            double acc = 0.0;
            for (int64_t k = 0; k < K; ++k) {
                const float xv = xr[k];
                const float bp = lut_lookup(table_i, xv - pr[k], dmin, scale, size);
                const float bn = lut_lookup(table_i, xv - nr[k], dmin, scale, size);
                const float denom = 1.0f + xv / v_sat;
                acc += (double)(bp - bn) / (double)denom;
            }
            /* fmin/fmax (non-NaN operand wins), as the kernels' fminf/fmaxf clamp */
            out[m * O + o] = fmin(fmax(acc, out_min), out_max);
        }
    }
}

/* ekv_cuda.cu:224-250: dX[m,k] = sum_o G[m,o] ((Dp - Dn) inv_d - (Ip - In) / (v_sat d^2)) */
void oracle_grad_x(const float* x, const float* wp, const float* wn, const float* grad, const float* table_i,
                   const float* table_ddelta, int64_t M, int64_t K, int64_t O, int size, double delta_min,
                   double delta_max, float v_sat, double* grad_x) {
    const float scale = lut_scale(size, delta_min, delta_max);
    const float dmin = (float)delta_min;
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m) {
        const float* gr = grad + m * O;
        for (int64_t k = 0; k < K; ++k) {
            const float xv = x[m * K + k];
            const float denominator = 1.0f + xv / v_sat;
            const float inv_denominator = 1.0f / denominator;
            const float denominator_term = 1.0f / (v_sat * denominator * denominator);
            double acc = 0.0;
            for (int64_t o = 0; o < O; ++o) {
                const float dp = xv - wp[o * K + k];
                const float dn = xv - wn[o * K + k];
                const float ip = lut_lookup(table_i, dp, dmin, scale, size);
                const float in = lut_lookup(table_i, dn, dmin, scale, size);
                const float gp = lut_lookup(table_ddelta, dp, dmin, scale, size);
                const float gn = lut_lookup(table_ddelta, dn, dmin, scale, size);
                const float derivative = (gp - gn) * inv_denominator - (ip - in) * denominator_term;
                acc += (double)gr[o] * (double)derivative;
            }
            grad_x[m * K + k] = acc;
        }
    }
}

/* ekv_cuda.cu:324-339: dVth+[o,k] = -sum_m G D(x-wp)/d, dVth-[o,k] = +sum_m G D(x-wn)/d */
void oracle_grad_w(const float* x, const float* wp, const float* wn, const float* grad, const float* table_ddelta,
                   int64_t M, int64_t K, int64_t O, int size, double delta_min, double delta_max, float v_sat,
                   double* grad_wp, double* grad_wn) {
    const float scale = lut_scale(size, delta_min, delta_max);
    const float dmin = (float)delta_min;
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < O; ++o) {
        for (int64_t k = 0; k < K; ++k) {
            const float p = wp[o * K + k];
            const float q = wn[o * K + k];
            double acc_p = 0.0, acc_n = 0.0;
            for (int64_t m = 0; m < M; ++m) {
                const float xv = x[m * K + k];
                const float g = grad[m * O + o];
                const float inv_denominator = 1.0f / (1.0f + xv / v_sat);
                const float gp = lut_lookup(table_ddelta, xv - p, dmin, scale, size);
                const float gn = lut_lookup(table_ddelta, xv - q, dmin, scale, size);
                acc_p += (double)g * (double)(-gp * inv_denominator);
                acc_n += (double)g * (double)(gn * inv_denominator);
            }
            grad_wp[o * K + k] = acc_p;
            grad_wn[o * K + k] = acc_n;
        }
    }
}

/* Single lookup, exposed for the boundary tests (clamp ends, nodes, NaN). */
float oracle_lut_lookup(const float* table, float delta, double delta_min, double delta_max, int size) {
    return lut_lookup(table, delta, (float)delta_min, lut_scale(size, delta_min, delta_max), size);
}
