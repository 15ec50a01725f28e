/*
 * f16_oracle.c -- CPU restatement of the reference's double-precision F-16 model
 * (the Python modules under cuda_fdm/ref/) and of its IC seeding (cuda_fdm/ic.py).
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP path and the
 * CPU baseline timed by bench.py.  Nothing in the product package may link, load or call
 * it; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg do.
 *
 * Each function restates the Python reference operation for operation (same operand
 * order, same libm calls: Python's `x ** y` is C pow(), math.* are the libm functions), so
 * that with gcc -O2 -ffp-contract=off on x86-64 the results are the ones the Python
 * reference produces.  Citations name the Python file:line each block follows.
 *
 * Pinning (what checks this file, besides "it reads like the reference"):
 *   - tables: exact at breakpoints, clamped ends, bilinear closed forms (tests);
 *   - ISA: sea-level known answers quoted by the reference (f16_gen.cuh:20-47 values);
 *   - mass: J * Jinv = I, closed forms at 0/3000/6000/6972 lb;
 *   - frames: |q| = 1, orthonormal DCMs, Euler<->quat round trips;
 *   - composed fdm_step: oracle/_ref, the reference's own host-compilable C
 *     (cuda_fdm/gen/fdm.cuh) built from its sources, compared per step and per trajectory;
 *   - seed: golden vectors written by tests/golden/make_fdm_golden.py from cuda_fdm/ic.py.
 *
 * State vector: 101 doubles in the reference's FdmState order (cuda_fdm/ic.py:92-114).
 */
#include <math.h>
#include <string.h>
#include <stdint.h>

#include "../2026_ai_pilot_challenge-1st_solution_amd/csrc/f16_model_gen.h"

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ constants */
/* cuda_fdm/ref/jsb_const.py:6-28 */
#define RADTODEG 57.295779513082320876798154814105
#define KTSTOFPS 1.68781
#define INCHTOFT (1.0 / 12)
#define FTTOM 0.3048
#define SLUGTOLB 32.174049
#define LBTOSLUG (1.0 / SLUGTOLB)
#define KGTOSLUG 0.06852168
#define KtoDegR 1.8
static const double FPSTOKTS = 1.0 / KTSTOFPS;
static const double Rstar = 8.31432 * (KGTOSLUG / (KtoDegR * FTTOM * FTTOM));
static const double Mair = 28.9645 * KGTOSLUG / 1000.0;
static const double g0 = 9.80665 / FTTOM;
#define SHRatio 1.40
#define StdDaySLtemperature 518.67
#define StdDaySLpressure 2116.228
static const double EarthRadius = 6356766.0 / FTTOM;   /* jsb_const.py:40 */

/* cuda_fdm/ref/jsb_frames.py:9-19 */
#define SEMI_MAJOR 20925646.32546
#define SEMI_MINOR 20855486.5951
#define GM 14.0764417572E15
#define J2 1.08262982E-03
#define ROTATION_RATE 0.00007292115
static const double EC = SEMI_MINOR / SEMI_MAJOR;
#define SEA_LEVEL_RADIUS_ SEMI_MAJOR   /* jsb_fdm.py:20 */

/* cuda_fdm/ref/jsb_fdm.py:18-20 */
static const double DT = 1.0 / 60.0;

/* ISA rows (jsb_const.py:30-39) */
static const double ATM_ALT[9] = {0.0000, 36089.2388, 65616.7979, 104986.8766, 154199.4751,
                                  167322.8346, 232939.6325, 278385.8268, 298556.4304};
static const double ATM_TMP[9] = {518.67, 389.97, 389.97, 411.57, 487.17, 487.17, 386.37,
                                  336.5028, 336.5028};

static const double F16M_IMAGE[F16M_IMAGE_LEN] = F16M_IMAGE_INIT;
static const f16m_aero_term AERO_TERMS[F16M_NAERO] = F16M_AERO_TERMS_INIT;

/* derived tables computed once, as the reference computes them at construction */
static double g_lapse[8], g_pbrk[9], g_dbrk[9];
static double g_idleff, g_slgravity, g_ec2, g_e2, g_std_sl_soundspeed;
static int g_init = 0;

void orc_init(void)
{
    if (g_init) return;
    /* StandardAtmosphere.__init__ (jsb_atmos.py:11-33) */
    for (int b = 0; b < 8; b++)
        g_lapse[b] = (ATM_TMP[b + 1] - ATM_TMP[b]) / (ATM_ALT[b + 1] - ATM_ALT[b]);
    g_pbrk[0] = StdDaySLpressure;
    for (int b = 0; b < 8; b++) {
        double Tmb = ATM_TMP[b], deltaH = ATM_ALT[b + 1] - ATM_ALT[b], Lmb = g_lapse[b];
        if (Lmb != 0.0) {
            double Exp = g0 * Mair / (Rstar * Lmb);
            double factor = Tmb / (Tmb + Lmb * deltaH);
            g_pbrk[b + 1] = g_pbrk[b] * pow(factor, Exp);
        } else {
            g_pbrk[b + 1] = g_pbrk[b] * exp(-g0 * Mair * deltaH / (Rstar * Tmb));
        }
    }
    /* __init_density_bp (jsb_atmos.py:74-76) */
    double Reng = Rstar / Mair;
    for (int i = 0; i < 9; i++) g_dbrk[i] = g_pbrk[i] / (Reng * ATM_TMP[i]);
    g_idleff = pow(F16M_ENG_MILTHRUST, 0.2) * 107.0;               /* jsb_propulsion.py:23 */
    g_slgravity = GM / (SEMI_MAJOR * SEMI_MAJOR);                   /* jsb_fdm.py:19 */
    g_ec2 = EC * EC;                                                /* jsb_frames.py:16-18 */
    g_e2 = 1.0 - g_ec2;
    g_std_sl_soundspeed = sqrt(SHRatio * Reng * StdDaySLtemperature); /* jsb_auxiliary.py:17 */
    g_init = 1;
}

/* ------------------------------------------------------------------ tables */
/* Table1D.value (jsb_tables.py:22-40) */
static double table1d(const double *x, const double *y, int n, double key)
{
    if (key <= x[0]) return y[0];
    if (key >= x[n - 1]) return y[n - 1];
    int r = 1;
    while (r < n - 1 && x[r] < key) r++;
    double span = x[r] - x[r - 1], factor;
    if (span != 0.0) {
        factor = (key - x[r - 1]) / span;
        if (factor > 1.0) factor = 1.0;
    } else {
        factor = 1.0;
    }
    return factor * (y[r] - y[r - 1]) + y[r - 1];
}

/* Table2D.value (jsb_tables.py:52-80) */
static double table2d(const double *rx, int nr, const double *cx, int nc, const double *d,
                      double rowKey, double colKey)
{
    int r = 1;
    while (r < nr - 1 && rx[r] < rowKey) r++;
    while (r > 1 && rx[r - 1] > rowKey) r--;
    int c = 1;
    while (c < nc - 1 && cx[c] < colKey) c++;
    while (c > 1 && cx[c - 1] > colKey) c--;
    double rF = (rowKey - rx[r - 1]) / (rx[r] - rx[r - 1]);
    double cF = (colKey - cx[c - 1]) / (cx[c] - cx[c - 1]);
    if (rF > 1.0) rF = 1.0; else if (rF < 0.0) rF = 0.0;
    if (cF > 1.0) cF = 1.0; else if (cF < 0.0) cF = 0.0;
    double col1 = rF * (d[r * nc + c - 1] - d[(r - 1) * nc + c - 1]) + d[(r - 1) * nc + c - 1];
    double col2 = rF * (d[r * nc + c] - d[(r - 1) * nc + c]) + d[(r - 1) * nc + c];
    return col1 + cF * (col2 - col1);
}

#define T1(name, key) table1d(F16M_IMAGE + F16M_T_##name##_RG, F16M_IMAGE + F16M_T_##name##_OFF, \
                              F16M_T_##name##_NR, (key))
#define T2(name, rk, ck) table2d(F16M_IMAGE + F16M_T_##name##_RG, F16M_T_##name##_NR,          \
                                 F16M_IMAGE + F16M_T_##name##_CG, F16M_T_##name##_NC,          \
                                 F16M_IMAGE + F16M_T_##name##_OFF, (rk), (ck))

/* exported for table unit tests */
double orc_table1d(const double *x, const double *y, int n, double key) { return table1d(x, y, n, key); }
double orc_table2d(const double *rx, int nr, const double *cx, int nc, const double *d, double r, double c)
{ return table2d(rx, nr, cx, nc, d, r, c); }
const double *orc_model_image(void) { return F16M_IMAGE; }

/* ------------------------------------------------------------------ linear algebra */
/* jsb_lin.py:5-43 (matmul uses Python sum(), whose integer 0 start is exact) */
static void matmul(const double A[3][3], const double B[3][3], double O[3][3])
{
    for (int i = 0; i < 3; i++)
        for (int j = 0; j < 3; j++)
            O[i][j] = A[i][0] * B[0][j] + A[i][1] * B[1][j] + A[i][2] * B[2][j];
}
static void matvec(const double A[3][3], const double v[3], double o[3])
{
    double a = A[0][0] * v[0] + A[0][1] * v[1] + A[0][2] * v[2];
    double b = A[1][0] * v[0] + A[1][1] * v[1] + A[1][2] * v[2];
    double c = A[2][0] * v[0] + A[2][1] * v[1] + A[2][2] * v[2];
    o[0] = a; o[1] = b; o[2] = c;
}
static void transpose(const double A[3][3], double O[3][3])
{
    for (int i = 0; i < 3; i++)
        for (int j = 0; j < 3; j++) O[i][j] = A[j][i];
}
static void cross(const double a[3], const double b[3], double o[3])
{
    double x = a[1] * b[2] - a[2] * b[1];
    double y = a[2] * b[0] - a[0] * b[2];
    double z = a[0] * b[1] - a[1] * b[0];
    o[0] = x; o[1] = y; o[2] = z;
}
static const double OMEGA[3] = {0.0, 0.0, ROTATION_RATE};

/* ------------------------------------------------------------------ frames */
/* jsb_frames.py:25-27 */
static void Ti2ec_from_epa(double epa, double T[3][3])
{
    double ce = cos(epa), se = sin(epa);
    T[0][0] = ce;  T[0][1] = se; T[0][2] = 0.0;
    T[1][0] = -se; T[1][1] = ce; T[1][2] = 0.0;
    T[2][0] = 0.0; T[2][1] = 0.0; T[2][2] = 1.0;
}

/* location_derived (jsb_frames.py:30-66); the geodetic latitude/altitude it also returns
 * are not consumed by the step or the seed and are omitted. */
static void location_derived(const double ecef[3], double *radius, double *mLat, double Tl2ec[3][3])
{
    double x = ecef[0], y = ecef[1], z = ecef[2];
    double rad = sqrt(x * x + y * y + z * z);
    double rxy = sqrt(x * x + y * y);
    double sinLon, cosLon, sinLat, cosLat;
    if (rxy == 0.0) { sinLon = 0.0; cosLon = 1.0; } else { sinLon = y / rxy; cosLon = x / rxy; }
    if (rad == 0.0) { sinLat = 0.0; cosLat = 1.0; } else { sinLat = z / rad; cosLat = rxy / rad; }
    *mLat = (rxy == 0.0 && z == 0.0) ? 0.0 : atan2(z, rxy);
    double Tec2l[3][3] = {{-cosLon * sinLat, -sinLon * sinLat, cosLat},
                          {-sinLon, cosLon, 0.0},
                          {-cosLon * cosLat, -sinLon * cosLat, -sinLat}};
    transpose(Tec2l, Tl2ec);
    *radius = rad;
}

/* gravity_j2 (jsb_frames.py:69-80) */
static void gravity_j2(const double ecef[3], double latitude, double o[3])
{
    double x = ecef[0], y = ecef[1], z = ecef[2];
    double r = sqrt(x * x + y * y + z * z);
    double sinLat = sin(latitude);
    double adivr = SEMI_MAJOR / r;
    double preCommon = 1.5 * J2 * adivr * adivr;
    double xy = 1.0 - 5.0 * (sinLat * sinLat);
    double zz = 3.0 - 5.0 * (sinLat * sinLat);
    double GMOverr2 = GM / (r * r);
    o[0] = -GMOverr2 * ((1.0 + (preCommon * xy)) * x / r);
    o[1] = -GMOverr2 * ((1.0 + (preCommon * xy)) * y / r);
    o[2] = -GMOverr2 * ((1.0 + (preCommon * zz)) * z / r);
}

/* quat_to_T (jsb_frames.py:84-94) */
static void quat_to_T(const double q[4], double T[3][3])
{
    double q0 = q[0], q1 = q[1], q2 = q[2], q3 = q[3];
    double q0q0 = q0 * q0, q1q1 = q1 * q1, q2q2 = q2 * q2, q3q3 = q3 * q3;
    double q0q1 = q0 * q1, q0q2 = q0 * q2, q0q3 = q0 * q3;
    double q1q2 = q1 * q2, q1q3 = q1 * q3, q2q3 = q2 * q3;
    T[0][0] = q0q0 + q1q1 - q2q2 - q3q3; T[0][1] = 2.0 * (q1q2 + q0q3); T[0][2] = 2.0 * (q1q3 - q0q2);
    T[1][0] = 2.0 * (q1q2 - q0q3); T[1][1] = q0q0 - q1q1 + q2q2 - q3q3; T[1][2] = 2.0 * (q2q3 + q0q1);
    T[2][0] = 2.0 * (q1q3 + q0q2); T[2][1] = 2.0 * (q2q3 - q0q1); T[2][2] = q0q0 - q1q1 - q2q2 + q3q3;
}

/* quat_normalize (jsb_frames.py:179-184) */
static void quat_normalize(double q[4])
{
    double mag = sqrt(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]);
    if (mag == 0.0) return;
    double inv = 1.0 / mag;
    q[0] = q[0] * inv; q[1] = q[1] * inv; q[2] = q[2] * inv; q[3] = q[3] * inv;
}

/* euler_to_quat (jsb_frames.py:97-107) */
static void euler_to_quat(double phi, double tht, double psi, double q[4])
{
    double thtd2 = 0.5 * tht, psid2 = 0.5 * psi, phid2 = 0.5 * phi;
    double St = sin(thtd2), Sp = sin(psid2), Sf = sin(phid2);
    double Ct = cos(thtd2), Cp = cos(psid2), Cf = cos(phid2);
    double CfCt = Cf * Ct, CfSt = Cf * St, SfSt = Sf * St, SfCt = Sf * Ct;
    q[0] = CfCt * Cp + SfSt * Sp;
    q[1] = SfCt * Cp - CfSt * Sp;
    q[2] = CfSt * Cp + SfCt * Sp;
    q[3] = CfCt * Sp - SfSt * Cp;
    quat_normalize(q);
}

/* mat_to_quat (jsb_frames.py:110-137): FGMatrix33 data[] is column-major */
static void mat_to_quat(const double m[3][3], double Q[4])
{
    double d[9] = {m[0][0], m[1][0], m[2][0], m[0][1], m[1][1], m[2][1], m[0][2], m[1][2], m[2][2]};
    double t[4] = {1.0 + d[0] + d[4] + d[8], 1.0 + d[0] - d[4] - d[8],
                   1.0 - d[0] + d[4] - d[8], 1.0 - d[0] - d[4] + d[8]};
    int idx = 0;
    for (int i = 1; i < 4; i++)
        if (t[i] > t[idx]) idx = i;
    Q[0] = Q[1] = Q[2] = Q[3] = 0.0;
    if (idx == 0) {
        Q[0] = 0.5 * sqrt(t[0]);
        Q[1] = 0.25 * (d[7] - d[5]) / Q[0];
        Q[2] = 0.25 * (d[2] - d[6]) / Q[0];
        Q[3] = 0.25 * (d[3] - d[1]) / Q[0];
    } else if (idx == 1) {
        Q[1] = 0.5 * sqrt(t[1]);
        Q[0] = 0.25 * (d[7] - d[5]) / Q[1];
        Q[2] = 0.25 * (d[3] + d[1]) / Q[1];
        Q[3] = 0.25 * (d[2] + d[6]) / Q[1];
    } else if (idx == 2) {
        Q[2] = 0.5 * sqrt(t[2]);
        Q[0] = 0.25 * (d[2] - d[6]) / Q[2];
        Q[1] = 0.25 * (d[3] + d[1]) / Q[2];
        Q[3] = 0.25 * (d[7] + d[5]) / Q[2];
    } else {
        Q[3] = 0.5 * sqrt(t[3]);
        Q[0] = 0.25 * (d[3] - d[1]) / Q[3];
        Q[1] = 0.25 * (d[6] + d[2]) / Q[3];
        Q[2] = 0.25 * (d[7] + d[5]) / Q[3];
    }
}

/* mat_to_euler (jsb_frames.py:140-163) */
static void mat_to_euler(const double m[3][3], double e[3])
{
    double d6 = m[0][2], theta, phi, psi;
    int gimbal = 0;
    if (d6 <= -1.0) { theta = 0.5 * M_PI; gimbal = 1; }
    else if (1.0 <= d6) { theta = -0.5 * M_PI; gimbal = 1; }
    else theta = asin(-d6);
    if (gimbal) { phi = atan2(-m[2][1], m[1][1]); psi = 0.0; }
    else {
        phi = atan2(m[1][2], m[2][2]);
        psi = atan2(m[0][1], m[0][0]);
        if (psi < 0.0) psi += 2 * M_PI;
    }
    e[0] = phi; e[1] = theta; e[2] = psi;
}

/* quat_qdot (jsb_frames.py:170-176) */
static void quat_qdot(const double q[4], const double pqr[3], double o[4])
{
    double p = pqr[0], qq = pqr[1], r = pqr[2];
    o[0] = -0.5 * (q[1] * p + q[2] * qq + q[3] * r);
    o[1] = 0.5 * (q[0] * p - q[3] * qq + q[2] * r);
    o[2] = 0.5 * (q[3] * p + q[0] * qq - q[1] * r);
    o[3] = 0.5 * (-q[2] * p + q[1] * qq + q[0] * r);
}

/* ------------------------------------------------------------------ atmosphere */
static double atm_geopot(double h) { double ER = EarthRadius; return (h * ER) / (ER + h); }      /* jsb_atmos.py:35-37 */
static double atm_geometric(double g) { double ER = EarthRadius; return (g * ER) / (ER - g); }   /* jsb_atmos.py:39-41 */

static double atm_temperature(double altitude)     /* jsb_atmos.py:43-49 */
{
    double gp = atm_geopot(altitude);
    if (gp >= 0.0) return table1d(ATM_ALT, ATM_TMP, 9, gp);
    return table1d(ATM_ALT, ATM_TMP, 9, 0.0) + gp * g_lapse[0];
}

static double atm_pressure(double altitude)        /* jsb_atmos.py:51-72 */
{
    double gp = atm_geopot(altitude);
    double BaseAlt = ATM_ALT[0];
    int b = 0;
    for (int bb = 0; bb < 9 - 2; bb++) {
        double testAlt = ATM_ALT[bb + 1];
        if (gp < testAlt) { b = bb; break; }
        BaseAlt = testAlt;
        b = bb + 1;
    }
    double Tmb = atm_temperature(atm_geometric(BaseAlt));
    double deltaH = gp - BaseAlt, Lmb = g_lapse[b];
    if (Lmb != 0.0) {
        double Exp = g0 * Mair / (Rstar * Lmb);
        double factor = Tmb / (Tmb + Lmb * deltaH);
        return g_pbrk[b] * pow(factor, Exp);
    }
    return g_pbrk[b] * exp(-g0 * Mair * deltaH / (Rstar * Tmb));
}

static double atm_density_altitude(double density)  /* jsb_atmos.py:78-96 */
{
    int b = 0;
    for (int bb = 0; bb < 9 - 2; bb++) {
        if (density >= g_dbrk[bb + 1]) { b = bb; break; }
        b = bb + 1;
    }
    double Tmb = ATM_TMP[b], Hb = ATM_ALT[b], Lmb = g_lapse[b], pb = g_dbrk[b], da;
    if (Lmb != 0.0) {
        double Exp = -1.0 / (1.0 + (g0 * Mair) / (Rstar * Lmb));
        da = Hb + (Tmb / Lmb) * (pow(density / pb, Exp) - 1);
    } else {
        double Factor = -(Rstar * Tmb) / (g0 * Mair);
        da = Hb + Factor * log(density / pb);
    }
    return atm_geometric(da);
}

typedef struct { double T, P, rho, a, sigma, densalt; } Atmos;

static void atm_calculate(double altitude, Atmos *o)  /* jsb_atmos.py:98-111 */
{
    double Reng = Rstar / Mair;
    double T = atm_temperature(altitude);
    double P = atm_pressure(altitude);
    double rho = P / (Reng * T);
    o->T = T; o->P = P; o->rho = rho;
    o->a = sqrt(SHRatio * Reng * T);
    double rho_sl = StdDaySLpressure / (Reng * StdDaySLtemperature);
    o->sigma = rho / rho_sl;
    o->densalt = atm_density_altitude(rho);
}

/* ------------------------------------------------------------------ mass balance */
typedef struct { double cg[3], mass_slug, J[3][3], Jinv[3][3], RPBody[3]; } Mass;

static void structural_to_body(const double r[3], const double cg[3], double o[3])  /* jsb_massbalance.py:43-46 */
{
    o[0] = INCHTOFT * (cg[0] - r[0]);
    o[1] = INCHTOFT * (r[1] - cg[1]);
    o[2] = INCHTOFT * (cg[2] - r[2]);
}

static void pm_inertia(double mass_sl, const double r[3], const double cg[3], double M[3][3])  /* jsb_massbalance.py:22-36 */
{
    double vx = INCHTOFT * (cg[0] - r[0]), vy = INCHTOFT * (r[1] - cg[1]), vz = INCHTOFT * (cg[2] - r[2]);
    double sx = mass_sl * vx, sy = mass_sl * vy, sz = mass_sl * vz;
    double xx = sx * vx, yy = sy * vy, zz = sz * vz;
    double xy = -sx * vy, xz = -sx * vz, yz = -sy * vz;
    M[0][0] = yy + zz; M[0][1] = xy;      M[0][2] = xz;
    M[1][0] = xy;      M[1][1] = xx + zz; M[1][2] = yz;
    M[2][0] = xz;      M[2][1] = yz;      M[2][2] = xx + yy;
}

static void mb_compute(double fuel, Mass *o)   /* jsb_massbalance.py:49-83 */
{
    const double BASE_CG[3] = {F16M_BASECG_X, F16M_BASECG_Y, F16M_BASECG_Z};
    const double PILOT_LOC[3] = {F16M_PILOT_X, F16M_PILOT_Y, F16M_PILOT_Z};
    const double TANK0[3] = {F16M_TANK0_X, F16M_TANK0_Y, F16M_TANK0_Z};
    const double TANK1[3] = {F16M_TANK1_X, F16M_TANK1_Y, F16M_TANK1_Z};
    const double AERORP[3] = {F16M_AERORP_X, F16M_AERORP_Y, F16M_AERORP_Z};
    const double EMPTY_WT = F16M_EMPTYWT, PILOT_WT = F16M_PILOT_WT;
    double t0 = fuel / 2.0, t1 = t0;
    double tanks_wt = t0 + t1;
    double weight = EMPTY_WT + tanks_wt + PILOT_WT;
    for (int i = 0; i < 3; i++) {
        double me = EMPTY_WT * BASE_CG[i], mp = PILOT_WT * PILOT_LOC[i];
        double m0 = t0 * TANK0[i], m1 = t1 * TANK1[i];
        o->cg[i] = (me + mp + m0 + m1) / weight;
    }
    double mJ[3][3] = {{F16M_IXX, -F16M_IXY, F16M_IXZ},
                       {-F16M_IXY, F16M_IYY, -F16M_IYZ},
                       {F16M_IXZ, -F16M_IYZ, F16M_IZZ}};
    double tmp[3][3];
    const double masses[4] = {LBTOSLUG * EMPTY_WT, LBTOSLUG * PILOT_WT, LBTOSLUG * t0, LBTOSLUG * t1};
    const double *locs[4] = {BASE_CG, PILOT_LOC, TANK0, TANK1};
    for (int k = 0; k < 4; k++) {
        pm_inertia(masses[k], locs[k], o->cg, tmp);
        for (int i = 0; i < 3; i++)
            for (int j = 0; j < 3; j++) mJ[i][j] = mJ[i][j] + tmp[i][j];
    }
    double Ixx = mJ[0][0], Iyy = mJ[1][1], Izz = mJ[2][2];
    double Ixy = -mJ[0][1], Ixz = -mJ[0][2], Iyz = -mJ[1][2];
    double k1 = (Iyy * Izz - Iyz * Iyz);
    double k2 = (Iyz * Ixz + Ixy * Izz);
    double k3 = (Ixy * Iyz + Iyy * Ixz);
    double denom = 1.0 / (Ixx * k1 - Ixy * k2 - Ixz * k3);
    k1 *= denom; k2 *= denom; k3 *= denom;
    double k4 = (Izz * Ixx - Ixz * Ixz) * denom;
    double k5 = (Ixy * Ixz + Iyz * Ixx) * denom;
    double k6 = (Ixx * Iyy - Ixy * Ixy) * denom;
    double Jinv[3][3] = {{k1, k2, k3}, {k2, k4, k5}, {k3, k5, k6}};
    double J[3][3] = {{Ixx, -Ixy, -Ixz}, {-Ixy, Iyy, -Iyz}, {-Ixz, -Iyz, Izz}};
    memcpy(o->Jinv, Jinv, sizeof Jinv);
    memcpy(o->J, J, sizeof J);
    structural_to_body(AERORP, o->cg, o->RPBody);
    o->mass_slug = LBTOSLUG * weight;
}

/* exported for the mass-balance unit tests: out = cg[3], mass, J[9], Jinv[9], RPBody[3] */
void orc_mass(double fuel, double *out)
{
    orc_init();
    Mass m;
    mb_compute(fuel, &m);
    memcpy(out, m.cg, 3 * sizeof(double));
    out[3] = m.mass_slug;
    memcpy(out + 4, m.J, 9 * sizeof(double));
    memcpy(out + 13, m.Jinv, 9 * sizeof(double));
    memcpy(out + 22, m.RPBody, 3 * sizeof(double));
}

/* exported for the atmosphere unit tests: out = T, P, rho, a, sigma, densalt */
void orc_atmos(double alt_ft, double *out)
{
    orc_init();
    Atmos a;
    atm_calculate(alt_ft, &a);
    out[0] = a.T; out[1] = a.P; out[2] = a.rho; out[3] = a.a; out[4] = a.sigma; out[5] = a.densalt;
}

/* ------------------------------------------------------------------ FCS (jsb_fcs.py) */
static double clip(double x, double lo, double hi) { return x < lo ? lo : (x > hi ? hi : x); }  /* :24-25 */

static int equal_roundoff(double a, double b)   /* jsb_fcs.py:28-30; Python max(1.0,|a|,|b|) */
{
    double m = 1.0, fa = fabs(a), fb = fabs(b);
    if (fa > m) m = fa;
    if (fb > m) m = fb;
    return fabs(a - b) <= 1e-9 * m;
}

/* Kinemat.run (jsb_fcs.py:42-78); doscale is true for every F-16 kinematic */
static double kinemat_run(const double *det, const double *tim, int n, double *output,
                          double inp, int has_seed, double seed, double fcs_dt)
{
    double dt0 = fcs_dt;
    double Input = inp;
    Input *= det[n - 1];
    double Output = has_seed ? seed : *output;
    Input = clip(Input, det[0], det[n - 1]);
    while (dt0 > 0.0 && !equal_roundoff(Input, Output)) {
        int ind = 1;
        for (;;) {
            int cond = (Input < Output) ? (det[ind] < Output) : (det[ind] <= Output);
            if (!cond) break;
            ind += 1;
            if (ind >= n) break;
        }
        if (ind >= n) ind = n - 1;
        if (tim[ind] <= 0.0) { Output = Input; break; }
        double Rate = (det[ind] - det[ind - 1]) / tim[ind];
        double ThisInput = clip(Input, det[ind - 1], det[ind]);
        double ThisDt = fabs((ThisInput - Output) / Rate);
        if (dt0 < ThisDt) {
            ThisDt = dt0;
            if (Output < Input) Output += ThisDt * Rate;
            else Output -= ThisDt * Rate;
        } else {
            Output = ThisInput;
        }
        dt0 -= ThisDt;
    }
    *output = Output;
    return Output;
}

/* PID.run (jsb_fcs.py:90-104). pid[0]=input_prev, pid[1]=input_prev2, pid[2]=i_out_total */
static double pid_run(double kp, double ki, double kd, double *pid, double Input, double trigger,
                      int has_clip, double lo, double hi, double fcs_dt)
{
    double Dval = (Input - pid[0]) / fcs_dt;
    double test = trigger, I_out_delta = 0.0;
    if (fabs(test) < 0.000001) I_out_delta = 1.5 * Input - 0.5 * pid[0];
    if (test < 0.0) pid[2] = 0.0;
    pid[2] += ki * fcs_dt * I_out_delta;
    double Output = kp * Input + pid[2] + kd * Dval;
    pid[1] = (test < 0.0) ? 0.0 : pid[0];
    pid[0] = Input;
    if (has_clip) Output = clip(Output, lo, hi);
    return Output;
}

static double aerosurface_zc(double Input, double InMin, double InMax, double OutMin, double OutMax)
{   /* jsb_fcs.py:107-113 */
    if (Input == 0.0) return 0.0;
    if (Input > 0.0) return (Input / InMax) * OutMax;
    return (Input / InMin) * OutMin;
}

typedef struct { double ail, elev, rud, lef, flap, sb, gear; } FcsOut;

/* FCS state: 15 doubles = kinematic outputs (tef, aileron, elevator, rudder, gear, lef)
 * followed by the roll, g-load and yaw PIDs (input_prev, input_prev2, i_out_total). */
#define S_KIN 86

/* F16FCS.step (jsb_fcs.py:143-268) */
static void fcs_step(double *fcs15, double c_ail, double c_ele, double c_rud, double alpha, double mach,
                     double vc, double vg, double n_pilot_y, double n_pilot_z, double p_aero,
                     double q_aero, double r_aero, double pitch_rad, double roll_rad, double fcs_dt,
                     FcsOut *out)
{
    static const double d_tef[3] = {-1.0, 0.0, 1.0}, t_tef[3] = {3.0, 0.0, 3.0};
    static const double d_ail[2] = {-1.0, 1.0}, t_ail[2] = {0.3, 0.3};
    static const double d_ele[2] = {-1.0, 1.0}, t_ele[2] = {0.3, 0.3};
    static const double d_rud[2] = {-1.0, 1.0}, t_rud[2] = {0.4, 0.4};
    static const double d_gear[2] = {0.0, 1.0}, t_gear[2] = {0.0, 5.0};
    static const double d_lef[2] = {-1.0, 1.0}, t_lef[2] = {3.0, 3.0};
    const double c_pitch_trim = 0.0, c_yaw_trim = 0.0, c_gear = 0.0, gear_force = 0.30;
    double *kin = fcs15, *pid = fcs15 + 6;

    /* Flaps */
    double tef_pos_rad = (vc < 250) ? 0.349 : ((mach > 0.9) ? -0.0349 : 0.0);
    double tef_pos_norm = 2.864789 * tef_pos_rad;
    double tef_control = kinemat_run(d_tef, t_tef, 3, &kin[0], tef_pos_norm, 0, 0.0, fcs_dt);

    /* Roll */
    double roll_rate_norm = 0.31821 * p_aero;
    double roll_trim_error = c_ail - roll_rate_norm;
    double ail_trig = (vc < 20.0) ? 0.0 : 1.0;
    double roll_rate_pid = pid_run(3.00000, 0.00050, -0.00125, pid + 0, roll_trim_error, ail_trig, 0, 0, 0, fcs_dt);
    double roll_rate_command = clip(roll_rate_pid + c_ail, -1.0, 1.0);
    double aileron_pos_rad = aerosurface_zc(roll_rate_command, -1.0, 1.0, -0.375, 0.375);
    double left_aileron_pos_norm = kinemat_run(d_ail, t_ail, 2, &kin[1], roll_rate_command, 0, 0.0, fcs_dt);
    double aileron_speed_comp = T1(FCS_AIL_SPEED, mach) * left_aileron_pos_norm;
    double left_flaperon_norm = clip(-tef_control - aileron_speed_comp, -1.0, 1.0);
    double right_flaperon_norm = clip(tef_control - aileron_speed_comp, -1.0, 1.0);
    double flaperon_summer = left_flaperon_norm + right_flaperon_norm;
    double flaperon_mix_rad = 1.4324 * flaperon_summer;
    double left_aileron_pos_rad = aerosurface_zc(aileron_speed_comp, -1.0, 1.0, -0.375, 0.375);
    double right_aileron_pos_rad = aerosurface_zc(-aileron_speed_comp, -1.0, 1.0, -0.375, 0.375);
    (void)left_aileron_pos_rad; (void)right_aileron_pos_rad;   /* diagnostics only (dht_*) */

    /* Pitch */
    double n_pilot_z_corr = cos(pitch_rad) * cos(roll_rad);
    double g_load_corrected = n_pilot_z - n_pilot_z_corr;
    double elevator_cmd_limiter = clip(c_ele + c_pitch_trim, -1.0, 0.44);
    double elevator_scheduler = T1(FCS_ELEV_SCHED, alpha) * elevator_cmd_limiter;
    double alpha_limiter_norm = 1.0472 * alpha;
    double pitch_rate_norm = 6.2 * q_aero;
    double g_load_norm = 0.020 * g_load_corrected;
    double pitch_trim_error = elevator_scheduler + pitch_rate_norm - g_load_norm;
    double elev_trig = (vc < 5.0) ? 0.0 : 1.0;
    double g_load_pid = pid_run(0.3000, 0.0250, 0.0000, pid + 3, pitch_trim_error, elev_trig, 1, -1.0, 1.0, fcs_dt);
    double pitch_scheduler = clip(elevator_scheduler + alpha_limiter_norm + g_load_pid, -1.0, 1.0);
    double elevator_pos_norm = kinemat_run(d_ele, t_ele, 2, &kin[2], pitch_scheduler, 0, 0.0, fcs_dt);
    double elevator_pos_rad = aerosurface_zc(elevator_pos_norm, -1.0, 1.0, -0.436, 0.436);

    /* Yaw */
    double yaw_rate_norm = T1(FCS_YAW_RATE, vg) * r_aero;
    double yaw_load_norm = 0.25 * n_pilot_y;
    double yaw_trim_error = c_rud + yaw_rate_norm + yaw_load_norm;
    double rud_trig = (vc < 10.0) ? 0.0 : 1.0;
    double yaw_load_pid = pid_run(0.105500, 0.000010, 0.00005, pid + 6, yaw_trim_error, rud_trig, 1, -1.0, 1.0, fcs_dt);
    double yaw_scheduler = clip(c_rud + c_yaw_trim + yaw_load_pid, -1.0, 1.0);
    double rudder_pos_norm = kinemat_run(d_rud, t_rud, 2, &kin[3], yaw_scheduler, 1, yaw_load_pid, fcs_dt);
    double rudder_pos_rad = aerosurface_zc(rudder_pos_norm, -1.0, 1.0, -0.524, 0.524);

    /* Landing gear: position forced externally, kinematic seeded by it */
    double gear_wow = 0.0;
    double gear_pos_norm = kinemat_run(d_gear, t_gear, 2, &kin[4], c_gear, 1, gear_force, fcs_dt);

    /* LEF */
    double lef_pos_rad;
    if (gear_wow == 1 && gear_pos_norm > 0) lef_pos_rad = -0.0349;
    else if (gear_pos_norm == 0 && alpha > 0.2618) lef_pos_rad = 0.436;
    else if (gear_wow == 0 && alpha > 0.0873) lef_pos_rad = 0.262;
    else if (mach > 0.9) lef_pos_rad = -0.0349;
    else lef_pos_rad = 0.0;
    double lef_pos_norm = 2.293578 * lef_pos_rad;
    kinemat_run(d_lef, t_lef, 2, &kin[5], lef_pos_norm, 0, 0.0, fcs_dt);

    out->ail = aileron_pos_rad; out->elev = elevator_pos_rad; out->rud = rudder_pos_rad;
    out->lef = lef_pos_rad; out->flap = flaperon_mix_rad; out->sb = 0.0; out->gear = gear_pos_norm;
}

/* ------------------------------------------------------------------ engine (jsb_propulsion.py) */
#define S_ENG 82   /* N1, N2, N2norm, FuelFlow_pph */

static double seek(double v, double target, double accel, double decel, double dt)  /* :63-72 */
{
    if (v > target) { v -= dt * decel; if (v < target) v = target; }
    else if (v < target) { v += dt * accel; if (v > target) v = target; }
    return v;
}

static double spool_val(double delay, double densratio, double N2norm)  /* :85-87 */
{
    double x = N2norm + 0.1;
    double n = (x < 1.0) ? x : 1.0;        /* Python min(1.0, x) */
    return delay / (1 + 3 * pow(1 - n, 3) + (1 - densratio));
}

typedef struct { double thrust, fuel_burn, forces[3], moments[3]; } EngOut;

static void eng_step(double *eng, double throttle_pos_norm, double mach, double densalt, double T,
                     double densratio, double dt, const double cg[3], EngOut *o)   /* :89-128 */
{
    const double MILTHRUST = F16M_ENG_MILTHRUST, MAXTHRUST = F16M_ENG_MAXTHRUST;
    const double IDLEN1 = F16M_ENG_IDLEN1, IDLEN2 = F16M_ENG_IDLEN2;
    const double MAXN1 = F16M_ENG_MAXN1, MAXN2 = F16M_ENG_MAXN2;
    double ThrottlePos = throttle_pos_norm, AugmentCmd;
    if (ThrottlePos > 1.0) { AugmentCmd = ThrottlePos - 1.0; ThrottlePos -= AugmentCmd; }
    else AugmentCmd = 0.0;
    double N1_factor = MAXN1 - IDLEN1, N2_factor = MAXN2 - IDLEN2, d = F16M_ENG_BYPASSRATIO;
    double N2norm0 = eng[2];
    double n2up = spool_val(1.0 * 90.0 / (d + 3.0), densratio, N2norm0);
    double n2dn = spool_val(3.0 * 90.0 / (d + 3.0), densratio, N2norm0);
    double n1up = spool_val(1.0 * 90.0 / (d + 3.0), densratio, N2norm0);
    double n1dn = spool_val(2.4 * 90.0 / (d + 3.0), densratio, N2norm0);
    eng[1] = seek(eng[1], IDLEN2 + ThrottlePos * N2_factor, n2up, n2dn, dt);
    eng[0] = seek(eng[0], IDLEN1 + ThrottlePos * N1_factor, n1up, n1dn, dt);
    eng[2] = (eng[1] - IDLEN2) / N2_factor;
    double N2norm = eng[2];
    double idlethrust = MILTHRUST * T2(ENG_IDLE, mach, densalt);
    double milthrust = (MILTHRUST - idlethrust) * T2(ENG_MIL, mach, densalt);
    double thrust = idlethrust + milthrust * N2norm * N2norm;
    double correctedTSFC = F16M_ENG_TSFC * sqrt(T / 389.7) * (0.84 + pow(1 - N2norm, 2));
    eng[3] = seek(eng[3], thrust * correctedTSFC, 1000.0, 10000.0, dt);
    if (eng[3] < g_idleff) eng[3] = g_idleff;
    thrust = thrust * (1.0 - 0.0);            /* BLEEDDEMAND = 0 */
    if (AugmentCmd > 0.0) {                   /* AUGMETHOD == 2 */
        double tdiff = (MAXTHRUST * T2(ENG_AUG, mach, densalt)) - thrust;
        thrust += tdiff * AugmentCmd;
        eng[3] = seek(eng[3], thrust * F16M_ENG_ATSFC, 5000.0, 10000.0, dt);
    }
    double rz = INCHTOFT * (cg[2] - 0.0), ry = INCHTOFT * (0.0 - cg[1]);
    o->thrust = thrust;
    o->forces[0] = thrust; o->forces[1] = 0.0; o->forces[2] = 0.0;
    o->moments[0] = 0.0; o->moments[1] = rz * thrust; o->moments[2] = -ry * thrust;
    o->fuel_burn = eng[3] / 3600.0 * dt;
}

/* ------------------------------------------------------------------ auxiliary (jsb_auxiliary.py) */
static double pitot_total_pressure(double mach, double p)   /* :20-26 */
{
    if (mach < 0) return p;
    if (mach < 1) return p * pow(1 + 0.2 * mach * mach, 3.5);
    return p * 166.92158009316827 * pow(mach, 7.0) / pow(7 * mach * mach - 1, 2.5);
}

static double mach_from_impact_pressure(double qc, double p)   /* :29-36 */
{
    double A = qc / p + 1;
    double M = sqrt(5.0 * (pow(A, 1. / 3.5) - 1));
    if (M > 1.0)
        for (int i = 0; i < 10; i++)
            M = 0.8812848543473311 * sqrt(A * pow(1 - 1.0 / (7.0 * M * M), 2.5));
    return M;
}

static double vcalibrated_from_mach(double mach, double p)   /* :39-42 */
{
    double qc = pitot_total_pressure(mach, p) - p;
    return g_std_sl_soundspeed * mach_from_impact_pressure(qc, StdDaySLpressure);
}

typedef struct { double alpha, beta, Vt, qbar, mach, p, q, r, vg, npy, npz, vc_kts; } Aux;

static void auxiliary(const double vUVW[3], const double vPQR[3], const double vned[3], double rho,
                      double a, double P, const double cg[3], const double pba[3],
                      const double ppqridot[3], const double ppqri[3], Aux *o)   /* :45-73 */
{
    const double EYE[3] = {F16M_EYEPOINT_X, F16M_EYEPOINT_Y, F16M_EYEPOINT_Z};
    double u = vUVW[0], v = vUVW[1], w = vUVW[2];
    double AeroU2 = u * u, AeroV2 = v * v, AeroW2 = w * w;
    double mUW = AeroU2 + AeroW2;
    double Vt2 = mUW + AeroV2;
    double Vt = sqrt(Vt2);
    double alpha = 0.0, beta = 0.0;
    if (Vt > 0.001) {
        beta = atan2(v, sqrt(mUW));
        if (mUW >= 1e-6) alpha = atan2(w, u);
    }
    o->alpha = alpha; o->beta = beta; o->Vt = Vt;
    o->qbar = 0.5 * rho * Vt2;
    o->mach = Vt / a;
    o->vg = sqrt(vned[0] * vned[0] + vned[1] * vned[1]);
    double eye[3], c1[3], c2[3], c3[3], acc[3];
    structural_to_body(EYE, cg, eye);
    cross(ppqridot, eye, c1);
    for (int i = 0; i < 3; i++) acc[i] = pba[i] + c1[i];
    cross(ppqri, eye, c2);
    cross(ppqri, c2, c3);
    for (int i = 0; i < 3; i++) acc[i] = acc[i] + c3[i];
    o->npy = acc[1] / g_slgravity;
    o->npz = acc[2] / g_slgravity;
    double vcas = (fabs(o->mach) > 0.0) ? vcalibrated_from_mach(o->mach, P) : 0.0;
    o->vc_kts = vcas * FPSTOKTS;
    o->p = vPQR[0]; o->q = vPQR[1]; o->r = vPQR[2];
}

/* ------------------------------------------------------------------ aerodynamics (jsb_aero.py) */
static double aero_table(const f16m_aero_term *t, const double *ctx)
{
    const double *I = F16M_IMAGE;
    if (t->kind == 1) return table1d(I + t->rg, I + t->off, t->nr, ctx[t->row_var]);
    return table2d(I + t->rg, t->nr, I + t->cg, t->nc, I + t->off, ctx[t->row_var], ctx[t->col_var]);
}

/* F16Aero.compute (jsb_aero.py:75-107) -> body forces and moments */
static void aero_compute(const Aux *ax, const FcsOut *f, const double RPBody[3], double F[3], double M[3])
{
    double Vt = ax->Vt, twovel = 2.0 * Vt;
    double ctx[F16M_NVAR];
    ctx[F16M_V_QBAR] = ax->qbar; ctx[F16M_V_SW] = F16M_SW; ctx[F16M_V_BW] = F16M_BW;
    ctx[F16M_V_CBAR] = F16M_CBAR;
    ctx[F16M_V_ALPHA] = ax->alpha; ctx[F16M_V_BETA] = ax->beta;
    ctx[F16M_V_BI2VEL] = (twovel != 0) ? F16M_BW / twovel : 0.0;
    ctx[F16M_V_CI2VEL] = (twovel != 0) ? F16M_CBAR / twovel : 0.0;
    ctx[F16M_V_MACH] = ax->mach;
    ctx[F16M_V_KCLGE] = T1(KCLGE, 765.0);         /* aero/h_b-mac-ft (jsb_fdm.py:86) */
    ctx[F16M_V_P] = ax->p; ctx[F16M_V_Q] = ax->q; ctx[F16M_V_R] = ax->r;
    ctx[F16M_V_AIL] = f->ail; ctx[F16M_V_ELEV] = f->elev; ctx[F16M_V_RUD] = f->rud;
    ctx[F16M_V_LEF] = f->lef; ctx[F16M_V_FLAP] = f->flap; ctx[F16M_V_SB] = f->sb;
    ctx[F16M_V_GEAR] = f->gear;
    double sum[6] = {0, 0, 0, 0, 0, 0};
    for (int i = 0; i < F16M_NAERO; i++) {      /* _eval_func, jsb_aero.py:62-73 */
        const f16m_aero_term *t = &AERO_TERMS[i];
        double v = 1.0;
        for (int k = 0; k < t->nfac; k++) v *= ctx[t->fac[k]];
        if (t->has_value) v *= t->value;
        if (t->kind) v *= aero_table(t, ctx);
        sum[t->axis] += v;
    }
    double drag = -sum[F16M_AX_DRAG], side = sum[F16M_AX_SIDE], lift = -sum[F16M_AX_LIFT];
    double a = ax->alpha, b = ax->beta;
    double ca = cos(a), sa = sin(a), cb = cos(b), sb = sin(b);
    double Fx = ca * cb * drag + (-ca * sb) * side + (-sa) * lift;
    double Fy = sb * drag + cb * side + 0.0 * lift;
    double Fz = sa * cb * drag + (-sa * sb) * side + ca * lift;
    double rx = RPBody[0], ry = RPBody[1], rz = RPBody[2];
    F[0] = Fx; F[1] = Fy; F[2] = Fz;
    M[0] = sum[F16M_AX_ROLL] + (ry * Fz - rz * Fy);
    M[1] = sum[F16M_AX_PITCH] + (rz * Fx - rx * Fz);
    M[2] = sum[F16M_AX_YAW] + (rx * Fy - ry * Fx);
}

/* ------------------------------------------------------------------ accelerations (jsb_accel.py) */
typedef struct { double vUVWidot[3], vPQRidot[3], vBodyAccel[3], vPQRi[3]; } Accel;

static void accelerations(const double force[3], const double moment[3], double mass,
                          const double J[3][3], const double Jinv[3][3], const double vUVW[3],
                          const double vPQR[3], const double Ti2b[3][3], const double vGrav[3],
                          Accel *o)   /* :10-31 (vUVWdot/vPQRdot are not consumed and omitted) */
{
    (void)vUVW;
    double Tb2i[3][3], Tw[3], JvPQRi[3], cr[3], mm[3], tmp[3];
    transpose(Ti2b, Tb2i);
    matvec(Ti2b, OMEGA, Tw);
    for (int i = 0; i < 3; i++) o->vPQRi[i] = vPQR[i] + Tw[i];
    matvec(J, o->vPQRi, JvPQRi);
    cross(o->vPQRi, JvPQRi, cr);
    for (int i = 0; i < 3; i++) mm[i] = moment[i] - cr[i];
    matvec(Jinv, mm, o->vPQRidot);
    double s = 1.0 / mass;
    for (int i = 0; i < 3; i++) o->vBodyAccel[i] = force[i] * s;
    matvec(Tb2i, o->vBodyAccel, tmp);
    for (int i = 0; i < 3; i++) o->vUVWidot[i] = tmp[i] + vGrav[i];
}

/* ------------------------------------------------------------------ state layout */
/* FdmState order (cuda_fdm/ic.py:92-114) */
#define S_POS 0
#define S_VEL 3
#define S_Q 6
#define S_PQRI 10
#define S_EPA 13
#define S_FUEL 14
#define S_UVWIDOT 15
#define S_PQRIDOT 18
#define S_QDOT 21
#define S_DQ 25      /* 3 x 4 */
#define S_DPQRI 37   /* 3 x 3 */
#define S_DIVEL 46   /* 3 x 3 */
#define S_DUVW 55    /* 3 x 3 */
#define S_PBA 64
#define S_PPQRIDOT 67
#define S_PPQRI 70
#define S_PAUX 73    /* alpha, mach, vc, vg, npy, npz, p, q, r */

typedef struct {
    double vUVW[3], vPQR[3], vned[3], ecef[3], Ti2b[3][3], Tec2i[3][3], Tl2ec[3][3];
    double radius, mLat, euler[3];
} Kin;

/* FDM._kinematics_from_state (jsb_fdm.py:121-140) */
static void kinematics(const double *st, Kin *k)
{
    double Ti2ec[3][3], Tl2i[3][3], Tb2i[3][3], Tl2b[3][3], Tb2l[3][3], cr[3], d[3], Tw[3];
    Ti2ec_from_epa(st[S_EPA], Ti2ec);
    transpose(Ti2ec, k->Tec2i);
    matvec(Ti2ec, st + S_POS, k->ecef);
    location_derived(k->ecef, &k->radius, &k->mLat, k->Tl2ec);
    matmul(k->Tec2i, k->Tl2ec, Tl2i);
    quat_to_T(st + S_Q, k->Ti2b);
    transpose(k->Ti2b, Tb2i);
    matmul(k->Ti2b, Tl2i, Tl2b);
    transpose(Tl2b, Tb2l);
    cross(OMEGA, st + S_POS, cr);
    for (int i = 0; i < 3; i++) d[i] = st[S_VEL + i] - cr[i];
    matvec(k->Ti2b, d, k->vUVW);
    matvec(k->Ti2b, OMEGA, Tw);
    for (int i = 0; i < 3; i++) k->vPQR[i] = st[S_PQRI + i] - Tw[i];
    matvec(Tb2l, k->vUVW, k->vned);
    mat_to_euler(Tl2b, k->euler);
}

typedef struct { Accel acc; Aux aux; EngOut eng; double alt_asl; } ForceOut;

/* FDM._force_path (jsb_fdm.py:76-119).  `st` carries prev-aux / prev-accel, the FCS and the
 * engine state (updated in place); `fcs_st`/`eng_st` let the seed run throwaway copies. */
static void force_path(const double *st, double *fcs_st, double *eng_st, double fuel,
                       double c_ail, double c_ele, double c_rud, double c_thr,
                       const double *pba, const double *ppqridot, const double *ppqri,
                       const Kin *k, double fcs_dt, ForceOut *o)
{
    const double *pa = st + S_PAUX;
    double alt_asl = k->radius - SEA_LEVEL_RADIUS_;
    Atmos at;
    Mass mb;
    FcsOut fo;
    atm_calculate(alt_asl, &at);
    mb_compute(fuel, &mb);
    fcs_step(fcs_st, c_ail, c_ele, c_rud, pa[0], pa[1], pa[2], pa[3], pa[4], pa[5], pa[6], pa[7],
             pa[8], k->euler[1], k->euler[0], fcs_dt, &fo);
    auxiliary(k->vUVW, k->vPQR, k->vned, at.rho, at.a, at.P, mb.cg, pba, ppqridot, ppqri, &o->aux);
    double thr_pos = 2.0 * c_thr;
    eng_step(eng_st, thr_pos, o->aux.mach, at.densalt, at.T, at.sigma, DT, mb.cg, &o->eng);
    double Fa[3], Ma[3], force[3], moment[3], grav[3], vGrav[3];
    aero_compute(&o->aux, &fo, mb.RPBody, Fa, Ma);
    for (int i = 0; i < 3; i++) {
        force[i] = Fa[i] + o->eng.forces[i];
        moment[i] = Ma[i] + o->eng.moments[i];
    }
    gravity_j2(k->ecef, k->mLat, grav);
    matvec(k->Tec2i, grav, vGrav);
    accelerations(force, moment, mb.mass_slug, mb.J, mb.Jinv, k->vUVW, k->vPQR, k->Ti2b, vGrav, &o->acc);
    o->alt_asl = alt_asl;
}

/* FDM.step (jsb_fdm.py:212-244).  obs17 (may be NULL): eci_pos, eci_vel, euler, vUVW,
 * alpha, beta, mach, Vt, alt_asl -- the fdm_step_batch output row (fdm_kernel.cu:41-46). */
static void fdm_step(double *st, double c_ail, double c_ele, double c_rud, double c_thr,
                     double fcs_dt, double *obs17)
{
    int i;
    /* quaternion: rect-Euler + normalize (_integ_quat_rect, :38-43) */
    memmove(st + S_DQ + 4, st + S_DQ, 8 * sizeof(double));
    memcpy(st + S_DQ, st + S_QDOT, 4 * sizeof(double));
    for (i = 0; i < 4; i++) st[S_Q + i] = st[S_Q + i] + DT * st[S_DQ + i];
    quat_normalize(st + S_Q);
    /* vPQRi: rect-Euler (_integ_rect, :23-26) */
    memmove(st + S_DPQRI + 3, st + S_DPQRI, 6 * sizeof(double));
    memcpy(st + S_DPQRI, st + S_PQRIDOT, 3 * sizeof(double));
    for (i = 0; i < 3; i++) st[S_PQRI + i] = st[S_PQRI + i] + DT * st[S_DPQRI + i];
    /* ECI position: AB3 on the velocity history (_integ_ab3, :33-36) */
    memmove(st + S_DIVEL + 3, st + S_DIVEL, 6 * sizeof(double));
    memcpy(st + S_DIVEL, st + S_VEL, 3 * sizeof(double));
    for (i = 0; i < 3; i++)
        st[S_POS + i] = st[S_POS + i] + (DT / 12.0) * (23.0 * st[S_DIVEL + i] - 16.0 * st[S_DIVEL + 3 + i]
                                                       + 5.0 * st[S_DIVEL + 6 + i]);
    /* ECI velocity: AB2 (_integ_ab2, :28-31) */
    memmove(st + S_DUVW + 3, st + S_DUVW, 6 * sizeof(double));
    memcpy(st + S_DUVW, st + S_UVWIDOT, 3 * sizeof(double));
    for (i = 0; i < 3; i++)
        st[S_VEL + i] = st[S_VEL + i] + DT * (1.5 * st[S_DUVW + i] - 0.5 * st[S_DUVW + 3 + i]);
    st[S_EPA] += ROTATION_RATE * DT;

    Kin k;
    kinematics(st, &k);
    quat_qdot(st + S_Q, st + S_PQRI, st + S_QDOT);

    ForceOut fo;
    double pba[3], ppd[3], ppq[3];
    memcpy(pba, st + S_PBA, sizeof pba);
    memcpy(ppd, st + S_PPQRIDOT, sizeof ppd);
    memcpy(ppq, st + S_PPQRI, sizeof ppq);
    force_path(st, st + S_KIN, st + S_ENG, st[S_FUEL], c_ail, c_ele, c_rud, c_thr, pba, ppd, ppq,
               &k, fcs_dt, &fo);
    st[S_FUEL] -= fo.eng.fuel_burn;
    for (i = 0; i < 3; i++) {
        st[S_UVWIDOT + i] = fo.acc.vUVWidot[i];
        st[S_PQRIDOT + i] = fo.acc.vPQRidot[i];
        st[S_PBA + i] = fo.acc.vBodyAccel[i];
        st[S_PPQRIDOT + i] = fo.acc.vPQRidot[i];
        st[S_PPQRI + i] = fo.acc.vPQRi[i];
    }
    double *pa = st + S_PAUX;
    pa[0] = fo.aux.alpha; pa[1] = fo.aux.mach; pa[2] = fo.aux.vc_kts; pa[3] = fo.aux.vg;
    pa[4] = fo.aux.npy; pa[5] = fo.aux.npz; pa[6] = fo.aux.p; pa[7] = fo.aux.q; pa[8] = fo.aux.r;
    if (obs17) {
        for (i = 0; i < 3; i++) {
            obs17[i] = st[S_POS + i];
            obs17[3 + i] = st[S_VEL + i];
            obs17[6 + i] = k.euler[i];
            obs17[9 + i] = k.vUVW[i];
        }
        obs17[12] = fo.aux.alpha; obs17[13] = fo.aux.beta; obs17[14] = fo.aux.mach;
        obs17[15] = fo.aux.Vt; obs17[16] = fo.alt_asl;
    }
}

/* ------------------------------------------------------------------ public entry points */
/* fcs_rate: components' dt is 1/fcs_rate s (120 for cuda_fdm/ref/jsb_fcs.py:19, 60 for the
 * 184-D lineage research/competition_36500/runtime/cuda_fdm/ref/jsb_fcs.py:19). */
static double fcs_dt_of(int fcs_rate) { return 1.0 / (double)fcs_rate; }

/* One aircraft, `substeps` steps with the action held (fdm_step_batch semantics). */
void orc_fdm_step1(double *st101, const double *act4, int substeps, int fcs_rate, double *obs17)
{
    orc_init();
    double dt = fcs_dt_of(fcs_rate);
    for (int s = 0; s < substeps; s++) fdm_step(st101, act4[0], act4[1], act4[2], act4[3], dt, obs17);
}

/* Batch over aircraft (AoS rows of 101 doubles), OpenMP across aircraft. */
void orc_fdm_step_batch(double *states, const double *actions, long nac, int substeps, int fcs_rate,
                        double *obs17, int nthreads)
{
    orc_init();
    double dt = fcs_dt_of(fcs_rate);
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static)
#endif
    for (long a = 0; a < nac; a++) {
        double *st = states + a * 101;
        const double *ac = actions + a * 4;
        for (int s = 0; s < substeps; s++)
            fdm_step(st, ac[0], ac[1], ac[2], ac[3], dt, obs17 ? obs17 + a * 17 : NULL);
    }
    (void)nthreads;
}

/* Trajectory driver: `ndec` decisions of `substeps` steps each; actions (ndec, nac, 4). */
void orc_fdm_rollout(double *states, const double *actions, long nac, int ndec, int substeps,
                     int fcs_rate, int nthreads)
{
    orc_init();
    double dt = fcs_dt_of(fcs_rate);
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static)
#endif
    for (long a = 0; a < nac; a++) {
        double *st = states + a * 101;
        for (int d = 0; d < ndec; d++) {
            const double *ac = actions + ((long)d * nac + a) * 4;
            for (int s = 0; s < substeps; s++) fdm_step(st, ac[0], ac[1], ac[2], ac[3], dt, NULL);
        }
    }
    (void)nthreads;
}

int orc_num_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------ IC seeding (cuda_fdm/ic.py) */
/* geodetic_to_ecef (ic.py:18-45) */
static void geodetic_to_ecef(double lat_gd, double lon, double alt_asl, double o[3])
{
    double a = SEMI_MAJOR, e2 = g_e2;
    double sphi = sin(lat_gd), cphi = cos(lat_gd), slam = sin(lon), clam = cos(lon);
    double N = a / sqrt(1.0 - e2 * sphi * sphi);
    double A = cphi * cphi, B = sphi * sphi, P = N, Q = N * (1.0 - e2);
    double b = A * P + B * Q;
    double cst = A * P * P + B * Q * Q;
    double R = a + alt_asl;
    double t = -b + sqrt(b * b - cst + R * R);
    o[0] = (N + t) * cphi * clam;
    o[1] = (N + t) * cphi * slam;
    o[2] = (N * (1.0 - e2) + t) * sphi;
}

/* FDM.seed without golden derivatives (jsb_fdm.py:142-210, ic_uvwdot=None branch). */
static void fdm_seed(double *st, const double eci_pos[3], const double eci_vel[3],
                     const double euler[3], const double vPQR[3], double epa, double fuel,
                     double fuelflow_pph, const double prev_aux[9], double fcs_dt)
{
    memset(st, 0, 101 * sizeof(double));
    memcpy(st + S_POS, eci_pos, 3 * sizeof(double));
    memcpy(st + S_VEL, eci_vel, 3 * sizeof(double));
    st[S_EPA] = epa;
    st[S_FUEL] = fuel;
    memcpy(st + S_PAUX, prev_aux, 9 * sizeof(double));
    double Ti2ec[3][3], Tec2i[3][3], ecef[3], Tl2ec[3][3], Tl2i[3][3], Ti2l[3][3], qL[4];
    double Tl2b[3][3], Ti2b[3][3], radius, mlat, Tw[3];
    Ti2ec_from_epa(epa, Ti2ec);
    transpose(Ti2ec, Tec2i);
    matvec(Ti2ec, st + S_POS, ecef);
    location_derived(ecef, &radius, &mlat, Tl2ec);
    matmul(Tec2i, Tl2ec, Tl2i);
    transpose(Tl2i, Ti2l);
    euler_to_quat(euler[0], euler[1], euler[2], qL);
    quat_to_T(qL, Tl2b);
    matmul(Tl2b, Ti2l, Ti2b);
    mat_to_quat(Ti2b, st + S_Q);
    matvec(Ti2b, OMEGA, Tw);
    for (int i = 0; i < 3; i++) st[S_PQRI + i] = vPQR[i] + Tw[i];
    /* throwaway FCS and engine for one force path at throttle 0.8 */
    Kin k;
    kinematics(st, &k);
    double tmp_fcs[15] = {0};
    double tmp_eng[4] = {100.0, 100.0, (100.0 - F16M_ENG_IDLEN2) / (F16M_ENG_MAXN2 - F16M_ENG_IDLEN2),
                         fuelflow_pph};
    const double z3[3] = {0.0, 0.0, 0.0};
    double pqri[3];
    memcpy(pqri, st + S_PQRI, sizeof pqri);
    ForceOut fo;
    force_path(st, tmp_fcs, tmp_eng, fuel, 0.0, 0.0, 0.0, 0.8, z3, z3, pqri, &k, fcs_dt, &fo);
    memcpy(st + S_UVWIDOT, fo.acc.vUVWidot, 3 * sizeof(double));
    memcpy(st + S_PQRIDOT, fo.acc.vPQRidot, 3 * sizeof(double));
    quat_qdot(st + S_Q, st + S_PQRI, st + S_QDOT);
    memcpy(st + S_PBA, fo.acc.vBodyAccel, 3 * sizeof(double));
    memcpy(st + S_PPQRIDOT, fo.acc.vPQRidot, 3 * sizeof(double));
    memcpy(st + S_PPQRI, fo.acc.vPQRi, 3 * sizeof(double));
    for (int j = 0; j < 3; j++) {     /* deques filled with the IC value (only 3 of 5 stored) */
        memcpy(st + S_DQ + 4 * j, st + S_QDOT, 4 * sizeof(double));
        memcpy(st + S_DPQRI + 3 * j, st + S_PQRIDOT, 3 * sizeof(double));
        memcpy(st + S_DIVEL + 3 * j, st + S_VEL, 3 * sizeof(double));
        memcpy(st + S_DUVW + 3 * j, st + S_UVWIDOT, 3 * sizeof(double));
    }
    /* fresh FCS (zeros) and engine */
    st[S_ENG + 0] = 100.0;
    st[S_ENG + 1] = 100.0;
    st[S_ENG + 2] = (100.0 - F16M_ENG_IDLEN2) / (F16M_ENG_MAXN2 - F16M_ENG_IDLEN2);
    st[S_ENG + 3] = fuelflow_pph;
}

/* build_seed_vector (ic.py:117-138) with ic_to_seedargs (ic.py:55-89), geodetic latitude.
 * ic = [lat_deg, lon_deg, alt_ft, vt_fps, phi_deg, theta_deg, psi_deg, alpha_deg, beta_deg, fuel_lbs] */
void orc_build_seed(const double *ic, int fcs_rate, double *st101)
{
    orc_init();
    const double D2R = M_PI / 180.0;
    double lat = ic[0] * D2R, lon = ic[1] * D2R, alt_ft = ic[2], vt = ic[3];
    double phi = ic[4] * D2R, theta = ic[5] * D2R, psi = ic[6] * D2R;
    double alpha = ic[7] * D2R, beta = ic[8] * D2R, fuel = ic[9];
    double ecef[3], Ti2ec[3][3], Tec2i[3][3], eci_pos[3], Tl2ec[3][3], Tl2i[3][3], Ti2l[3][3];
    double qL[4], Tl2b[3][3], Ti2b[3][3], Tb2i[3][3], radius, mlat, vb[3], vi[3], cr[3];
    geodetic_to_ecef(lat, lon, alt_ft, ecef);
    Ti2ec_from_epa(0.0, Ti2ec);
    transpose(Ti2ec, Tec2i);
    matvec(Tec2i, ecef, eci_pos);
    location_derived(ecef, &radius, &mlat, Tl2ec);
    matmul(Tec2i, Tl2ec, Tl2i);
    transpose(Tl2i, Ti2l);
    euler_to_quat(phi, theta, psi, qL);
    quat_to_T(qL, Tl2b);
    matmul(Tl2b, Ti2l, Ti2b);
    transpose(Ti2b, Tb2i);
    vb[0] = vt * cos(alpha) * cos(beta);
    vb[1] = vt * sin(beta);
    vb[2] = vt * sin(alpha) * cos(beta);
    matvec(Tb2i, vb, vi);
    cross(OMEGA, eci_pos, cr);
    double eci_vel[3] = {vi[0] + cr[0], vi[1] + cr[1], vi[2] + cr[2]};
    double euler[3] = {phi, theta, psi}, vPQR[3] = {0.0, 0.0, 0.0};
    Atmos at;
    atm_calculate(alt_ft, &at);
    double mach = vt / at.a;
    double vcas = (fabs(mach) > 0) ? vcalibrated_from_mach(mach, at.P) : 0.0;
    double prev_aux[9] = {alpha, mach, vcas * FPSTOKTS, vt, 0.0, -1.0, 0.0, 0.0, 0.0};
    fdm_seed(st101, eci_pos, eci_vel, euler, vPQR, 0.0, fuel, 0.0, prev_aux, fcs_dt_of(fcs_rate));
}

/* Exported frame helpers for unit tests. */
void orc_euler_to_quat(double phi, double tht, double psi, double *q) { euler_to_quat(phi, tht, psi, q); }
void orc_quat_to_T(const double *q, double *T9) { quat_to_T(q, (double (*)[3])T9); }
void orc_mat_to_quat(const double *T9, double *q) { mat_to_quat((const double (*)[3])T9, q); }
void orc_mat_to_euler(const double *T9, double *e) { mat_to_euler((const double (*)[3])T9, e); }
void orc_gravity_j2(const double *ecef, double lat, double *g) { orc_init(); gravity_j2(ecef, lat, g); }
double orc_vcal_from_mach(double mach, double p) { orc_init(); return vcalibrated_from_mach(mach, p); }
double orc_idleff(void) { orc_init(); return g_idleff; }
void orc_geodetic_to_ecef(double lat, double lon, double alt, double *o) { orc_init(); geodetic_to_ecef(lat, lon, alt, o); }
