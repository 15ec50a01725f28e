/*
 * obs_oracle.c -- CPU restatement of the reference's observation / reward / termination path
 * for one engagement batch: the state9 bridge (cuda_fdm/rl_env.py:88-163), the reconstructor
 * (BatchObsReward, research/competition_36500/runtime/cuda_fdm/obs_reward.py:319-819) and the
 * termination rule (cuda_fdm/rl_env.py:467-484, src/dogfight/envs/termination.py:12-14).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP observation/reward kernels.  Only tests/,
 * __graft_entry__.smoke() and bench.py's CPU baseline load it.
 *
 * Aircraft a of engagement e is 2e (plane 0) or 2e+1 (plane 1); partner = a ^ 1.  Functions
 * follow the reference's torch expressions term by term (torch's 3x3 batched products may
 * round differently from these plain sums; agreement is at the 1e-12 level, pinned by the
 * golden vectors written from the reference, tests/golden/make_obs_golden.py).
 */
#include <math.h>
#include <string.h>

/* ---- constants: research/competition_36500/runtime/claude_code/my_observation.py:103-160,
 *      cuda_fdm/rl_env.py:33-41, MY_REWARD_CONFIG (claude_code/my_reward.py:45-103) ---- */
static const double D2R = 3.141592653589793 / 180.0;
static const double R2D = 180.0 / 3.141592653589793;
#define FT2M 0.3048
#define M2FT_OBS 3.28084
#define G_ACC 9.80665
#define ROTATION_RATE 7.292115e-5
#define SEA_LEVEL_RADIUS_FT 20925646.32546
#define WGS_A 6378137.0
#define WGS_E2 0.0066943799901411
#define ORIGIN_LAT_DEG 37.240778
#define ORIGIN_LON_DEG 131.869556
#define MAX_SPEED 600.0
#define REL_VEL 600.0
#define MAX_RANGE_M 2500.0
#define MAX_CLOSURE 1000.0
#define VSPEED_SCALE 100.0
#define PQR_SCALE 4.0
#define AOA_SCALE 30.0
#define SIDESLIP_SCALE 15.0
#define MIN_ALT_M (1000.0 * FT2M)
#define ALT_DANGER 300.0
#define MAX_ALT_M 15000.0
#define ENERGY_ADV 5000.0
#define PURSUIT_ATA 30.0
#define PURSUIT_RANGE 3000.0
#define FUEL_BURN 8.0e-5
#define FUEL_REF 300.0
#define EPISODE_MAX 200.0
#define ACCEL_SCALE 150.0
#define T2_START 100.0
#define T3_START 150.0
#define MIN_DMG_FT 500.0
#define T1_MAX 3000.0
#define T2_MAX 3500.0
#define T3_MAX 4000.0
#define T1_CONE 1.0
#define T2_CONE 2.0
#define T3_CONE 3.0
#define ALT_LOG_SCALE_M 304.8
#define ALT_LOG_FLOOR 1e-4
#define TIME_TOL 1.0e-8

static double clampd(double x, double lo, double hi) { return x < lo ? lo : (x > hi ? hi : x); }
static double vnorm(const double v[3]) { return sqrt(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]); }
static void mv(const double A[3][3], const double v[3], double o[3])
{
    double a = A[0][0] * v[0] + A[0][1] * v[1] + A[0][2] * v[2];
    double b = A[1][0] * v[0] + A[1][1] * v[1] + A[1][2] * v[2];
    double c = A[2][0] * v[0] + A[2][1] * v[1] + A[2][2] * v[2];
    o[0] = a; o[1] = b; o[2] = c;
}
static void mvT(const double A[3][3], const double v[3], double o[3])
{
    double a = A[0][0] * v[0] + A[1][0] * v[1] + A[2][0] * v[2];
    double b = A[0][1] * v[0] + A[1][1] * v[1] + A[2][1] * v[2];
    double c = A[0][2] * v[0] + A[1][2] * v[1] + A[2][2] * v[2];
    o[0] = a; o[1] = b; o[2] = c;
}
static void mm(const double A[3][3], const double B[3][3], double C[3][3])
{
    double T[3][3];
    for (int i = 0; i < 3; i++)
        for (int j = 0; j < 3; j++) T[i][j] = A[i][0] * B[0][j] + A[i][1] * B[1][j] + A[i][2] * B[2][j];
    memcpy(C, T, sizeof T);
}

/* ------------------------------------------------------------------ state9 bridge */
static double g_ox, g_oy, g_oz, g_oslat, g_oclat, g_oslon, g_oclon;
static int g_init;

static void geodetic2ecef(double lat, double lon, double h, double *x, double *y, double *z)
{   /* rl_env.py:46-55 */
    double slat = sin(lat), clat = cos(lat), slon = sin(lon), clon = cos(lon);
    double N = WGS_A / sqrt(1.0 - WGS_E2 * slat * slat);
    *x = (N + h) * clat * clon;
    *y = (N + h) * clat * slon;
    *z = (N * (1.0 - WGS_E2) + h) * slat;
}

static void obs_init(void)
{
    if (g_init) return;
    double la = ORIGIN_LAT_DEG * D2R, lo = ORIGIN_LON_DEG * D2R;
    geodetic2ecef(la, lo, 0.0, &g_ox, &g_oy, &g_oz);          /* rl_env.py:59-60 */
    g_oslat = sin(la); g_oclat = cos(la); g_oslon = sin(lo); g_oclon = cos(lo);
    g_init = 1;
}

/* kinematics_state + ned_from_ecef_altasl + state9_flat (rl_env.py:88-163, 583-592):
 * N/E/D m (D = -MSL), roll/pitch/yaw deg, body u/v/w m/s */
void orc_state9(const double *st, double s9[9])
{
    obs_init();
    double px = st[0], py = st[1], pz = st[2], vx = st[3], vy = st[4], vz = st[5];
    double q0 = st[6], q1 = st[7], q2 = st[8], q3 = st[9], epa = st[13];
    double ce = cos(epa), se = sin(epa);
    double ex = ce * px + se * py, ey = -se * px + ce * py, ez = pz;
    double radius = sqrt(ex * ex + ey * ey + ez * ez);
    double rxy = sqrt(ex * ex + ey * ey);
    double sinLat = ez / radius, cosLat = rxy / radius, sinLon = ey / rxy, cosLon = ex / rxy;
    double Tl2ec[3][3] = {{-cosLon * sinLat, -sinLon, -cosLon * cosLat},
                          {-sinLon * sinLat, cosLon, -sinLon * cosLat},
                          {cosLat, 0.0, -sinLat}};
    double Tec2i[3][3] = {{ce, -se, 0.0}, {se, ce, 0.0}, {0.0, 0.0, 1.0}};
    double Tl2i[3][3], Ti2b[3][3], Tl2b[3][3];
    mm(Tec2i, Tl2ec, Tl2i);
    double q0q0 = q0 * q0, q1q1 = q1 * q1, q2q2 = q2 * q2, q3q3 = q3 * q3;
    double q0q1 = q0 * q1, q0q2 = q0 * q2, q0q3 = q0 * q3, q1q2 = q1 * q2, q1q3 = q1 * q3, q2q3 = q2 * q3;
    double T[3][3] = {{q0q0 + q1q1 - q2q2 - q3q3, 2 * (q1q2 + q0q3), 2 * (q1q3 - q0q2)},
                      {2 * (q1q2 - q0q3), q0q0 - q1q1 + q2q2 - q3q3, 2 * (q2q3 + q0q1)},
                      {2 * (q1q3 + q0q2), 2 * (q2q3 - q0q1), q0q0 - q1q1 - q2q2 + q3q3}};
    memcpy(Ti2b, T, sizeof T);
    mm(Ti2b, Tl2i, Tl2b);
    double d02 = clampd(Tl2b[0][2], -1.0, 1.0);
    double theta = asin(-d02);
    double phi = atan2(Tl2b[1][2], Tl2b[2][2]);
    double psi = atan2(Tl2b[0][1], Tl2b[0][0]);
    if (psi < 0.0) psi = psi + 2 * M_PI;
    double dv[3] = {vx - (-ROTATION_RATE * py), vy - (ROTATION_RATE * px), vz}, vb[3];
    mv(Ti2b, dv, vb);
    double exm = ex * FT2M, eym = ey * FT2M, ezm = ez * FT2M;
    double alt_m = (radius - SEA_LEVEL_RADIUS_FT) * FT2M;
    /* ecef_to_geodetic_latlon: Bowring (rl_env.py:64-74) */
    double b = WGS_A * sqrt(1.0 - WGS_E2);
    double ep2 = (WGS_A * WGS_A - b * b) / (b * b);
    double p = sqrt(exm * exm + eym * eym);
    double lon = atan2(eym, exm);
    double th = atan2(ezm * WGS_A, p * b);
    double sth = sin(th), cth = cos(th);
    double s3 = sth * sth * sth, c3 = cth * cth * cth;
    double lat = atan2(ezm + ep2 * b * s3, p - WGS_E2 * WGS_A * c3);
    double hx, hy, hz;
    geodetic2ecef(lat, lon, alt_m, &hx, &hy, &hz);
    double dx = hx - g_ox, dy = hy - g_oy, dz = hz - g_oz;
    s9[0] = -g_oslat * g_oclon * dx - g_oslat * g_oslon * dy + g_oclat * dz;
    s9[1] = -g_oslon * dx + g_oclon * dy;
    s9[2] = -alt_m;
    s9[3] = phi * R2D; s9[4] = theta * R2D; s9[5] = psi * R2D;
    s9[6] = vb[0] * FT2M; s9[7] = vb[1] * FT2M; s9[8] = vb[2] * FT2M;
}

/* ------------------------------------------------------------------ geometry (obs_reward.py:53-187) */
static void ned_to_body(double roll, double pitch, double yaw, double R[3][3])
{   /* Tx @ (Ty @ Tz) */
    double r = roll * D2R, p = pitch * D2R, y = yaw * D2R;
    double cr = cos(r), sr = sin(r), cp = cos(p), sp = sin(p), cy = cos(y), sy = sin(y);
    double Tx[3][3] = {{1, 0, 0}, {0, cr, sr}, {0, -sr, cr}};
    double Ty[3][3] = {{cp, 0, -sp}, {0, 1, 0}, {sp, 0, cp}};
    double Tz[3][3] = {{cy, sy, 0}, {-sy, cy, 0}, {0, 0, 1}};
    double TyTz[3][3];
    mm(Ty, Tz, TyTz);
    mm(Tx, TyTz, R);
}

static void unit_or_self(const double v[3], double o[3])
{   /* _unit: v / |v| if |v| > 0 else v */
    double n = vnorm(v);
    if (n > 0) { o[0] = v[0] / n; o[1] = v[1] / n; o[2] = v[2] / n; }
    else { o[0] = v[0]; o[1] = v[1]; o[2] = v[2]; }
}

static double ata_deg(const double *own, const double *tgt)
{
    double d[3] = {tgt[0] - own[0], tgt[1] - own[1], tgt[2] - own[2]}, pu[3], pt[3], R[3][3];
    unit_or_self(d, pu);
    ned_to_body(own[3], own[4], own[5], R);
    mv(R, pu, pt);
    return acos(clampd(pt[0], -1.0, 1.0)) * R2D;
}

static double aspect_deg(const double *own, const double *tgt)
{
    double R[3][3], d[3] = {own[0] - tgt[0], own[1] - tgt[1], own[2] - tgt[2]}, pu[3], b[3];
    ned_to_body(tgt[3], tgt[4], tgt[5], R);
    unit_or_self(d, pu);
    mv(R, pu, b);
    double pt0 = -b[0], pt1 = -b[1], pt2 = b[2];
    double sign = pt1 > 0 ? 1.0 : (pt1 < 0 ? -1.0 : (pt2 >= 0 ? 1.0 : -1.0));
    return sign * acos(clampd(pt0, -1.0, 1.0)) * R2D;
}

static void los_az_el(const double *own, const double *tgt, double *az, double *el)
{
    double d[3] = {tgt[0] - own[0], tgt[1] - own[1], tgt[2] - own[2]}, du[3], db[3], R[3][3];
    unit_or_self(d, du);
    ned_to_body(own[3], own[4], own[5], R);
    mv(R, du, db);
    *az = atan2(db[1], db[0]) * R2D;
    *el = -asin(clampd(db[2], -1.0, 1.0)) * R2D;
}

static void cross(const double a[3], const double b[3], double o[3])
{
    double x = a[1] * b[2] - a[2] * b[1], y = a[2] * b[0] - a[0] * b[2], z = a[0] * b[1] - a[1] * b[0];
    o[0] = x; o[1] = y; o[2] = z;
}

static void dir_frame(const double x[3], double R[3][3])
{   /* obs_reward.py:124-156: rows x, y, z; roll fixed by gravity; north then east fallback */
    double nx = vnorm(x);
    if (!(nx >= 1e-8)) {
        double I[3][3] = {{1, 0, 0}, {0, 1, 0}, {0, 0, 1}};
        memcpy(R, I, sizeof I);
        return;
    }
    double xn[3] = {x[0] / nx, x[1] / nx, x[2] / nx};
    const double refs[3][3] = {{0, 0, 1}, {1, 0, 0}, {0, 1, 0}};
    double zc[3][3], nz[3];
    for (int r = 0; r < 3; r++) {
        double d = xn[0] * refs[r][0] + xn[1] * refs[r][1] + xn[2] * refs[r][2];
        for (int i = 0; i < 3; i++) zc[r][i] = refs[r][i] - d * xn[i];
        nz[r] = vnorm(zc[r]);
    }
    int pick = (nz[0] >= 1e-6) ? 0 : ((nz[1] >= 1e-6) ? 1 : 2);
    double z[3], y[3], n;
    n = vnorm(zc[pick]);
    for (int i = 0; i < 3; i++) z[i] = zc[pick][i] / (n > 1e-300 ? n : 1e-300);
    cross(z, xn, y);
    n = vnorm(y);
    for (int i = 0; i < 3; i++) y[i] = y[i] / (n > 1e-300 ? n : 1e-300);
    cross(xn, y, z);
    for (int i = 0; i < 3; i++) { R[0][i] = xn[i]; R[1][i] = y[i]; R[2][i] = z[i]; }
}

static void bank_sincos(const double Rnb[3][3], const double dir[3], double *s, double *c)
{   /* obs_reward.py:159-166; body y axis in NED = column 1 of Rb2n = row 1 of Rnb */
    double Rf[3][3], by[3] = {Rnb[1][0], Rnb[1][1], Rnb[1][2]}, yv[3];
    dir_frame(dir, Rf);
    mv(Rf, by, yv);
    double mu = atan2(yv[2], yv[1]);
    *s = sin(mu); *c = cos(mu);
}

static void log_so3(const double R[3][3], double out[3])
{   /* obs_reward.py:169-186 */
    double tr = R[0][0] + R[1][1] + R[2][2];
    double cos_t = clampd((tr - 1.0) * 0.5, -1.0, 1.0);
    double theta = acos(cos_t);
    double ax[3] = {R[2][1] - R[1][2], R[0][2] - R[2][0], R[1][0] - R[0][1]};
    double denom = 2.0 * sin(theta);
    int ok = (theta >= 1e-8) && (fabs(denom) >= 1e-8);
    double scale = ok ? theta / denom : 0.0;
    for (int i = 0; i < 3; i++) out[i] = ax[i] * scale;
}

static double normz(double x, double lo, double hi)
{   /* normalize_t (obs_reward.py:192-198) */
    if (hi <= lo) return 0.0;
    double mid = (hi + lo) * 0.5, half = (hi - lo) * 0.5;
    return (clampd(x, lo, hi) - mid) / half;
}

static double damage_rate(double r_ft, double ata, double t)
{   /* damage_rate_t (obs_reward.py:206-218): tier 1 > 2 > 3 */
    double a = fabs(ata);
    if (r_ft >= MIN_DMG_FT && r_ft <= T1_MAX && a < T1_CONE)
        return 1.0 * (T1_MAX - r_ft) / (T1_MAX - MIN_DMG_FT);
    if (t >= T2_START && r_ft >= MIN_DMG_FT && r_ft <= T2_MAX && a < T2_CONE)
        return 0.3 * (T2_MAX - r_ft) / (T2_MAX - MIN_DMG_FT);
    if (t >= T3_START && r_ft >= MIN_DMG_FT && r_ft <= T3_MAX && a < T3_CONE)
        return 0.1 * (T3_MAX - r_ft) / (T3_MAX - MIN_DMG_FT);
    return 0.0;
}

/* ---- final-safe geometry (obs_reward.py:233-310), MY_REWARD_CONFIG values ---- */
static double smoothstep(double x, double e0, double e1)
{
    double z = clampd((x - e0) / (e1 - e0), 0.0, 1.0);
    return z * z * (3.0 - 2.0 * z);
}

static void velocity_ned(const double *s9, double vn[3])
{
    double R[3][3];
    ned_to_body(s9[3], s9[4], s9[5], R);
    mvT(R, s9 + 6, vn);
}

static void unit_fallback(const double v[3], const double fb[3], double o[3])
{   /* _unit_fallback_t: v/|v| if |v| >= 1e-9 else fb/max(|fb|, 1e-9) */
    double n = vnorm(v), fn = vnorm(fb);
    if (n >= 1e-9) { for (int i = 0; i < 3; i++) o[i] = v[i] / (n > 1e-9 ? n : 1e-9); }
    else { for (int i = 0; i < 3; i++) o[i] = fb[i] / (fn > 1e-9 ? fn : 1e-9); }
}

static double alignment(const double a[3], const double b[3])
{   /* _alignment_t, power 3 */
    const double ex[3] = {1.0, 0.0, 0.0};
    double au[3], bu[3];
    unit_fallback(a, ex, au);
    unit_fallback(b, au, bu);
    double q = (1.0 + clampd(au[0] * bu[0] + au[1] * bu[1] + au[2] * bu[2], -1.0, 1.0)) * 0.5;
    return clampd(pow(q, 3.0), 0.0, 1.0);
}

static double final_safe_side(const double *own, const double *tgt, double t)
{
    const double ex[3] = {1.0, 0.0, 0.0};
    double rel[3] = {tgt[0] - own[0], tgt[1] - own[1], tgt[2] - own[2]};
    double dist_m = vnorm(rel), dist_ft = dist_m / FT2M;
    double los[3];
    unit_fallback(rel, ex, los);
    double ata = fabs(ata_deg(own, tgt));
    double Rnb[3][3];
    ned_to_body(own[3], own[4], own[5], Rnb);
    double forward[3] = {Rnb[0][0], Rnb[0][1], Rnb[0][2]};
    double own_v[3], tgt_v[3];
    velocity_ned(own, own_v);
    velocity_ned(tgt, tgt_v);
    double own_speed = vnorm(own_v);
    if (own_speed < 30.0) own_speed = 30.0;
    double tau = clampd(dist_m / own_speed, 0.30, 1.50);
    double lv[3] = {tgt[0] + tgt_v[0] * tau - own[0], tgt[1] + tgt_v[1] * tau - own[1],
                    tgt[2] + tgt_v[2] * tau - own[2]};
    double lead[3], path[3];
    unit_fallback(lv, los, lead);
    unit_fallback(own_v, forward, path);
    double q_nose = alignment(forward, lead), q_path = alignment(path, lead);
    double intercept = 0.40 * q_nose + 0.60 * q_path;
    intercept /= 0.40 + 0.60;
    double direct = alignment(forward, los);
    double lead_w = smoothstep(dist_ft, 1000.0, 2500.0) * smoothstep(ata, 3.0, 8.0);
    double safe_lead = lead_w * intercept + (1.0 - lead_w) * direct;
    double broad = (ata <= 30.0) ? 1.0 : clampd((180.0 - ata) / (180.0 - 30.0), 0.0, 1.0);
    double angle_gate = 1.0 - smoothstep(ata, 3.0, 8.0);
    double range_gate = smoothstep(dist_ft, 600.0, 900.0) * (1.0 - smoothstep(dist_ft, 3200.0, 4300.0));
    double closing = (own_v[0] - tgt_v[0]) * los[0] + (own_v[1] - tgt_v[1]) * los[1]
                     + (own_v[2] - tgt_v[2]) * los[2];
    double mean_speed = 0.5 * (vnorm(own_v) + vnorm(tgt_v));
    double cr = closing / (mean_speed > 100.0 ? mean_speed : 100.0);
    double desired = 0.20 * smoothstep(dist_ft, 2000.0, 4500.0)
                     + (-0.12) * (1.0 - smoothstep(dist_ft, 650.0, 900.0));
    double zq = (cr - desired) / 0.15;
    double closure_q = exp(-0.5 * (zq * zq));
    double control = clampd(angle_gate * range_gate * closure_q, 0.0, 1.0);
    double fine = damage_rate(dist_ft, ata, t);
    double side = 0.50 * broad + 0.20 * safe_lead + 0.20 * control + 0.10 * fine;
    return clampd(side, 0.0, 1.0);
}

static double altitude_log(const double *s9)
{
    double x = (-s9[2]) / ALT_LOG_SCALE_M;
    return log(x < ALT_LOG_FLOOR ? ALT_LOG_FLOOR : x);
}

/* ------------------------------------------------------------------ reconstructor */
typedef struct {
    long nenv;
    double *hp, *fuel, *t_sec, *prev_att;
    unsigned char *prev_valid;
    double *pqr, *dealt, *taken, *hp_loss, *act_hist, *prev_x;
    unsigned char *prev_x_valid;
    double *prev_alt_log;
    double *prev_vel_ned, *accel;      /* NULL unless the 214-D acceleration features are on */
} OrcObr;

/* cfg: own_w, damage_scale, shaping_scale, win, loss, timeout_win, timeout_loss, timeout_draw */
enum { C_OWNW, C_DMG, C_SHAPE, C_WIN, C_LOSS, C_TWIN, C_TLOSS, C_TDRAW };
static const double DT_STEP = 6.0 / 60.0;   /* STEP_RATIO / SIM_HZ */

/* orc_state9 over n aircraft rows of 101 doubles (row-major (n, 101) -> (n, 9)). */
void orc_state9_batch(const double *st, long n, double *s9)
{
    obs_init();
    for (long i = 0; i < n; ++i) orc_state9(st + 101 * i, s9 + 9 * i);
}

void orc_obr_reset_envs(OrcObr *o, const unsigned char *mask)
{   /* reset_all / reset_envs (obs_reward.py:517-541) */
    for (long e = 0; e < o->nenv; e++) {
        if (mask && !mask[e]) continue;
        o->t_sec[e] = 0.0;
        for (int k = 0; k < 2; k++) {
            long a = 2 * e + k;
            o->hp[a] = 1.0; o->fuel[a] = 1.0;
            o->prev_valid[a] = 0; o->prev_x_valid[a] = 0;
            o->dealt[a] = o->taken[a] = o->hp_loss[a] = o->prev_x[a] = o->prev_alt_log[a] = 0.0;
            for (int i = 0; i < 3; i++) {
                o->prev_att[3 * a + i] = 0.0; o->pqr[3 * a + i] = 0.0;
                if (o->accel) { o->accel[3 * a + i] = 0.0; o->prev_vel_ned[3 * a + i] = 0.0; }
            }
            for (int i = 0; i < 20; i++) o->act_hist[20 * a + i] = 0.0;
        }
    }
}

void orc_obr_init_reward(OrcObr *o, const double *s9, const unsigned char *mask)
{   /* initialize_reward_state (obs_reward.py:727-744) */
    for (long e = 0; e < o->nenv; e++) {
        if (mask && !mask[e]) continue;
        const double *so = s9 + 18 * e, *sp = so + 9;
        double S_o = final_safe_side(so, sp, o->t_sec[e]);
        double S_p = final_safe_side(sp, so, o->t_sec[e]);
        o->prev_x[2 * e] = clampd(S_o - S_p, -1.0, 1.0);
        o->prev_x[2 * e + 1] = clampd(S_p - S_o, -1.0, 1.0);
        o->prev_x_valid[2 * e] = o->prev_x_valid[2 * e + 1] = 1;
        o->prev_alt_log[2 * e] = altitude_log(so);
        o->prev_alt_log[2 * e + 1] = altitude_log(sp);
    }
}

/* One RL step after the physics: push actions, advance the reconstructor, terminate, reward.
 * s9: (2*nenv, 9); actions: (2*nenv, 4). */
void orc_obr_step(OrcObr *o, const double *s9, const double *actions, const double *cfg,
                  int mode, double coef, double min_alt, double max_time, double *reward,
                  unsigned char *term, unsigned char *trunc)
{
    const double dt = DT_STEP;
    long nac = 2 * o->nenv;
    /* push_actions (obs_reward.py:571-575): roll by one, newest first */
    for (long a = 0; a < nac; a++) {
        double *h = o->act_hist + 20 * a;
        memmove(h + 4, h, 16 * sizeof(double));
        for (int c = 0; c < 4; c++) h[c] = actions[4 * a + c];
    }
    for (long e = 0; e < o->nenv; e++) {
        long ia = 2 * e, ib = ia + 1;
        const double *sa = s9 + 9 * ia, *sb = s9 + 9 * ib;
        /* advance (obs_reward.py:578-614) */
        double d[3] = {sb[0] - sa[0], sb[1] - sa[1], sb[2] - sa[2]};
        double r_ft = vnorm(d) * M2FT_OBS;
        double t_old = o->t_sec[e];
        double rate_a = damage_rate(r_ft, ata_deg(sa, sb), t_old);   /* a deals to b */
        double rate_b = damage_rate(r_ft, ata_deg(sb, sa), t_old);
        for (int k = 0; k < 2; k++) {
            long a = ia + k;
            const double *s = k ? sb : sa;
            double taken = k ? rate_a : rate_b, dealt = k ? rate_b : rate_a;
            double hp_before = o->hp[a];
            double hp_after = hp_before - taken * dt;
            if (hp_after < 0.0) hp_after = 0.0;
            o->hp_loss[a] = hp_before - hp_after;
            o->hp[a] = hp_after;
            double speed = vnorm(s + 6);
            double burn = FUEL_BURN * (speed / FUEL_REF);
            double f = o->fuel[a] - burn * dt;
            o->fuel[a] = f < 0.0 ? 0.0 : f;
            double Np[3][3], Nc[3][3], rd[3][3], lg[3];
            ned_to_body(o->prev_att[3 * a], o->prev_att[3 * a + 1], o->prev_att[3 * a + 2], Np);
            ned_to_body(s[3], s[4], s[5], Nc);
            for (int i = 0; i < 3; i++)       /* Rb2n_prev^T Rb2n_curr = Np Nc^T */
                for (int j = 0; j < 3; j++) rd[i][j] = Np[i][0] * Nc[j][0] + Np[i][1] * Nc[j][1] + Np[i][2] * Nc[j][2];
            log_so3(rd, lg);
            for (int i = 0; i < 3; i++)
                o->pqr[3 * a + i] = o->prev_valid[a] ? lg[i] / (dt > 1e-8 ? dt : 1e-8) : 0.0;
            if (o->accel) {                     /* 214-D lineage: NED acceleration (cuda_fdm/obs_reward.py:568-575) */
                double vn[3];
                mvT(Nc, s + 6, vn);
                for (int i = 0; i < 3; i++) {
                    o->accel[3 * a + i] = o->prev_valid[a] ? (vn[i] - o->prev_vel_ned[3 * a + i]) / (dt > 1e-8 ? dt : 1e-8) : 0.0;
                    o->prev_vel_ned[3 * a + i] = vn[i];
                }
            }
            for (int i = 0; i < 3; i++) o->prev_att[3 * a + i] = s[3 + i];
            o->prev_valid[a] = 1;
            o->dealt[a] = dealt;
            o->taken[a] = taken;
        }
        double t_new = t_old + dt;
        o->t_sec[e] = t_new;
        /* termination (rl_env.py:467-484) */
        int finite = 1;
        for (int i = 0; i < 9; i++) if (!isfinite(sa[i]) || !isfinite(sb[i])) finite = 0;
        double alt_a = -sa[2], alt_b = -sb[2];
        int te = (alt_a < min_alt) || (alt_b < min_alt) || (o->hp[ia] <= 0.0) || (o->hp[ib] <= 0.0) || !finite;
        int tr = !te && (t_new >= max_time - TIME_TOL);
        term[e] = (unsigned char)te;
        trunc[e] = (unsigned char)tr;
        /* compute_reward (obs_reward.py:747-819) */
        double S_a = final_safe_side(sa, sb, t_new), S_b = final_safe_side(sb, sa, t_new);
        double G[2] = {clampd(S_a - S_b, -1.0, 1.0), clampd(S_b - S_a, -1.0, 1.0)};
        double alt_log[2] = {altitude_log(sa), altitude_log(sb)};
        double shaping_mult = cfg[C_SHAPE] / 0.0001;
        double r_shape[2];
        for (int k = 0; k < 2; k++) {
            long a = ia + k, p = ia + (1 - k);
            double prev = o->prev_x_valid[a] ? o->prev_x[a] : G[k];
            r_shape[k] = shaping_mult * 5.0 / 200.0 * 0.5 * (prev + G[k]) * dt;
            if (mode == 1)
                r_shape[k] = o->prev_x_valid[p] ? (o->prev_alt_log[p] - alt_log[1 - k]) * coef : 0.0;
        }
        for (int k = 0; k < 2; k++) {
            long a = ia + k, p = ia + (1 - k);
            double loss_o = o->hp_loss[a], loss_t = o->hp_loss[p];
            double r_dmg;
            if (mode == 2) r_dmg = loss_t * cfg[C_DMG];
            else if (mode == 3) r_dmg = -(loss_o * cfg[C_OWNW]) * cfg[C_DMG];
            else r_dmg = (loss_t - loss_o * cfg[C_OWNW]) * cfg[C_DMG];
            const double *so = k ? sb : sa, *st = k ? sa : sb;
            double hp_o = o->hp[a], hp_t = o->hp[p];
            int own_below = (-so[2]) < MIN_ALT_M, tgt_below = (-st[2]) < MIN_ALT_M;
            double r_term = 0.0;
            if (te && own_below) r_term = -(hp_o > 0.0 ? hp_o : 0.0) * cfg[C_DMG];
            if (te && !own_below && tgt_below) r_term = (hp_t > 0.0 ? hp_t : 0.0) * cfg[C_DMG];
            int hp_only = te && !own_below && !tgt_below;
            if (hp_only && hp_t <= 0.0) r_term = r_term + cfg[C_WIN];
            if (hp_only && hp_o <= 0.0) r_term = r_term + cfg[C_LOSS];
            if (tr) r_term = hp_o > hp_t ? cfg[C_TWIN] : (hp_o < hp_t ? cfg[C_TLOSS] : cfg[C_TDRAW]);
            reward[a] = r_dmg + r_shape[k] + r_term;
        }
        for (int k = 0; k < 2; k++) {
            o->prev_x[ia + k] = G[k];
            o->prev_x_valid[ia + k] = 1;
            o->prev_alt_log[ia + k] = alt_log[k];
        }
    }
}

/* ------------------------------------------------------------------ observation */
static float store(double v)
{   /* torch.nan_to_num(nan=0, posinf=10, neginf=-10) then float32 */
    if (isnan(v)) v = 0.0;
    else if (isinf(v)) v = v > 0 ? 10.0 : -10.0;
    return (float)v;
}

/* build_obs (obs_reward.py:617-723); obs_dim 184, or 214 with the NED-acceleration vectors of
 * the 214-D lineage (cuda_fdm/obs_reward.py build_obs, claude_code/my_observation.py:217-230). */
void orc_obr_build_obs(const OrcObr *o, const double *s9, int obs_dim, const unsigned char *mask,
                       float *obs)
{
    long nac = 2 * o->nenv;
    for (long a = 0; a < nac; a++) {
        if (mask && !mask[a >> 1]) continue;
        long p = a ^ 1, e = a >> 1;
        const double *so = s9 + 9 * a, *st = s9 + 9 * p;
        float *out = obs + (long)obs_dim * a;
        double t = o->t_sec[e];
        double Rno[3][3], Rnt[3][3];
        ned_to_body(so[3], so[4], so[5], Rno);
        ned_to_body(st[3], st[4], st[5], Rnt);
        double own_vn[3], tgt_vn[3], rel_vn[3];
        mvT(Rno, so + 6, own_vn);
        mvT(Rnt, st + 6, tgt_vn);
        for (int i = 0; i < 3; i++) rel_vn[i] = tgt_vn[i] - own_vn[i];
        double own_spd = vnorm(so + 6), tgt_spd = vnorm(st + 6);
        double own_alt = -so[2], tgt_alt = -st[2];
        double delta[3] = {st[0] - so[0], st[1] - so[1], st[2] - so[2]};
        double dist = vnorm(delta), los_u[3] = {0, 0, 0}, closure = 0.0;
        if (dist > 1e-6) {
            for (int i = 0; i < 3; i++) los_u[i] = delta[i] / dist;
            closure = (own_vn[0] - tgt_vn[0]) * los_u[0] + (own_vn[1] - tgt_vn[1]) * los_u[1]
                      + (own_vn[2] - tgt_vn[2]) * los_u[2];
        }
        double ata = ata_deg(so, st), en_ata = ata_deg(st, so), aa = aspect_deg(so, st), az, el;
        los_az_el(so, st, &az, &el);
        double u = so[6], v = so[7], w = so[8], aoa = 0.0, ss = 0.0;
        if (!(own_spd < 1.0)) {
            aoa = atan2(w, u) * R2D;
            ss = atan2(v, sqrt(u * u + w * w)) * R2D;
        }
        double vspeed = -own_vn[2];
        double e_adv = (own_alt + own_spd * own_spd / (2.0 * G_ACC)) - (tgt_alt + tgt_spd * tgt_spd / (2.0 * G_ACC));
        double cone = t >= T3_START ? T3_CONE : (t >= T2_START ? T2_CONE : T1_CONE);
        double maxr_ft = t >= T3_START ? T3_MAX : (t >= T2_START ? T2_MAX : T1_MAX);
        double cc = cone > 1e-6 ? cone : 1e-6;
        double min_r_m = MIN_DMG_FT * FT2M, max_r_m = maxr_ft * FT2M;
        double span = max_r_m - min_r_m;
        if (span < 1e-6) span = 1e-6;
        double obs_s, obc, tbs, tbc;
        bank_sincos(Rno, own_vn, &obs_s, &obc);
        bank_sincos(Rnt, tgt_vn, &tbs, &tbc);
        double pf_ata = 1.0 - fabs(ata) / PURSUIT_ATA; if (pf_ata < 0.0) pf_ata = 0.0;
        double pf_rng = 1.0 - dist / PURSUIT_RANGE; if (pf_rng < 0.0) pf_rng = 0.0;
        double sc[50] = {
            normz(own_spd, 0.0, MAX_SPEED), normz(tgt_spd, 0.0, MAX_SPEED),
            tanh(aoa / AOA_SCALE), tanh(ss / SIDESLIP_SCALE),
            tanh((own_alt - MIN_ALT_M) / ALT_DANGER), normz(vspeed, -VSPEED_SCALE, VSPEED_SCALE),
            normz(o->hp[a], 0.0, 1.0), normz(o->hp[p], 0.0, 1.0), o->hp[a] - o->hp[p],
            e_adv / (fabs(e_adv) + ENERGY_ADV), normz(dist, 0.0, MAX_RANGE_M),
            normz(closure, -MAX_CLOSURE, MAX_CLOSURE),
            sin(ata * D2R), cos(ata * D2R), sin(aa * D2R), cos(aa * D2R),
            sin(az * D2R), cos(az * D2R), sin(el * D2R), cos(el * D2R),
            2.0 * exp(-((ata / 3.0) * (ata / 3.0))) - 1.0, tanh((cone - fabs(ata)) / cc),
            2.0 * exp(-((en_ata / 3.0) * (en_ata / 3.0))) - 1.0, tanh((cone - fabs(en_ata)) / cc),
            tanh((dist - min_r_m) / span), tanh((max_r_m - dist) / span), normz(t, 0.0, EPISODE_MAX),
            sin(so[3] * D2R), cos(so[3] * D2R), sin(so[4] * D2R), cos(so[4] * D2R),
            sin(so[5] * D2R), cos(so[5] * D2R), sin(st[3] * D2R), cos(st[3] * D2R),
            sin(st[4] * D2R), cos(st[4] * D2R), sin(st[5] * D2R), cos(st[5] * D2R),
            obs_s, obc, tbs, tbc,
            normz(o->fuel[a], 0.0, 1.0), normz(o->fuel[p], 0.0, 1.0),
            clampd(2.0 * o->dealt[a] - 1.0, -1.0, 1.0), clampd(2.0 * o->taken[a] - 1.0, -1.0, 1.0),
            2.0 * (pf_ata * pf_rng) - 1.0,
            normz(own_alt, 0.0, MAX_ALT_M), normz(tgt_alt, 0.0, MAX_ALT_M)};
        for (int i = 0; i < 50; i++) out[i] = store(sc[i]);
        /* frame-expressed vectors (my_observation.py _VEC_LAYOUT order) */
        double om_o[3], om_t[3];
        mvT(Rno, o->pqr + 3 * a, om_o);
        mvT(Rnt, o->pqr + 3 * p, om_t);
        double I3[3][3] = {{1, 0, 0}, {0, 1, 0}, {0, 0, 1}}, Fmv[3][3], Fov[3][3], Flos[3][3];
        dir_frame(own_vn, Fmv);
        dir_frame(tgt_vn, Fov);
        dir_frame(delta, Flos);
        const double (*F[6])[3] = {I3, Rno, Rnt, Fmv, Fov, Flos};
        const double grav[3] = {0, 0, 1};
        const double *V[9] = {grav, los_u, own_vn, tgt_vn, rel_vn, om_o, om_t,
                              o->accel ? o->accel + 3 * a : NULL, o->accel ? o->accel + 3 * p : NULL};
        /* vector, kind (0 unit, 1 vel, 2 omega, 3 accel), skipped frame */
        const int spec[9][3] = {{0, 0, 0}, {1, 0, 5}, {2, 1, 3}, {3, 1, 4}, {4, 1, -1},
                                {5, 2, -1}, {6, 2, -1}, {7, 3, 3}, {8, 3, 4}};
        int nvec = obs_dim == 214 ? 9 : 7, col = 50;
        for (int s = 0; s < nvec; s++) {
            for (int f = 0; f < 6; f++) {
                if (f == spec[s][2]) continue;
                double comp[3];
                mv(F[f], V[spec[s][0]], comp);
                for (int r = 0; r < 3; r++) {
                    double val = comp[r];
                    if (spec[s][1] == 1) val = normz(comp[r], -REL_VEL, REL_VEL);
                    else if (spec[s][1] == 2) val = tanh(comp[r] / PQR_SCALE);
                    else if (spec[s][1] == 3) val = normz(comp[r], -ACCEL_SCALE, ACCEL_SCALE);
                    out[col++] = store(val);
                }
            }
        }
        for (int i = 0; i < 20; i++) out[col + i] = store(o->act_hist[20 * a + i]);
    }
}
