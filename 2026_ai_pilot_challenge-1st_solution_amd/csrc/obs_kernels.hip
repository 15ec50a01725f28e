// obs_kernels.hip -- observation, reward, termination and autoreset kernels (gfx950).
//
// One lane per aircraft; the two aircraft of an engagement sit in adjacent lanes (2e, 2e+1) of
// one wavefront and trade what each computed about itself (state9, attitude, NED velocity,
// damage rate, geometry score, ...) through __shfl_xor(x, 1).  So every aircraft's state9 and
// attitude trigonometry is evaluated once per launch, where the reference evaluates each of
// them in both the advance thread (one per engagement) and both observation threads.
//
// Kernels mirror the reference's launch set (research/competition_36500/runtime/cuda_fdm/
// obs_reward.py:410-469: advance, init_reward, build_obs; external_observation.cu for the 214-D
// variant) and add env_post_step, which is GpuDogfightVecEnv.step's whole post-physics sequence
// (cuda_fdm/rl_env.py:540-580) in one launch.
#include <hip/hip_runtime.h>

#include <math.h>

#include "f16_capi_common.h"
#include "f16_fdm.h"
#include "f16_obs.h"
#include "f16_state.h"
#include "fdm_image.h"
#include "fdm_quad.h"
#include "fdm_split.h"
#include "obs_device.h"
#include "philox.h"

namespace f16obs {

constexpr int kObsBlock = 256;
// Kernels that write observation rows run one wave per workgroup: each lane builds the vector
// block of its row (the 114 or 144 columns the frames produce out of order) in a wave-private
// LDS tile (odd pitch: lane-per-row stores hit distinct banks), then the wave copies the tile
// out in consecutive 8-byte pieces; the rows' scalar block and action history are contiguous
// and go out from registers.  The tile is 29 KB (184-D) or 37 KB (214-D), so four wavefronts
// fit a CU's LDS.
constexpr int kRowBlock = 64;
// The two-wave post-physics step runs two groups of 64 aircraft per workgroup.
constexpr int kPostGroups = 2;
constexpr int kPostSplitBlock = 2 * kRowBlock * kPostGroups;
constexpr double kFuelBurn = 8.0e-5;          // fuel proxy burn per second at 300 m/s
constexpr double kFuelRef = 300.0;
constexpr double kSeaLevelRadiusFtT = 20925646.32546;

__device__ __forceinline__ double xch(double v) { return __shfl_xor(v, 1); }
__device__ __forceinline__ int xchi(int v) { return __shfl_xor(v, 1); }

F16_HD void attitude_rpy(double roll, double pitch, double yaw, Att& A) {
  const double s9[9] = {0.0, 0.0, 0.0, roll, pitch, yaw, 0.0, 0.0, 0.0};
  attitude(s9, A);
}

// This aircraft's kinematics as the observation sees them.
struct Kin9 {
  double s9[9];
  Att A;
  double vn[3];    // NED velocity R^T (u, v, w)
  double spd;      // |(u, v, w)|
};

// The partner aircraft's, received through the lane exchange.
struct Peer {
  double s9[9];
  double R[3][3];
  double sr, cr, sp, cp, sy, cy;
  double vn[3];
  double spd;
};

// Geometry from this aircraft to its partner.
struct Geo {
  double delta[3];  // partner - own position, NED m
  double dist;
  double b[3];      // own body-frame unit line of sight R (delta / |delta|)
  double ata;       // antenna train angle, deg
};

// Reconstructor values the observation reads for one aircraft.
struct ObsIn {
  double hp, fuel, dealt, taken, t;
  double pqr[3];
  double accel[3];
};

__device__ __forceinline__ void make_kin(const double* st, long ld, const Origin& O, Kin9& k) {
  state9(st, ld, O, k.s9, &k.A);
  mtv3(k.A.R, k.s9 + 6, k.vn);
  k.spd = norm3(k.s9 + 6);
}

__device__ __forceinline__ void exchange(const Kin9& k, Peer& p) {
#pragma unroll
  for (int i = 0; i < 9; ++i) p.s9[i] = xch(k.s9[i]);
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) p.R[i][j] = xch(k.A.R[i][j]);
  p.sr = xch(k.A.sr); p.cr = xch(k.A.cr); p.sp = xch(k.A.sp);
  p.cp = xch(k.A.cp); p.sy = xch(k.A.sy); p.cy = xch(k.A.cy);
#pragma unroll
  for (int i = 0; i < 3; ++i) p.vn[i] = xch(k.vn[i]);
  p.spd = xch(k.spd);
}

__device__ __forceinline__ void pair_geo(const Kin9& k, const Peer& p, Geo& g) {
#pragma unroll
  for (int i = 0; i < 3; ++i) g.delta[i] = p.s9[i] - k.s9[i];
  g.dist = norm3(g.delta);
  double u[3];
  unit_or_self(g.delta, u);
  mv3(k.A.R, u, g.b);
  g.ata = acos(clampd(g.b[0], -1.0, 1.0)) * kR2D;
}

__device__ __forceinline__ bool finite9(const double s[9]) {
  bool ok = true;
#pragma unroll
  for (int i = 0; i < 9; ++i) ok = ok && isfinite(s[i]);
  return ok;
}

__device__ __forceinline__ double safe_side(const Kin9& k, const Peer& p, const Geo& g, double t) {
  return final_safe_side(k.s9, k.A.R, k.vn, p.s9, p.vn, g.ata, t);
}

// obs_reward.py:727-744: re-anchor G and the log altitude at time t.
__device__ __forceinline__ void lane_init_reward(const Kin9& k, const Peer& p, const Geo& g,
                                                 long a, double t, const F16Recon& r) {
  const double s_own = safe_side(k, p, g, t);
  const double s_opp = xch(s_own);
  r.prev_x[a] = clampd(s_own - s_opp, -1.0, 1.0);
  r.prev_x_valid[a] = 1;
  r.prev_alt_log[a] = altitude_log(-k.s9[2]);
}

// The decision's damage exchange, HP, fuel proxy and clock of this aircraft (lane_advance's
// arithmetic, shared with the four-role step's scalar-block wave, which forms them from the
// same loads instead of waiting for them).  Both lanes of a pair call it together (xch).
struct HpFuel { double dealt, taken, hp, fuel, t; };
__device__ __forceinline__ HpFuel advance_hp_fuel(const Kin9& k, const Geo& g, double hp_before,
                                                  double fuel_before, double t_old) {
  HpFuel o;
  o.dealt = damage_rate(g.dist * kM2FtObs, g.ata, t_old);
  o.taken = xch(o.dealt);
  double hp = hp_before - o.taken * kDtStep;
  o.hp = hp < 0.0 ? 0.0 : hp;
  const double burn = kFuelBurn * (k.spd * (1.0 / kFuelRef));
  double fuel = fuel_before - burn * kDtStep;
  o.fuel = fuel < 0.0 ? 0.0 : fuel;
  o.t = t_old + kDtStep;
  return o;
}

struct AdvOut {
  double reward;
  bool term, trunc;
  ObsIn obs;                // this aircraft's reconstructor values after the update
  float hist[kActHist];     // the new action history as observation features
};

// One decision of the reconstructor, termination and reward for this aircraft
// (obs_reward.py:571-614 push_actions/advance, 747-819 compute_reward; rl_env.py:467-484).
// Every reconstructor value the decision reads is loaded before anything is written back, so the
// loads go out together.  The new action history is also returned as observation features.
__device__ __forceinline__ AdvOut lane_advance(const Kin9& k, const Peer& p, const Geo& g, long a,
                                               long e, const double* __restrict__ act,
                                               const F16Recon& r, const F16RewardCfg& c,
                                               double phys_fuel = 1.0) {
  const long ld = r.ld;
  AdvOut out;
  // ---- loads
  double h[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) h[i] = r.act_hist[i * ld + a];
  double an[4];
#pragma unroll
  for (int ch = 0; ch < 4; ++ch) an[ch] = act[4 * a + ch];
  const double t_old = r.t_sec[e];
  const double hp_before = r.hp[a];
  const double fuel_before = r.fuel[a];
  const bool prev_valid = r.prev_valid[a] != 0;
  double patt[3], pvel[3] = {0.0, 0.0, 0.0};
#pragma unroll
  for (int i = 0; i < 3; ++i) patt[i] = r.prev_att[i * ld + a];
  if (r.accel) {
#pragma unroll
    for (int i = 0; i < 3; ++i) pvel[i] = r.prev_vel_ned[i * ld + a];
  }
  const bool pxv = r.prev_x_valid[a] != 0;
  const double prev_x = r.prev_x[a];
  const double prev_alt_log = r.prev_alt_log[a];
  // ---- action history: roll by one decision, newest first
#pragma unroll
  for (int i = 0; i < 16; ++i) r.act_hist[(i + 4) * ld + a] = h[i];
#pragma unroll
  for (int ch = 0; ch < 4; ++ch) r.act_hist[ch * ld + a] = an[ch];
#pragma unroll
  for (int ch = 0; ch < 4; ++ch) out.hist[ch] = obs_value(an[ch]);
#pragma unroll
  for (int i = 0; i < 16; ++i) out.hist[4 + i] = obs_value(h[i]);
  // damage exchanged inside the cones, rated at the time entering the decision
  const HpFuel hf = advance_hp_fuel(k, g, hp_before, fuel_before, t_old);
  const double dealt = hf.dealt, taken = hf.taken, hp = hf.hp, fuel = hf.fuel;
  const double hp_loss = hp_before - hp;
  r.hp_loss[a] = hp_loss;
  r.hp[a] = hp;
  r.fuel[a] = fuel;
  // body rates from the attitude change since the previous decision
  double pqr[3] = {0.0, 0.0, 0.0};
  if (prev_valid) {
    Att P;
    attitude_rpy(patt[0], patt[1], patt[2], P);
    so3_rates(P.R, k.A.R, pqr);
  }
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    r.pqr[i * ld + a] = pqr[i];
    r.prev_att[i * ld + a] = k.s9[3 + i];
  }
  double acc[3] = {0.0, 0.0, 0.0};
  if (r.accel) {   // 214-D lineage: NED acceleration from the velocity difference
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      if (prev_valid) acc[i] = (k.vn[i] - pvel[i]) * (1.0 / kDtStep);
      r.accel[i * ld + a] = acc[i];
      r.prev_vel_ned[i * ld + a] = k.vn[i];
    }
  }
  r.prev_valid[a] = 1;
  r.dealt[a] = dealt;
  r.taken[a] = taken;
  const double t_new = hf.t;
  if (!(a & 1)) r.t_sec[e] = t_new;
  // termination (rl_env.py:467-484): hard deck, HP, non-finite; truncation at the time limit
  const double alt_o = -k.s9[2], alt_t = -p.s9[2];
  const double hp_t = xch(hp);
  const bool finite = finite9(k.s9) && finite9(p.s9);
  const double phys_fuel_t = xch(phys_fuel);
  const bool fuel_out = c.fuel_exhaustion && (phys_fuel <= 0.0 || phys_fuel_t <= 0.0);
  const bool te = (alt_o < c.min_alt_m) || (alt_t < c.min_alt_m) || (hp <= 0.0) || (hp_t <= 0.0) ||
                  !finite || fuel_out;
  const bool tr = !te && (t_new >= c.max_time_s - kTimeTol);
  // reward: damage + potential shaping (or altitude hunting) + terminal
  const double s_own = safe_side(k, p, g, t_new);
  const double s_opp = xch(s_own);
  const double G = clampd(s_own - s_opp, -1.0, 1.0);
  const double alt_log = altitude_log(alt_o);
  const double alt_log_t = xch(alt_log);
  const double pxv_t = xch(pxv ? 1.0 : 0.0);
  const double prev_alt_log_t = xch(prev_alt_log);
  double r_shape;
  if (c.mode == 1) {
    r_shape = pxv_t != 0.0 ? (prev_alt_log_t - alt_log_t) * c.alt_hunt_coef : 0.0;
  } else {
    const double prev = pxv ? prev_x : G;
    r_shape = c.shaping_reward_scale / 0.0001 * 5.0 / 200.0 * 0.5 * (prev + G) * kDtStep;
  }
  const double loss_t = xch(hp_loss);
  double r_dmg;
  if (c.mode == 2) r_dmg = loss_t * c.damage_scale;
  else if (c.mode == 3) r_dmg = -(hp_loss * c.own_damage_weight) * c.damage_scale;
  else r_dmg = (loss_t - hp_loss * c.own_damage_weight) * c.damage_scale;
  const bool own_below = alt_o < kMinAltM, tgt_below = alt_t < kMinAltM;
  double r_term = 0.0;
  if (te && own_below) r_term = -(hp > 0.0 ? hp : 0.0) * c.damage_scale;
  if (te && !own_below && tgt_below) r_term = (hp_t > 0.0 ? hp_t : 0.0) * c.damage_scale;
  const bool hp_only = te && !own_below && !tgt_below;
  if (hp_only && hp_t <= 0.0) r_term = r_term + c.win_reward;
  if (hp_only && hp <= 0.0) r_term = r_term + c.loss_reward;
  if (tr) r_term = hp > hp_t ? c.timeout_win_reward
                             : (hp < hp_t ? c.timeout_loss_reward : c.timeout_draw_reward);
  r.prev_x[a] = G;
  r.prev_x_valid[a] = 1;
  r.prev_alt_log[a] = alt_log;
  out.reward = r_dmg + r_shape + r_term;
  out.term = te;
  out.trunc = tr;
  out.obs.hp = hp; out.obs.fuel = fuel; out.obs.dealt = dealt; out.obs.taken = taken;
  out.obs.t = t_new;
#pragma unroll
  for (int i = 0; i < 3; ++i) { out.obs.pqr[i] = pqr[i]; out.obs.accel[i] = acc[i]; }
  return out;
}

// Feature transforms stored as float32: tanh and a Gaussian from the hardware exp2/reciprocal
// (absolute error < 3e-7, far inside the float32 output's tolerance).
__device__ __forceinline__ double tanh_feat(double x) {
  const float xf = (float)x;
  const float t = __builtin_amdgcn_exp2f(fabsf(xf) * -2.8853900817779268f);
  return copysignf((1.0f - t) * __builtin_amdgcn_rcpf(1.0f + t), xf);
}
__device__ __forceinline__ double gauss_feat(double z) {      // e^{-z^2}
  const float zf = (float)z;
  return __builtin_amdgcn_exp2f(-(zf * zf) * 1.4426950408889634f);
}

// Where one observation row goes.  Rows are built lane-per-row in a wave-private LDS tile and
// copied out coalesced by the wave (the frames produce the vector block's columns out of
// order).  Two tile layouts:
//   FULL:  the whole row is staged (pitch D | 1); the wave copies the tile as one flat array.
//          Fastest while every wavefront of the launch is resident at once.
//   !FULL: only the vector block, columns [50, D - 20), is staged (pitch (D - 70) | 1, 29 KB
//          for 184-D, 37 KB for 214-D, so four wavefronts fit a CU's LDS); the scalar block
//          and the action history, 50 + 20 contiguous floats, are stored by the lane straight
//          from registers to `row_all` and, when set, `row_live` (rows of the output matrices,
//          16-byte aligned for D = 184, 8-byte for D = 214).  Used for launches larger than
//          the FULL tile lets the GPU hold.
// `tile` = this lane's tile row, holding column tile_col0<FULL>() at tile[0].
struct ObsOut {
  float* tile;
  float* row_all;
  float* row_live;
};

constexpr int kVecCol0 = 50;                      // first vector-block column
template <int D, bool FULL> constexpr int tile_pitch() { return FULL ? (D | 1) : ((D - 70) | 1); }
template <bool FULL> constexpr int tile_col0() { return FULL ? 0 : kVecCol0; }

// n consecutive floats of a row, from registers, at column C0: 16-byte stores where the row
// layout allows (D and C0 multiples of 4), 8-byte otherwise.
template <int D, int C0, int N>
__device__ __forceinline__ void store_run(float* row, const float (&v)[N]) {
  static_assert(N % 2 == 0 && C0 % 2 == 0, "even runs at even columns");
  int i = 0;
  if constexpr (D % 4 == 0 && C0 % 4 == 0) {
#pragma unroll
    for (; i + 4 <= N; i += 4)
      *reinterpret_cast<float4*>(row + C0 + i) = make_float4(v[i], v[i + 1], v[i + 2], v[i + 3]);
  }
#pragma unroll
  for (; i < N; i += 2) *reinterpret_cast<float2*>(row + C0 + i) = make_float2(v[i], v[i + 1]);
}

// A contiguous run of the row outside the vector block: into the tile (FULL) or to the rows.
template <int D, bool FULL, int C0, int N>
__device__ __forceinline__ void store_run2(const ObsOut& out, const float (&v)[N]) {
  if constexpr (FULL) {
#pragma unroll
    for (int i = 0; i < N; ++i) out.tile[C0 + i] = v[i];
  } else {
    store_run<D, C0, N>(out.row_all, v);
    if (out.row_live) store_run<D, C0, N>(out.row_live, v);
  }
}

template <bool FULL>
__device__ __forceinline__ void put_vec(float* tile, int j, double v) {
  tile[j - tile_col0<FULL>()] = obs_value(v);
}

enum VecKind { kRaw = 0, kVel = 1, kRate = 2, kAcc = 3 };

// The observation's vector block (my_observation.py _VEC_LAYOUT): vectors in order, each in the
// six frames 0 NED, 1 own body, 2 partner body, 3 own motion, 4 partner motion, 5 line of sight,
// minus one skipped frame.  Column of (vector s, frame f) in the row:
struct VecSlot { int kind, skip; };
constexpr VecSlot kVecs[9] = {{kRaw, 0}, {kRaw, 5}, {kVel, 3}, {kVel, 4}, {kVel, -1},
                              {kRate, -1}, {kRate, -1}, {kAcc, 3}, {kAcc, 4}};
__host__ __device__ constexpr int vec_base(int s) {
  return s == 0 ? 50 : vec_base(s - 1) + 3 * (kVecs[s - 1].skip >= 0 ? 5 : 6);
}
__host__ __device__ constexpr int vec_col(int s, int f) {
  return vec_base(s) + 3 * (f - ((kVecs[s].skip >= 0 && f > kVecs[s].skip) ? 1 : 0));
}
static_assert(vec_base(7) == 164 && vec_base(9) == 194, "184/214-D layout");

__device__ __forceinline__ double vec_feature(double x, int kind) {
  if (kind == kVel) return normz(x, -600.0, 600.0);
  if (kind == kRate) return tanh_feat(x * 0.25);
  if (kind == kAcc) return normz(x, -150.0, 150.0);
  return x;
}

// Frame f applied to every vector that uses it (frame-major, so only one frame is live at a time)
template <int F, bool FULL>
__device__ __forceinline__ void emit_frame(float* vec, const double Fm[3][3],
                                           const double (&V)[9][3], int nvec) {
#pragma unroll
  for (int s = 0; s < 9; ++s) {
    if (s >= nvec || kVecs[s].skip == F) continue;
    double comp[3];
    mv3(Fm, V[s], comp);
#pragma unroll
    for (int q = 0; q < 3; ++q)
      put_vec<FULL>(vec, vec_col(s, F) + q, vec_feature(comp[q], kVecs[s].kind));
  }
}

// bank angle of the body y axis about the direction-of-motion frame (obs_reward.py:159-166)
__device__ __forceinline__ void bank_of(const double R[3][3], const double F[3][3], double& s,
                                        double& co) {
  const double by[3] = {R[1][0], R[1][1], R[1][2]};
  const double y1 = F[1][0] * by[0] + F[1][1] * by[1] + F[1][2] * by[2];
  const double y2 = F[2][0] * by[0] + F[2][1] * by[1] + F[2][2] * by[2];
  sc_atan2(y2, y1, s, co);                   // sin, cos of atan2(y2, y1)
}

// The observation row (obs_reward.py:617-723; 214-D: cuda_fdm/external_observation.cu) in two
// parts that read the same inputs: the vector block, columns [50, D - 20), into the tile, and
// the scalar block [0, 50) with the action history.  All lanes of a pair call each part
// together.  The scalar block needs the bank of the own and partner body y axes about their
// motion frames; the vector block forms the own motion frame anyway and hands them over in
// `bank` (bs, bc, tbs, tbc) when given one.  The vector block emits frames [F0, F1) of the six
// (all of them by default; the four-role step gives two waves three frames each).
template <int D, bool FULL, int F0 = 0, int F1 = 6>
__device__ __forceinline__ void obs_vector_block(const Kin9& k, const Peer& p, const Geo& g,
                                                 const ObsIn& own, const ObsOut& out,
                                                 double* bank) {
  static_assert(0 <= F0 && F0 < F1 && F1 <= 6, "frames [F0, F1) of the six");
  constexpr int nvec = D == 214 ? 9 : 7;
  float* o1 = out.tile;
  double V[9][3];
  const bool los_ok = g.dist > 1e-6;
  const double idist = fm_rcp(los_ok ? g.dist : 1.0);
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    V[0][i] = i == 2 ? 1.0 : 0.0;                                  // gravity direction
    V[1][i] = los_ok ? g.delta[i] * idist : 0.0;                  // line of sight
    V[2][i] = k.vn[i];
    V[3][i] = p.vn[i];
    V[4][i] = p.vn[i] - k.vn[i];
    V[7][i] = own.accel[i];
  }
  mtv3(k.A.R, own.pqr, V[5]);                                      // own body rates in NED
#pragma unroll
  for (int i = 0; i < 3; ++i) { V[6][i] = xch(V[5][i]); V[8][i] = xch(own.accel[i]); }
  if constexpr (F0 <= 0 && 0 < F1) {
    const double I3[3][3] = {{1.0, 0.0, 0.0}, {0.0, 1.0, 0.0}, {0.0, 0.0, 1.0}};
    emit_frame<0, FULL>(o1, I3, V, nvec);
  }
  if constexpr (F0 <= 1 && 1 < F1) emit_frame<1, FULL>(o1, k.A.R, V, nvec);
  if constexpr (F0 <= 2 && 2 < F1) emit_frame<2, FULL>(o1, p.R, V, nvec);
  if constexpr (F1 > 3) {
    double Fm[3][3];
    dir_frame(k.vn, Fm);                                           // own motion frame
    if (bank) {
      bank_of(k.A.R, Fm, bank[0], bank[1]);
      bank[2] = xch(bank[0]); bank[3] = xch(bank[1]);
    }
    if constexpr (F0 <= 3) emit_frame<3, FULL>(o1, Fm, V, nvec);
    if constexpr (F0 <= 4 && 4 < F1) {
#pragma unroll
      for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int q = 0; q < 3; ++q) Fm[i][q] = xch(Fm[i][q]);       // partner's motion frame
      emit_frame<4, FULL>(o1, Fm, V, nvec);
    }
    if constexpr (F1 > 5) {
      dir_frame(g.delta, Fm);                                      // line-of-sight frame
      emit_frame<5, FULL>(o1, Fm, V, nvec);
    }
  }
}

// hist: 0 = read the action history from the reconstructor, 1 = already stored (by
// lane_advance), 2 = all zero (a row after an autoreset).  `bank`: the vector block's bank
// values, or null to form them here.
template <int D, bool FULL>
__device__ __forceinline__ void obs_scalar_block(const Kin9& k, const Peer& p, const Geo& g,
                                                 const ObsIn& own, long a, const F16Recon& r,
                                                 const ObsOut& out, int hist,
                                                 const double* bank) {
  const long ld = r.ld;
  constexpr int nvec = D == 214 ? 9 : 7;
  double bs, bc, tbs, tbc;
  if (bank) {
    bs = bank[0]; bc = bank[1]; tbs = bank[2]; tbc = bank[3];
  } else {
    double Fm[3][3];
    dir_frame(k.vn, Fm);
    bank_of(k.A.R, Fm, bs, bc);
    tbs = xch(bs); tbc = xch(bc);
  }
  const bool los_ok = g.dist > 1e-6;
  const double idist = fm_rcp(los_ok ? g.dist : 1.0);
  double V1[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) V1[i] = los_ok ? g.delta[i] * idist : 0.0;
  // ---- scalars [0, 50)
  ObsIn tgt;
  tgt.hp = xch(own.hp); tgt.fuel = xch(own.fuel);
  double pb[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) pb[i] = xch(g.b[i]);
  const double en_ata = xch(g.ata);
  const double own_alt = -k.s9[2], tgt_alt = -p.s9[2];
  const double closure = (k.vn[0] - p.vn[0]) * V1[0] + (k.vn[1] - p.vn[1]) * V1[1] +
                         (k.vn[2] - p.vn[2]) * V1[2];
  // sines and cosines of the line-of-sight angles straight from the unit vectors they are
  // acos'd/atan2'd/asin'd from: ATA = acos(b0); aspect = +-acos(-pb0), signed by the partner's
  // body y; azimuth = atan2(b1, b0); elevation = -asin(b2)
  const double pt1 = -pb[1], pt2 = pb[2];
  const double sgn = pt1 > 0.0 ? 1.0 : (pt1 < 0.0 ? -1.0 : (pt2 >= 0.0 ? 1.0 : -1.0));
  const double cb0 = clampd(g.b[0], -1.0, 1.0), cpb0 = clampd(-pb[0], -1.0, 1.0);
  const double cb2 = clampd(g.b[2], -1.0, 1.0);
  const double s_ata = fm_sqrt((1.0 - cb0) * (1.0 + cb0)), c_ata = cb0;
  const double s_aa = sgn * fm_sqrt((1.0 - cpb0) * (1.0 + cpb0)), c_aa = cpb0;
  double s_az, c_az;
  sc_atan2(g.b[1], g.b[0], s_az, c_az);
  const double s_el = -cb2, c_el = fm_sqrt((1.0 - cb2) * (1.0 + cb2));
  const double u = k.s9[6], v = k.s9[7], w = k.s9[8];
  double aoa = 0.0, ss = 0.0;
  if (!(k.spd < 1.0)) {
    aoa = atan2(w, u) * kR2D;
    ss = atan2(v, fm_sqrt(u * u + w * w)) * kR2D;
  }
  const double e_adv = (own_alt + k.spd * k.spd * (1.0 / (2.0 * kGacc))) -
                       (tgt_alt + p.spd * p.spd * (1.0 / (2.0 * kGacc)));
  const double t = own.t;
  const double cone = t >= 150.0 ? 3.0 : (t >= 100.0 ? 2.0 : 1.0);
  const double maxr_ft = t >= 150.0 ? 4000.0 : (t >= 100.0 ? 3500.0 : 3000.0);
  const double cc = cone > 1e-6 ? cone : 1e-6;
  const double min_r = 500.0 * kFt2M, max_r = maxr_ft * kFt2M;
  double span = max_r - min_r;
  span = span < 1e-6 ? 1e-6 : span;
  double pf_ata = 1.0 - fabs(g.ata) * (1.0 / 30.0);
  pf_ata = pf_ata < 0.0 ? 0.0 : pf_ata;
  double pf_rng = 1.0 - g.dist * (1.0 / 3000.0);
  pf_rng = pf_rng < 0.0 ? 0.0 : pf_rng;
  float sc[kVecCol0];
  int j = 0;
  sc[j++] = obs_value(normz(k.spd, 0.0, 600.0));
  sc[j++] = obs_value(normz(p.spd, 0.0, 600.0));
  sc[j++] = obs_value(tanh_feat(aoa * (1.0 / 30.0)));
  sc[j++] = obs_value(tanh_feat(ss * (1.0 / 15.0)));
  sc[j++] = obs_value(tanh_feat((own_alt - kMinAltM) * (1.0 / 300.0)));
  sc[j++] = obs_value(normz(-k.vn[2], -100.0, 100.0));
  sc[j++] = obs_value(normz(own.hp, 0.0, 1.0));
  sc[j++] = obs_value(normz(tgt.hp, 0.0, 1.0));
  sc[j++] = obs_value(own.hp - tgt.hp);
  sc[j++] = obs_value(fm_div(e_adv, fabs(e_adv) + 5000.0));
  sc[j++] = obs_value(normz(g.dist, 0.0, 2500.0));
  sc[j++] = obs_value(normz(closure, -1000.0, 1000.0));
  sc[j++] = obs_value(s_ata); sc[j++] = obs_value(c_ata);
  sc[j++] = obs_value(s_aa); sc[j++] = obs_value(c_aa);
  sc[j++] = obs_value(s_az); sc[j++] = obs_value(c_az);
  sc[j++] = obs_value(s_el); sc[j++] = obs_value(c_el);
  const double icc = fm_rcp(cc), ispan = fm_rcp(span);
  sc[j++] = obs_value(2.0 * gauss_feat(g.ata * (1.0 / 3.0)) - 1.0);
  sc[j++] = obs_value(tanh_feat((cone - fabs(g.ata)) * icc));
  sc[j++] = obs_value(2.0 * gauss_feat(en_ata * (1.0 / 3.0)) - 1.0);
  sc[j++] = obs_value(tanh_feat((cone - fabs(en_ata)) * icc));
  sc[j++] = obs_value(tanh_feat((g.dist - min_r) * ispan));
  sc[j++] = obs_value(tanh_feat((max_r - g.dist) * ispan));
  sc[j++] = obs_value(normz(t, 0.0, 200.0));
  sc[j++] = obs_value(k.A.sr); sc[j++] = obs_value(k.A.cr);
  sc[j++] = obs_value(k.A.sp); sc[j++] = obs_value(k.A.cp);
  sc[j++] = obs_value(k.A.sy); sc[j++] = obs_value(k.A.cy);
  sc[j++] = obs_value(p.sr); sc[j++] = obs_value(p.cr);
  sc[j++] = obs_value(p.sp); sc[j++] = obs_value(p.cp);
  sc[j++] = obs_value(p.sy); sc[j++] = obs_value(p.cy);
  sc[j++] = obs_value(bs); sc[j++] = obs_value(bc);
  sc[j++] = obs_value(tbs); sc[j++] = obs_value(tbc);
  sc[j++] = obs_value(normz(own.fuel, 0.0, 1.0));
  sc[j++] = obs_value(normz(tgt.fuel, 0.0, 1.0));
  sc[j++] = obs_value(clampd(2.0 * own.dealt - 1.0, -1.0, 1.0));
  sc[j++] = obs_value(clampd(2.0 * own.taken - 1.0, -1.0, 1.0));
  sc[j++] = obs_value(2.0 * (pf_ata * pf_rng) - 1.0);
  sc[j++] = obs_value(normz(own_alt, 0.0, 15000.0));
  sc[j++] = obs_value(normz(tgt_alt, 0.0, 15000.0));
  store_run2<D, FULL, 0, kVecCol0>(out, sc);
  if (hist != 1) {
    float h[kActHist];
#pragma unroll
    for (int i = 0; i < kActHist; ++i) h[i] = hist == 0 ? obs_value(r.act_hist[i * ld + a]) : 0.0f;
    store_run2<D, FULL, vec_base(nvec), kActHist>(out, h);
  }
}

// One observation row to `out` (both blocks).  All lanes of a pair must call it together.
template <int D, bool FULL>
__device__ __forceinline__ void lane_build_obs(const Kin9& k, const Peer& p, const Geo& g,
                                               const ObsIn& own, long a, const F16Recon& r,
                                               const ObsOut& out, int hist = 0) {
  double bank[4];
  obs_vector_block<D, FULL>(k, p, g, own, out, bank);
  obs_scalar_block<D, FULL>(k, p, g, own, a, r, out, hist, bank);
}

// Copy the staged tile rows [0, n) out: the tile is walked as a flat array of n * Wt floats
// (Wt = D for FULL, D - 70 for the vector block), each lane moving W consecutive floats of one
// row per step (W = 4 for FULL 184-D, whose rows are 16-byte aligned, else 2), so every store
// instruction covers 64 * W consecutive floats of the destination (rows a0.. are contiguous
// there when FULL; the vector-block segments are when !FULL).  Rows go to out1 where bit `row`
// of m1 is set and to out2 where bit `row` of m2 is set (wave-uniform masks; out2 may be null).
// Four steps' LDS reads are issued before their stores.  NT threads (tid = 0..NT-1) share the
// copy.
template <int D, bool FULL, int NT = kRowBlock>
__device__ __forceinline__ void flush_tile(const float* S, long a0, int n, uint64_t m1,
                                           float* __restrict__ out1, uint64_t m2,
                                           float* __restrict__ out2, int tid) {
  constexpr int Wt = FULL ? D : D - 70, P = tile_pitch<D, FULL>(), C0 = tile_col0<FULL>();
  constexpr int W = (FULL && D % 4 == 0) ? 4 : 2;
  if (!out2) m2 = 0;
  const int total = n * Wt;
  for (int f0 = 0; f0 < total; f0 += 4 * NT * W) {
    float v[4][W];
    int fl[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int f = f0 + (u * NT + tid) * W;
      fl[u] = f;
      const int row = f / Wt, col = f - row * Wt;
      const float* src = S + (row < kRowBlock ? row : 0) * P + col;
#pragma unroll
      for (int w = 0; w < W; ++w) v[u][w] = src[w];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int f = fl[u];
      if (f < total) {
        const int row = f / Wt, col = f - row * Wt;
        const long off = (a0 + row) * D + C0 + col;
        if constexpr (W == 4) {
          const float4 x = make_float4(v[u][0], v[u][1], v[u][2], v[u][3]);
          if ((m1 >> row) & 1) *reinterpret_cast<float4*>(out1 + off) = x;
          if ((m2 >> row) & 1) *reinterpret_cast<float4*>(out2 + off) = x;
        } else {
          const float2 x = make_float2(v[u][0], v[u][1]);
          if ((m1 >> row) & 1) *reinterpret_cast<float2*>(out1 + off) = x;
          if ((m2 >> row) & 1) *reinterpret_cast<float2*>(out2 + off) = x;
        }
      }
    }
  }
}

// The same for a sparse set of rows (autoreset rows): one row at a time, set bits only.
template <int D, bool FULL, int NT = kRowBlock>
__device__ __forceinline__ void flush_sparse(const float* S, long a0, uint64_t m,
                                             float* __restrict__ out, int tid) {
  constexpr int Wt = FULL ? D : D - 70, P = tile_pitch<D, FULL>(), C0 = tile_col0<FULL>();
  while (m) {
    const int r = __builtin_ctzll(m);
    m &= m - 1;
    const float* src = S + r * P;
#pragma unroll
    for (int c = 2 * tid; c < Wt; c += 2 * NT)
      *reinterpret_cast<float2*>(out + (a0 + r) * D + C0 + c) = make_float2(src[c], src[c + 1]);
  }
}

__device__ __forceinline__ ObsIn load_obs_in(const F16Recon& r, long a, long e) {
  ObsIn o;
  const long ld = r.ld;
  o.hp = r.hp[a]; o.fuel = r.fuel[a]; o.dealt = r.dealt[a]; o.taken = r.taken[a];
  o.t = r.t_sec[e];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    o.pqr[i] = r.pqr[i * ld + a];
    o.accel[i] = r.accel ? r.accel[i * ld + a] : 0.0;
  }
  return o;
}

// ------------------------------------------------------------------------------ kernels
__global__ __launch_bounds__(kObsBlock) void advance_kernel(
    const double* __restrict__ st, long ld, const double* __restrict__ act, F16Recon r,
    F16RewardCfg c, Origin O, double* __restrict__ reward, unsigned char* __restrict__ term,
    unsigned char* __restrict__ trunc) {
  const long a = (long)blockIdx.x * kObsBlock + threadIdx.x;
  if (a >= 2L * r.nenv) return;     // nac is even: both lanes of a pair leave together
  const long e = a >> 1;
  Kin9 k;
  make_kin(st + a, ld, O, k);
  Peer p;
  exchange(k, p);
  Geo g;
  pair_geo(k, p, g);
  const AdvOut o = lane_advance(k, p, g, a, e, act, r, c, st[F16S_FUEL * ld + a]);
  reward[a] = o.reward;
  if (!(a & 1)) { term[e] = o.term; trunc[e] = o.trunc; }
}

__global__ __launch_bounds__(kObsBlock) void init_reward_kernel(
    const double* __restrict__ st, long ld, const unsigned char* __restrict__ mask, F16Recon r,
    Origin O) {
  const long a = (long)blockIdx.x * kObsBlock + threadIdx.x;
  if (a >= 2L * r.nenv) return;
  const long e = a >> 1;
  if (mask && !mask[e]) return;      // per engagement: the pair leaves together
  Kin9 k;
  make_kin(st + a, ld, O, k);
  Peer p;
  exchange(k, p);
  Geo g;
  pair_geo(k, p, g);
  lane_init_reward(k, p, g, a, r.t_sec[e], r);
}

// Future-aux training features of plane 0 (R/cuda_fdm/gen/obs_kernel.cu:348-355; the layout of
// R/cuda_fdm/future_aux.py:1-7), fp64: own NED position [m] and NED velocity [m/s], the
// partner's, own NED-to-body rotation row-major.  Written with the row that becomes the
// engagement's observation.
__device__ __forceinline__ void store_aux(const Kin9& k, const Peer& p, const F16Recon& r, long a) {
  if (!r.aux || (a & 1)) return;
  double* o = r.aux + (a >> 1) * kAuxDim;
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    o[i] = k.s9[i];
    o[3 + i] = k.vn[i];
    o[6 + i] = p.s9[i];
    o[9 + i] = p.vn[i];
#pragma unroll
    for (int j = 0; j < 3; ++j) o[12 + 3 * i + j] = k.A.R[i][j];
  }
}

template <int D, bool FULL>
__global__ __launch_bounds__(kRowBlock) void build_obs_kernel(
    const double* __restrict__ st, long ld, const unsigned char* __restrict__ mask, F16Recon r,
    Origin O, float* __restrict__ obs) {
  __shared__ float S[kRowBlock * tile_pitch<D, FULL>()];
  const int lane = threadIdx.x;
  const long a0 = (long)blockIdx.x * kRowBlock, a = a0 + lane;
  const long nac = 2L * r.nenv;
  const int n = (int)min((long)kRowBlock, nac - a0);
  const long e = a >> 1;
  const bool on = a < nac && (!mask || mask[e]);      // per engagement: pairs agree
  if (on) {
    Kin9 k;
    make_kin(st + a, ld, O, k);
    Peer p;
    exchange(k, p);
    Geo g;
    pair_geo(k, p, g);
    const ObsIn in = load_obs_in(r, a, e);
    lane_build_obs<D, FULL>(k, p, g, in, a, r,
                            ObsOut{S + lane * tile_pitch<D, FULL>(), obs + a * D, nullptr});
    store_aux(k, p, r, a);
  }
  const uint64_t keep = __ballot(on);
  __syncthreads();
  flush_tile<D, FULL>(S, a0, n, keep, obs, 0, nullptr, lane);
}

// Autoreset of this lane's aircraft from the initial-condition pool (rl_env.py:559-577): state
// rows copied in (NaN for a pick outside the pool), reconstructor reset, league opponent redraw,
// and the new state's kinematics, partner exchange, geometry and re-anchored reward state.
// Both lanes of an engagement call it together.
// The pool pair engagement e restarts from: io.pick[e], or floor(pool_size x0 / 2^32) of
// Philox4x32-10 with key = seed and counter = (e, step, 0, 0x5EED5EED).  -1 when out of range.
__device__ __forceinline__ long pool_pick(const F16EnvStepIO& io, long e, uint32_t step) {
  long pk;
  if (io.pick) {
    pk = io.pick[e];
  } else {
    uint32_t ctr[4] = {(uint32_t)e, step, 0u, 0x5EED5EEDu};
    f16rng::philox4x32_10(ctr, (uint32_t)io.seed, (uint32_t)(io.seed >> 32));
    pk = (long)(((uint64_t)ctr[0] * (uint64_t)io.pool_size) >> 32);
  }
  return (pk >= 0 && pk < io.pool_size) ? pk : -1;
}

// The kinematics of the pool row an autoreset copies in (NaN kinematics for a bad pick).
__device__ __forceinline__ void pool_kin(const F16EnvStepIO& io, const Origin& O, long pk,
                                         int odd, Kin9& k2) {
  if (pk >= 0) {
    make_kin(io.ic_pool + (pk * 2 + odd) * F16S_N, 1, O, k2);
  } else {
    const double qnan = __builtin_nan("");
    const double nan14[14] = {qnan, qnan, qnan, qnan, qnan, qnan, qnan,
                              qnan, qnan, qnan, qnan, qnan, qnan, qnan};   // fields 0..13
    make_kin(nan14, 1, O, k2);
  }
}

// The part of an autoreset that does not depend on the new state's geometry: state rows from
// pool row pk (NaN rows for pk < 0), reconstructor reset, league opponent redraw.
__device__ __forceinline__ void lane_reset_rows(const F16EnvStepIO& io, const F16Recon& r,
                                                long a, long e, int odd, uint32_t step, long pk,
                                                bool copy_state = true) {
  double* __restrict__ st = io.states;
  const long ld = io.ld;
  const bool ok = pk >= 0;
  const double* src = io.ic_pool + (ok ? pk * 2 + odd : 0) * F16S_N;
  const double qnan = __builtin_nan("");
  if (!copy_state) {
  } else if (ok) {
    // loads of a chunk before its stores: copied element by element, each load waited for the
    // store before it (the compiler cannot rule out the pool and the state overlapping)
    for (int f0 = 0; f0 < F16S_N; f0 += 17) {
      double v[17];
#pragma unroll
      for (int f = 0; f < 17; ++f) v[f] = f0 + f < F16S_N ? src[f0 + f] : 0.0;
#pragma unroll
      for (int f = 0; f < 17; ++f)
        if (f0 + f < F16S_N) st[(f0 + f) * ld + a] = v[f];
    }
  } else {
    for (int f = 0; f < F16S_N; ++f) st[f * ld + a] = qnan;
  }
  r.hp[a] = 1.0; r.fuel[a] = 1.0;
  r.prev_valid[a] = 0; r.prev_x_valid[a] = 0;
  r.dealt[a] = 0.0; r.taken[a] = 0.0; r.hp_loss[a] = 0.0; r.prev_x[a] = 0.0;
  r.prev_alt_log[a] = 0.0;
  if (io.opp_assign && !odd) {                     // league: draw this engagement's opponent
    uint32_t ctr[4] = {(uint32_t)e, step, 1u, 0x0FF0A55Eu};
    f16rng::philox4x32_10(ctr, (uint32_t)io.seed, (uint32_t)(io.seed >> 32));
    const float u = (float)(ctr[0] >> 8) * 0x1p-24f;
    int kk = io.n_opp - 1;
    for (int q = io.n_opp - 1; q >= 0; --q)
      if (io.opp_cdf[q] > u) kk = q;
    io.opp_assign[e] = kk;
  }
  for (int i = 0; i < 3; ++i) {
    r.prev_att[i * r.ld + a] = 0.0;
    r.pqr[i * r.ld + a] = 0.0;
    if (r.accel) { r.accel[i * r.ld + a] = 0.0; r.prev_vel_ned[i * r.ld + a] = 0.0; }
  }
  for (int i = 0; i < kActHist; ++i) r.act_hist[i * r.ld + a] = 0.0;
  if (!odd) r.t_sec[e] = 0.0;
}

__device__ __forceinline__ void lane_autoreset(const F16EnvStepIO& io, const F16Recon& r,
                                               const Origin& O, long a, long e, int odd,
                                               uint32_t step, Kin9& k2, Peer& p2, Geo& g2) {
  const long pk = pool_pick(io, e, step);
  lane_reset_rows(io, r, a, e, odd, step, pk);
  pool_kin(io, O, pk, odd, k2);
  exchange(k2, p2);
  pair_geo(k2, p2, g2);
  lane_init_reward(k2, p2, g2, a, 0.0, r);
}

// An autoreset from pool row pk >= 0 with the row's re-anchored reward state and aux features
// taken from the pool tables (io.pool_obs set); the state and observation rows are copied
// separately, by the whole group (copy_pool_rows).
__device__ __forceinline__ void lane_autoreset_cached(const F16EnvStepIO& io, const F16Recon& r,
                                                      long a, long e, int odd, uint32_t step,
                                                      long pk) {
  // every pool-table load before the first store (a load after a store to memory the compiler
  // cannot prove distinct waits for the data of every earlier load)
  const double px = io.pool_prev_x[pk * 2 + odd];
  const double pal = io.pool_prev_alt_log[pk * 2 + odd];
  const bool aux = r.aux && !odd;
  double v[kAuxDim];
  if (aux) {
    const double* src = io.pool_aux + pk * kAuxDim;
#pragma unroll
    for (int i = 0; i < kAuxDim; ++i) v[i] = src[i];
  }
  lane_reset_rows(io, r, a, e, odd, step, pk, false);
  r.prev_x[a] = px;
  r.prev_x_valid[a] = 1;
  r.prev_alt_log[a] = pal;
  if (aux) {
    double* o = r.aux + e * kAuxDim;
#pragma unroll
    for (int i = 0; i < kAuxDim; ++i) o[i] = v[i];
  }
}

// The index of the k-th set bit of m (k < popcount(m)).
__device__ __forceinline__ int nth_set_bit(uint64_t m, int k) {
  for (int j = 0; j < k; ++j) m &= m - 1;
  return __builtin_ctzll(m);
}

// State and observation rows of cached autoresets: row r of the group (bit r of m) restarts
// from pool aircraft pick[r] (= 2 pool row + plane).  Every thread of the group takes part: the
// 101 state doubles of all such rows are loaded together (contiguous in the pool) and stored
// into the structure-of-arrays states, then each observation row is copied in 8-byte pieces
// (coalesced).  With the full-row tile the observation rows also go into it, for the
// RunningNorm partial sums that read the tile.
template <int D, bool FULL, int NT>
__device__ __forceinline__ void copy_pool_rows(float* S, long a0, uint64_t m,
                                               const long* pick, const F16EnvStepIO& io,
                                               const float* __restrict__ pool_obs,
                                               float* __restrict__ out, int tid) {
  constexpr int P = tile_pitch<D, FULL>(), kU = 4;
  {
    const int total = __popcll(m) * F16S_N;      // item i: field i % 101 of the (i / 101)-th row
    for (int i0 = tid; i0 < total; i0 += kU * NT) {
      double v[kU];
      int row[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int i = i0 + u * NT;
        row[u] = i < total ? nth_set_bit(m, i / F16S_N) : 0;
        v[u] = i < total ? io.ic_pool[pick[row[u]] * F16S_N + i % F16S_N] : 0.0;
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int i = i0 + u * NT;
        if (i < total) io.states[(long)(i % F16S_N) * io.ld + a0 + row[u]] = v[u];
      }
    }
  }
  while (m) {
    const int r = __builtin_ctzll(m);
    m &= m - 1;
    const float* src = pool_obs + pick[r] * D;
#pragma unroll
    for (int c = 2 * tid; c < D; c += 2 * NT) {
      const float2 x = *reinterpret_cast<const float2*>(src + c);
      *reinterpret_cast<float2*>(out + (a0 + r) * D + c) = x;
      if constexpr (FULL) { S[r * P + c] = x.x; S[r * P + c + 1] = x.y; }
    }
  }
}

__device__ __forceinline__ ObsIn fresh_obs_in() {
  ObsIn f;
  f.hp = 1.0; f.fuel = 1.0; f.dealt = 0.0; f.taken = 0.0; f.t = 0.0;
  for (int i = 0; i < 3; ++i) { f.pqr[i] = 0.0; f.accel[i] = 0.0; }
  return f;
}

template <int D, bool FULL>
__global__ __launch_bounds__(kRowBlock) void env_post_step_kernel(const F16EnvStepIO io,
                                                                   F16Recon r, F16RewardCfg c,
                                                                   Origin O) {
  __shared__ float S[kRowBlock * tile_pitch<D, FULL>()];
  const int lane = threadIdx.x;
  const long a0 = (long)blockIdx.x * kRowBlock, a = a0 + lane;
  const long nac = 2L * r.nenv;
  const int n = (int)min((long)kRowBlock, nac - a0);
  const bool on = a < nac;                              // nac is even: pairs agree
  const uint32_t step = io.step + (io.step_base ? *io.step_base : 0u);
  const long e = a >> 1;
  const int odd = (int)(a & 1);
  double* __restrict__ st = io.states;
  const long ld = io.ld;
  constexpr int kHistCol = vec_base(D == 214 ? 9 : 7);
  float* tile = S + lane * tile_pitch<D, FULL>();
  bool d = false;
  Kin9 k;
  Peer p;
  Geo g;
  AdvOut o;
  if (on) {
    // fields 0..14 (position .. fuel) feed the kinematics and the reward; they are read once
    double f15[15];
#pragma unroll
    for (int f = 0; f < 15; ++f) f15[f] = st[f * ld + a];
    if (io.terminal_finite || io.finite_acc) {   // rl_env.py:545: every state value finite
      int fin = 1;
      if (io.state_finite) {                      // formed by the physics launch
        fin = io.state_finite[a] ? 1 : 0;
      } else {
        // the other 86 fields with all their loads in flight together
#pragma unroll
        for (int f = 0; f < 15; ++f) fin &= isfinite(f15[f]) ? 1 : 0;
        double v[F16S_N - 15];
#pragma unroll
        for (int j = 0; j < F16S_N - 15; ++j) v[j] = st[(15 + j) * ld + a];
#pragma unroll
        for (int j = 0; j < F16S_N - 15; ++j) fin &= isfinite(v[j]) ? 1 : 0;
      }
      fin &= xchi(fin);
      if (!odd) {
        if (io.terminal_finite) io.terminal_finite[e] = (unsigned char)fin;
        if (io.finite_acc && !fin) io.finite_acc[e] = 0;
      }
    }
    make_kin(f15, 1, O, k);
    exchange(k, p);
    pair_geo(k, p, g);
    o = lane_advance(k, p, g, a, e, io.actions, r, c, f15[F16S_FUEL]);
    if (io.reward) io.reward[a] = o.reward;
    if (io.reward_f32) io.reward_f32[a] = (float)o.reward;
    d = o.term || o.trunc;
    if (!odd) {
      if (io.reward0_f32) io.reward0_f32[e] = (float)o.reward;
      if (io.term) io.term[e] = o.term;
      if (io.trunc) io.trunc[e] = o.trunc;
      if (io.done) io.done[e] = d;
      if (io.done_f32) io.done_f32[e] = d ? 1.0f : 0.0f;
    }
    if (io.terminal_hp) io.terminal_hp[a] = o.obs.hp;
    if (io.terminal_alt_m) {
      const double x = f15[0], y = f15[1], z = f15[2];
      io.terminal_alt_m[a] = (fm_sqrt(x * x + y * y + z * z) - kSeaLevelRadiusFtT) * kFt2M;
    }
  }
  if (!io.terminal_obs) {
    // Nobody asks for the finished engagements' terminal rows, so every row is built once:
    // from the step's state for live engagements, from the autoreset state for finished ones.
    if (on && d) {
      lane_autoreset(io, r, O, a, e, odd, step, k, p, g);
      o.obs = fresh_obs_in();
#pragma unroll
      for (int i = 0; i < kActHist; ++i) o.hist[i] = 0.0f;
    }
    if (on) {
      const ObsOut out{tile, io.obs + a * D, nullptr};
      store_run2<D, FULL, kHistCol, kActHist>(out, o.hist);
      lane_build_obs<D, FULL>(k, p, g, o.obs, a, r, out, 1);
      store_aux(k, p, r, a);
    }
    const uint64_t rows = __ballot(on);
    __syncthreads();
    flush_tile<D, FULL>(S, a0, n, rows, io.obs, 0, nullptr, lane);
    return;
  }
  if (on) {
    // terminal observation (rl_env.py:552-554): every row to terminal_obs; the live
    // engagements' rows are also their observation
    const ObsOut out{tile, io.terminal_obs + a * D, d ? nullptr : io.obs + a * D};
    store_run2<D, FULL, kHistCol, kActHist>(out, o.hist);
    lane_build_obs<D, FULL>(k, p, g, o.obs, a, r, out, 1);
    if (!d) store_aux(k, p, r, a);
  }
  const uint64_t rows = __ballot(on), live = __ballot(on && !d), fresh = __ballot(on && d);
  __syncthreads();
  flush_tile<D, FULL>(S, a0, n, rows, io.terminal_obs, live, io.obs, lane);
  if (!fresh) return;      // uniform: no autoreset in this wave
  __syncthreads();
  if (on && d) {
    Kin9 k2;
    Peer p2;
    Geo g2;
    lane_autoreset(io, r, O, a, e, odd, step, k2, p2, g2);
    lane_build_obs<D, FULL>(k2, p2, g2, fresh_obs_in(), a, r,
                            ObsOut{tile, io.obs + a * D, nullptr}, 2);
    store_aux(k2, p2, r, a);
  }
  __syncthreads();
  flush_sparse<D, FULL>(S, a0, fresh, io.obs, lane);
}

// RunningNorm partial sums of a workgroup's 128 new observation rows straight from the full-row
// staging tiles, in norm_partial_kernel's order (policy_kernels.hip): block b = this workgroup,
// four 32-row phases each summed row by row in fp64 (rows past the batch add 0), the phases
// then added in order; block 0 also snapshots and advances the running count.  The results
// equal a norm_partial_kernel launch over the same rows bit for bit.
template <int D, int NT = kPostSplitBlock>
__device__ __forceinline__ void norm_partials_from_tiles(const float* S_all, double* sh,
                                                         long a_blk, long nac, long b,
                                                         const F16EnvStepIO& io, int tid) {
  constexpr int P = tile_pitch<D, true>(), kTile = kRowBlock * P;
  for (int idx = tid; idx < 4 * D; idx += NT) {
    const int ph = idx / D, c = idx - ph * D;
    const float* src = S_all + (ph >> 1) * kTile + ((ph & 1) * 32) * P + c;
    const long r0 = a_blk + ph * 32;
    double sum = 0.0, sq = 0.0;
    for (int i = 0; i < 32; ++i) {
      const double v = (r0 + i < nac) ? (double)src[i * P] : 0.0;
      sum += v;
      sq += v * v;
    }
    sh[(ph * 2) * D + c] = sum;
    sh[(ph * 2 + 1) * D + c] = sq;
  }
  __syncthreads();
  for (int c = tid; c < D; c += NT) {
    double sum = sh[c], sq = sh[D + c];
#pragma unroll
    for (int ph = 1; ph < 4; ++ph) { sum += sh[(ph * 2) * D + c]; sq += sh[(ph * 2 + 1) * D + c]; }
    io.norm_partial[b * 2 * D + c] = sum;
    io.norm_partial[b * 2 * D + D + c] = sq;
  }
  if (b == 0 && tid == 0) {
    const float cnt = *io.norm_count;
    *io.norm_count_snap = cnt;
    *io.norm_count = cnt + (float)nac;
  }
}

// env_post_step with each group of 64 aircraft spread over two wavefronts, two groups per
// 256-thread workgroup (the hardware then places its four wavefronts on the CU's four SIMDs),
// so a 16k-engagement step fills every SIMD instead of half of them.  Wave 0 (advance role) makes
// the reward, termination and reconstructor update, the row's scalar block and action history,
// the aux features and the autoreset rows; wave 1 (vector role) builds the vector block, the
// larger share of a row's arithmetic.  Both evaluate the kinematics and pair geometry (a few
// percent of the work) rather than trade them.  The vector role needs the body rates (and,
// 214-D, the NED acceleration) that the reconstructor update produces: it forms them from the
// previous attitude and velocity, read before the first barrier (after it the advance role
// overwrites them), with lane_advance's expressions, so they are bit-identical.  Rows of
// finished engagements are rebuilt from their autoreset state by the advance role after the
// flush, as the single-wave kernel's terminal path does; without terminal_obs their first
// build is not stored.  Results equal env_post_step_kernel's bit for bit.
template <int D, bool FULL>
struct PostSplitLds {
  float S_all[kPostGroups][kRowBlock * tile_pitch<D, FULL>()];
  uint64_t sh_mask[kPostGroups][3];    // live, finished and pool-table finished rows
  long sh_pick[kPostGroups][kRowBlock];  // pool table row of each pool-table autoreset
  double sh_norm[FULL ? 8 * D : 1];      // RunningNorm partials per phase (full tile)
};

template <int D, bool FULL>
__device__ __forceinline__ void post_split_body(const F16EnvStepIO& io, const F16Recon& r,
                                                const F16RewardCfg& c, const Origin& O,
                                                PostSplitLds<D, FULL>& L) {
  auto& S_all = L.S_all;
  auto& sh_mask = L.sh_mask;
  auto& sh_pick = L.sh_pick;
  auto& sh_norm = L.sh_norm;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int grp = wave >> 1, role = wave & 1;
  const int gtid = (int)(threadIdx.x & (2 * kRowBlock - 1));   // thread index within the group
  float* const S = S_all[grp];
  const long a0 = ((long)blockIdx.x * kPostGroups + grp) * kRowBlock, a = a0 + lane;
  const long nac = 2L * r.nenv;
  const int n = (int)max(0L, min((long)kRowBlock, nac - a0));
  const bool on = a < nac;                              // nac is even: pairs agree
  const long e = a >> 1;
  const int odd = (int)(a & 1);
  const double* __restrict__ st = io.states;
  const long ld = io.ld;
  constexpr int kHistCol = vec_base(D == 214 ? 9 : 7);
  float* tile = S + lane * tile_pitch<D, FULL>();
  float* const first_out = io.terminal_obs ? io.terminal_obs : io.obs;
  Kin9 k;
  Peer p;
  Geo g;
  double f15[15];
  if (role == 0) {
    bool d = false;
    int fin = 1;
    const bool want_fin = on && (io.terminal_finite || io.finite_acc);
    if (on) {
#pragma unroll
      for (int f = 0; f < 15; ++f) f15[f] = st[f * ld + a];
      if (want_fin && io.state_finite) fin = io.state_finite[a] ? 1 : 0;   // the physics launch's
    }
    // the finite flag, kinematics and pair geometry of this role
    auto front = [&]() {
      if (want_fin) {                               // rl_env.py:545: every state value finite
        if (!io.state_finite) {
#pragma unroll
          for (int f = 0; f < 15; ++f) fin &= isfinite(f15[f]) ? 1 : 0;
          double v[F16S_N - 15];
#pragma unroll
          for (int j = 0; j < F16S_N - 15; ++j) v[j] = st[(15 + j) * ld + a];
#pragma unroll
          for (int j = 0; j < F16S_N - 15; ++j) fin &= isfinite(v[j]) ? 1 : 0;
        }
        fin &= xchi(fin);
        if (!odd) {
          if (io.terminal_finite) io.terminal_finite[e] = (unsigned char)fin;
          if (io.finite_acc && !fin) io.finite_acc[e] = 0;
        }
      }
      if (on) {
        make_kin(f15, 1, O, k);
        exchange(k, p);
        pair_geo(k, p, g);
      }
    };
    // Only the vector role's reads of the previous attitude and velocity must precede the
    // barrier below (this role overwrites them after it).  With the full-row tile (one
    // workgroup per CU anyway) this role does its own arithmetic after the barrier, so the
    // vector role, which has the longer share, starts as soon as both roles' loads have landed
    // (3 % shorter launch at 16k engagements); with the vector-block tile, before it, which
    // keeps the register count within two workgroups per CU.
    if constexpr (!FULL) front();
    __syncthreads();   // the vector role has read the previous attitude and velocity
    if constexpr (FULL) front();
    if (on) {
      const AdvOut o = lane_advance(k, p, g, a, e, io.actions, r, c, f15[F16S_FUEL]);
      if (io.reward) io.reward[a] = o.reward;
      if (io.reward_f32) io.reward_f32[a] = (float)o.reward;
      d = o.term || o.trunc;
      if (!odd) {
        if (io.reward0_f32) io.reward0_f32[e] = (float)o.reward;
        if (io.term) io.term[e] = o.term;
        if (io.trunc) io.trunc[e] = o.trunc;
        if (io.done) io.done[e] = d;
        if (io.done_f32) io.done_f32[e] = d ? 1.0f : 0.0f;
      }
      if (io.terminal_hp) io.terminal_hp[a] = o.obs.hp;
      if (io.terminal_alt_m) {
        const double x = f15[0], y = f15[1], z = f15[2];
        io.terminal_alt_m[a] = (fm_sqrt(x * x + y * y + z * z) - kSeaLevelRadiusFtT) * kFt2M;
      }
      const ObsOut out{tile, first_out + a * D,
                       (io.terminal_obs && !d) ? io.obs + a * D : nullptr};
      store_run2<D, FULL, kHistCol, kActHist>(out, o.hist);
      obs_scalar_block<D, FULL>(k, p, g, o.obs, a, r, out, 1, nullptr);
      if (!d) store_aux(k, p, r, a);
    }
    const uint64_t live = __ballot(on && !d), fresh = __ballot(on && d);
    if (lane == 0) { sh_mask[grp][0] = live; sh_mask[grp][1] = fresh; }
  } else {
    bool prev_valid = false;
    double patt[3] = {0.0, 0.0, 0.0}, pvel[3] = {0.0, 0.0, 0.0};
    if (on) {
#pragma unroll
      for (int f = 0; f < 15; ++f) f15[f] = st[f * ld + a];
      make_kin(f15, 1, O, k);
      exchange(k, p);
      pair_geo(k, p, g);
      prev_valid = r.prev_valid[a] != 0;
#pragma unroll
      for (int i = 0; i < 3; ++i) patt[i] = r.prev_att[i * r.ld + a];
      if (r.accel) {
#pragma unroll
        for (int i = 0; i < 3; ++i) pvel[i] = r.prev_vel_ned[i * r.ld + a];
      }
    }
    __syncthreads();   // the advance role may now update the reconstructor
    if (on) {
      ObsIn own = fresh_obs_in();   // only pqr and accel are read by the vector block
      if (prev_valid) {             // lane_advance's body rates and acceleration
        Att P;
        attitude_rpy(patt[0], patt[1], patt[2], P);
        so3_rates(P.R, k.A.R, own.pqr);
      }
      if (r.accel) {
#pragma unroll
        for (int i = 0; i < 3; ++i)
          if (prev_valid) own.accel[i] = (k.vn[i] - pvel[i]) * (1.0 / kDtStep);
      }
      obs_vector_block<D, FULL>(k, p, g, own, ObsOut{tile, nullptr, nullptr}, nullptr);
    }
  }
  __syncthreads();   // the tile holds every row; the masks are published
  const uint64_t rows = __ballot(on), live = sh_mask[grp][0], fresh = sh_mask[grp][1];
  if (io.terminal_obs)
    flush_tile<D, FULL, 2 * kRowBlock>(S, a0, n, rows, io.terminal_obs, live, io.obs, gtid);
  else
    flush_tile<D, FULL, 2 * kRowBlock>(S, a0, n, live, io.obs, 0, nullptr, gtid);
  bool any_fresh = false;   // uniform over the workgroup, so every thread meets the same barriers
#pragma unroll
  for (int q = 0; q < kPostGroups; ++q) any_fresh |= sh_mask[q][1] != 0;
  if (!any_fresh) {
    if constexpr (FULL) {
      if (io.norm_partial)
        norm_partials_from_tiles<D>(&S_all[0][0], sh_norm, (long)blockIdx.x * 2 * kRowBlock, nac,
                                    blockIdx.x, io, threadIdx.x);
    }
    return;
  }
  __syncthreads();
  // Rows of finished engagements.  With the pool tables (io.pool_obs) the advance role restarts
  // them from the pool row with its cached reward anchors and aux features, and the group
  // copies the row's cached observation.  Otherwise (and for a pick outside the pool), split
  // again: the advance role restarts them from the pool (state rows, reconstructor, reward
  // anchor) and writes the scalar block; the vector role forms the same pool row's kinematics
  // from the pool itself and writes the vector block.
  const uint32_t step = io.step + (io.step_base ? *io.step_base : 0u);
  const bool mine = (fresh >> lane) & 1;
  const long pk = mine && io.pool_obs ? pool_pick(io, e, step) : -1;
  const bool cached = pk >= 0;
  const uint64_t from_table = __ballot(cached);    // the same in both roles
  if (mine && cached && role == 0) {
    lane_autoreset_cached(io, r, a, e, odd, step, pk);
    sh_pick[grp][lane] = pk * 2 + odd;
  }
  if (mine && !cached) {
    Kin9 k2;
    Peer p2;
    Geo g2;
    if (role == 0) {
      lane_autoreset(io, r, O, a, e, odd, step, k2, p2, g2);
      obs_scalar_block<D, FULL>(k2, p2, g2, fresh_obs_in(), a, r,
                                ObsOut{tile, io.obs + a * D, nullptr}, 2, nullptr);
      store_aux(k2, p2, r, a);
    } else {
      pool_kin(io, O, pool_pick(io, e, step), odd, k2);
      exchange(k2, p2);
      pair_geo(k2, p2, g2);
      obs_vector_block<D, FULL>(k2, p2, g2, fresh_obs_in(), ObsOut{tile, nullptr, nullptr},
                                nullptr);
    }
  }
  __syncthreads();
  flush_sparse<D, FULL, 2 * kRowBlock>(S, a0, fresh & ~from_table, io.obs, gtid);
  if (from_table)
    copy_pool_rows<D, FULL, 2 * kRowBlock>(S, a0, from_table, sh_pick[grp], io, io.pool_obs,
                                           io.obs, gtid);
  if constexpr (FULL) {   // the tiles now hold every new row, the rebuilt ones included
    if (io.norm_partial) {
      __syncthreads();     // (workgroup-uniform) the copied rows have landed in the tiles
      norm_partials_from_tiles<D>(&S_all[0][0], sh_norm, (long)blockIdx.x * 2 * kRowBlock, nac,
                                  blockIdx.x, io, threadIdx.x);
    }
  }
}

template <int D, bool FULL>
__global__ __launch_bounds__(kPostSplitBlock) void env_post_step_split_kernel(
    const F16EnvStepIO io, F16Recon r, F16RewardCfg c, Origin O) {
  __shared__ PostSplitLds<D, FULL> L;
  post_split_body<D, FULL>(io, r, c, O, L);
}

// The post-physics step of post_split_body (full-row tile) with each group of 64 aircraft on
// four wavefronts instead of two, for the 512-thread one-launch step: role 0 advances (finite
// flag, reward, termination, reconstructor update, action history, aux features), role 1 builds
// the scalar block, roles 2 and 3 the vector block's frames 0-2 and 3-5.  Every role forms the
// kinematics and pair geometry itself; role 1 forms the decision's HP, fuel proxy, damage and
// clock from the same loads with lane_advance's own arithmetic (advance_hp_fuel), and roles 1-3
// read what they need of the reconstructor before the first barrier, after which role 0
// overwrites it.  Groups map roles to waves in opposite orders (a SIMD holds waves w and w + 4),
// so each SIMD pairs the advance role with a vector role and the scalar role with the other.
// Every barrier is at the top level, met by all 512 threads.  Results equal post_split_body's
// bit for bit.
constexpr int kQuadPostBlock = 4 * kRowBlock * kPostGroups;   // 512

template <int D>
__device__ __forceinline__ void post_quad_body(const F16EnvStepIO& io, const F16Recon& r,
                                               const F16RewardCfg& c, const Origin& O,
                                               PostSplitLds<D, true>& L) {
  auto& S_all = L.S_all;
  auto& sh_mask = L.sh_mask;
  auto& sh_pick = L.sh_pick;
  auto& sh_norm = L.sh_norm;
  constexpr int NTG = 4 * kRowBlock;                    // threads per group
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int grp = wave >> 2;
  const int role = grp == 0 ? (wave & 3) : 3 - (wave & 3);
  const int gtid = (int)(threadIdx.x & (NTG - 1));
  float* const S = S_all[grp];
  const long a0 = ((long)blockIdx.x * kPostGroups + grp) * kRowBlock, a = a0 + lane;
  const long nac = 2L * r.nenv;
  const int n = (int)max(0L, min((long)kRowBlock, nac - a0));
  const bool on = a < nac;                              // nac is even: pairs agree
  const long e = a >> 1;
  const int odd = (int)(a & 1);
  const double* __restrict__ st = io.states;
  const long ld = io.ld;
  constexpr int kHistCol = vec_base(D == 214 ? 9 : 7);
  float* tile = S + lane * tile_pitch<D, true>();
  float* const first_out = io.terminal_obs ? io.terminal_obs : io.obs;
  Kin9 k;
  Peer p;
  Geo g;
  double f15[15];
  // ---- reads every role needs before role 0 rewrites the reconstructor
  bool prev_valid = false;
  double patt[3] = {0.0, 0.0, 0.0}, pvel[3] = {0.0, 0.0, 0.0};
  double hp_before = 0.0, fuel_before = 0.0, t_old = 0.0;
  bool d = false;
  int fin = 1;
  const bool want_fin = role == 0 && on && (io.terminal_finite || io.finite_acc);
  if (on) {
#pragma unroll
    for (int f = 0; f < 15; ++f) f15[f] = st[f * ld + a];
    if (role == 0) {
      if (want_fin && io.state_finite) fin = io.state_finite[a] ? 1 : 0;
    } else {
      prev_valid = r.prev_valid[a] != 0;
#pragma unroll
      for (int i = 0; i < 3; ++i) patt[i] = r.prev_att[i * r.ld + a];
      if (role == 1) {
        hp_before = r.hp[a];
        fuel_before = r.fuel[a];
        t_old = r.t_sec[e];
      } else if (r.accel) {
#pragma unroll
        for (int i = 0; i < 3; ++i) pvel[i] = r.prev_vel_ned[i * r.ld + a];
      }
    }
  }
  __syncthreads();   // roles 1-3 have read the previous reconstructor values
  if (role == 0) {
    if (want_fin) {                                 // rl_env.py:545: every state value finite
      if (!io.state_finite) {
#pragma unroll
        for (int f = 0; f < 15; ++f) fin &= isfinite(f15[f]) ? 1 : 0;
        double v[F16S_N - 15];
#pragma unroll
        for (int j = 0; j < F16S_N - 15; ++j) v[j] = st[(15 + j) * ld + a];
#pragma unroll
        for (int j = 0; j < F16S_N - 15; ++j) fin &= isfinite(v[j]) ? 1 : 0;
      }
      fin &= xchi(fin);
      if (!odd) {
        if (io.terminal_finite) io.terminal_finite[e] = (unsigned char)fin;
        if (io.finite_acc && !fin) io.finite_acc[e] = 0;
      }
    }
  }
  if (on) {
    make_kin(f15, 1, O, k);
    exchange(k, p);
    pair_geo(k, p, g);
  }
  if (role == 0) {
    if (on) {
      const AdvOut o = lane_advance(k, p, g, a, e, io.actions, r, c, f15[F16S_FUEL]);
      if (io.reward) io.reward[a] = o.reward;
      if (io.reward_f32) io.reward_f32[a] = (float)o.reward;
      d = o.term || o.trunc;
      if (!odd) {
        if (io.reward0_f32) io.reward0_f32[e] = (float)o.reward;
        if (io.term) io.term[e] = o.term;
        if (io.trunc) io.trunc[e] = o.trunc;
        if (io.done) io.done[e] = d;
        if (io.done_f32) io.done_f32[e] = d ? 1.0f : 0.0f;
      }
      if (io.terminal_hp) io.terminal_hp[a] = o.obs.hp;
      if (io.terminal_alt_m) {
        const double x = f15[0], y = f15[1], z = f15[2];
        io.terminal_alt_m[a] = (fm_sqrt(x * x + y * y + z * z) - kSeaLevelRadiusFtT) * kFt2M;
      }
      const ObsOut out{tile, first_out + a * D, (io.terminal_obs && !d) ? io.obs + a * D : nullptr};
      store_run2<D, true, kHistCol, kActHist>(out, o.hist);
      if (!d) store_aux(k, p, r, a);
    }
    const uint64_t live = __ballot(on && !d), fresh = __ballot(on && d);
    if (lane == 0) { sh_mask[grp][0] = live; sh_mask[grp][1] = fresh; }
  } else if (on) {
    ObsIn own = fresh_obs_in();
    if (role == 1) {                                // what lane_advance forms, formed again
      const HpFuel hf = advance_hp_fuel(k, g, hp_before, fuel_before, t_old);
      own.hp = hf.hp; own.fuel = hf.fuel; own.dealt = hf.dealt; own.taken = hf.taken;
      own.t = hf.t;
      obs_scalar_block<D, true>(k, p, g, own, a, r, ObsOut{tile, nullptr, nullptr}, 1, nullptr);
    } else {
      if (prev_valid) {                             // lane_advance's body rates and acceleration
        Att P;
        attitude_rpy(patt[0], patt[1], patt[2], P);
        so3_rates(P.R, k.A.R, own.pqr);
      }
      if (r.accel) {
#pragma unroll
        for (int i = 0; i < 3; ++i)
          if (prev_valid) own.accel[i] = (k.vn[i] - pvel[i]) * (1.0 / kDtStep);
      }
      if (role == 2)
        obs_vector_block<D, true, 0, 3>(k, p, g, own, ObsOut{tile, nullptr, nullptr}, nullptr);
      else
        obs_vector_block<D, true, 3, 6>(k, p, g, own, ObsOut{tile, nullptr, nullptr}, nullptr);
    }
  }
  __syncthreads();   // the tile holds every row; the masks are published
  const uint64_t rows = __ballot(on), live = sh_mask[grp][0], fresh = sh_mask[grp][1];
  if (io.terminal_obs)
    flush_tile<D, true, NTG>(S, a0, n, rows, io.terminal_obs, live, io.obs, gtid);
  else
    flush_tile<D, true, NTG>(S, a0, n, live, io.obs, 0, nullptr, gtid);
  bool any_fresh = false;   // uniform over the workgroup, so every thread meets the same barriers
#pragma unroll
  for (int q = 0; q < kPostGroups; ++q) any_fresh |= sh_mask[q][1] != 0;
  if (!any_fresh) {
    if (io.norm_partial)
      norm_partials_from_tiles<D, kQuadPostBlock>(&S_all[0][0], sh_norm,
                                                  (long)blockIdx.x * 2 * kRowBlock, nac,
                                                  blockIdx.x, io, threadIdx.x);
    return;
  }
  __syncthreads();
  // Rows of finished engagements: as post_split_body, the scalar block of a rebuilt row on
  // role 1 and its vector block on roles 2 and 3, each from the pool row's kinematics.
  const uint32_t step = io.step + (io.step_base ? *io.step_base : 0u);
  const bool mine = (fresh >> lane) & 1;
  const long pk = mine && io.pool_obs ? pool_pick(io, e, step) : -1;
  const bool cached = pk >= 0;
  const uint64_t from_table = __ballot(cached);    // the same in every role
  if (mine && cached && role == 0) {
    lane_autoreset_cached(io, r, a, e, odd, step, pk);
    sh_pick[grp][lane] = pk * 2 + odd;
  }
  if (mine && !cached) {
    Kin9 k2;
    Peer p2;
    Geo g2;
    if (role == 0) {
      lane_autoreset(io, r, O, a, e, odd, step, k2, p2, g2);
      store_aux(k2, p2, r, a);
    } else {
      pool_kin(io, O, pool_pick(io, e, step), odd, k2);
      exchange(k2, p2);
      pair_geo(k2, p2, g2);
      const ObsOut out{tile, nullptr, nullptr};
      if (role == 1)
        obs_scalar_block<D, true>(k2, p2, g2, fresh_obs_in(), a, r, out, 2, nullptr);
      else if (role == 2)
        obs_vector_block<D, true, 0, 3>(k2, p2, g2, fresh_obs_in(), out, nullptr);
      else
        obs_vector_block<D, true, 3, 6>(k2, p2, g2, fresh_obs_in(), out, nullptr);
    }
  }
  __syncthreads();
  flush_sparse<D, true, NTG>(S, a0, fresh & ~from_table, io.obs, gtid);
  if (from_table)
    copy_pool_rows<D, true, NTG>(S, a0, from_table, sh_pick[grp], io, io.pool_obs, io.obs, gtid);
  if (io.norm_partial) {
    __syncthreads();     // (workgroup-uniform) the copied rows have landed in the tiles
    norm_partials_from_tiles<D, kQuadPostBlock>(&S_all[0][0], sh_norm,
                                                (long)blockIdx.x * 2 * kRowBlock, nac,
                                                blockIdx.x, io, threadIdx.x);
  }
}

// post_quad_body on its own: the post-physics step of f16_env_post_step for batches whose rows
// fit the full-row tile (512-thread workgroups, four wavefronts per 64 aircraft: at 16,384
// engagements two wavefronts on every SIMD where env_post_step_split_kernel has one).  16,384
// engagements of random valid states, the launch alone: 28.7 us against 33.1 us.  Giving
// each role a quarter of the no-flags state scan (86 values that role 0 otherwise reads after
// the first barrier) was measured at 33.4 us and not kept: the loads then sit before the barrier
// on every role.
template <int D>
__global__ __launch_bounds__(kQuadPostBlock) void env_post_step_quad_kernel(
    const F16EnvStepIO io, F16Recon r, F16RewardCfg c, Origin O) {
  __shared__ PostSplitLds<D, true> L;
  post_quad_body<D>(io, r, c, O, L);
}

// A whole environment step in one launch, for batches whose rows fit the full-row tile: the
// workgroup first runs the FDM substeps of its 128 aircraft as fdm_step_split_kernel does (two
// wavefronts per 64 aircraft, model image and exchange fields in LDS), then, after a workgroup
// barrier, the post-physics step of env_post_step_split_kernel over the same 128 aircraft (its
// groups and roles are the FDM's pairs and roles: aircraft (2 blockIdx.x + wave / 2) * 64 + lane
// in both).  Every value the post-physics step reads of the new states, the per-aircraft finite
// flags and the kept actions was written by this workgroup before that barrier, which also makes
// the two phases' LDS (a union) safe to reuse.  Results equal the two launches bit for bit; the
// second launch's start-up, its wait for the last FDM workgroup and the write-back of the states
// at the kernel boundary are saved.  `act`: the controls read by the physics (io.actions is
// what the post-physics step reads, written from `act` when `act_keep` is set);
// `state_finite`: (nac) bytes, written by the physics and read back as io.state_finite.
template <int D>
union EnvStepLds {
  struct {
    double T[F16M_IMAGE_LEN];
    f16::SplitX X[f16::kSplitPairs];
  } fdm;
  PostSplitLds<D, true> post;
};
static_assert(f16::kSplitBlock == kPostSplitBlock && f16::kSplitAircraft == kPostGroups * kRowBlock,
              "the FDM pairs and the post-physics groups must cover the same aircraft");

template <int FCS_RATE, int D>
__global__ __launch_bounds__(kPostSplitBlock) void env_step_fused_kernel(
    const double* __restrict__ act, int S, double* act_keep,
    unsigned char* state_finite, const F16EnvStepIO io, F16Recon r, F16RewardCfg c,
    Origin O) {
  __shared__ EnvStepLds<D> L;
  f16::stage_image<kPostSplitBlock>(L.fdm.T);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int pair = wave >> 1;
  const int nac = 2 * r.nenv;
  const int i = blockIdx.x * f16::kSplitAircraft + pair * 64 + lane;
  const bool store = i < nac;
  const int ia = store ? i : nac - 1;   // lanes past the batch shadow the last aircraft
  if ((wave & 1) == 0)
    f16::split_flight<FCS_RATE>(io.states + ia, io.ld, S, store, nullptr, 0, L.fdm.T,
                                L.fdm.X[pair], lane, true);
  else
    f16::split_systems<FCS_RATE>(io.states + ia, io.ld, act + 4L * ia, S, store, L.fdm.T,
                                 L.fdm.X[pair], lane, state_finite + ia,
                                 act_keep ? act_keep + 4L * ia : nullptr);
  __syncthreads();   // the new states, finite flags and actions are written; LDS is free
  post_split_body<D, true>(io, r, c, O, L.post);
}

// The same step on 512-thread workgroups: each 64 aircraft on four wavefronts in both phases
// (fdm_quad.h's four physics roles, then post_quad_body's four post-physics roles), so that at
// 16,384 engagements every SIMD holds two wavefronts instead of one.  Results equal
// env_step_fused_kernel's bit for bit.
template <int D>
union EnvQuadLds {
  struct {
    double T[F16M_IMAGE_LEN];
    f16::QuadX X[f16::kQuadGroups];
  } fdm;
  PostSplitLds<D, true> post;
};
static_assert(f16::kQuadBlock == kQuadPostBlock && f16::kQuadAircraft == kPostGroups * kRowBlock,
              "the four-role physics groups and post-physics groups must cover the same aircraft");

template <int FCS_RATE, int D>
__global__ __launch_bounds__(kQuadPostBlock) void env_step_quad_kernel(
    const double* __restrict__ act, int S, double* act_keep,
    unsigned char* state_finite, const F16EnvStepIO io, F16Recon r, F16RewardCfg c,
    Origin O) {
  __shared__ EnvQuadLds<D> L;
  f16::stage_image<kQuadPostBlock>(L.fdm.T);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int grp = wave >> 2;
  const int role = f16::quad_role(grp, wave & 3);
  const int nac = 2 * r.nenv;
  const int i = blockIdx.x * f16::kQuadAircraft + grp * 64 + lane;
  const bool store = i < nac;
  const int ia = store ? i : nac - 1;   // lanes past the batch shadow the last aircraft
  double* const st = io.states + ia;
  // (two groups per workgroup: the physics roles run with their phase priorities, fdm_quad.h)
  if (role == f16::kRoleKin)
    f16::quad_kin<FCS_RATE, true>(st, io.ld, S, store, nullptr, 0, L.fdm.T, L.fdm.X[grp], lane,
                                  true);
  else if (role == f16::kRoleAero)
    f16::quad_aero<FCS_RATE, true>(S, L.fdm.T, L.fdm.X[grp], lane, true);
  else if (role == f16::kRoleFcs)
    f16::quad_fcs<FCS_RATE, true>(st, io.ld, act + 4L * ia, S, store, L.fdm.T, L.fdm.X[grp],
                                  lane, true, act_keep ? act_keep + 4L * ia : nullptr);
  else
    f16::quad_air<FCS_RATE, true>(st, io.ld, act + 4L * ia, S, store, L.fdm.T, L.fdm.X[grp],
                                  lane, state_finite + ia);
  __syncthreads();   // the new states, finite flags and actions are written; LDS is free
  post_quad_body<D>(io, r, c, O, L.post);
}

// Masked autoreset without a step: engagements with mask[e] != 0 get an initial-condition pool
// row (io.pick or the in-kernel Philox draw), the reconstructor reset and the reward state
// re-anchored -- the departure reseeding of the staggered warm-up (rl_env.py:386-434) on the
// device.  No observation is built (the warm-up builds them once at its end).
__global__ __launch_bounds__(kRowBlock) void reseed_kernel(const F16EnvStepIO io, F16Recon r,
                                                           const unsigned char* __restrict__ mask,
                                                           Origin O) {
  const long a = (long)blockIdx.x * kRowBlock + threadIdx.x;
  const long nac = 2L * r.nenv;
  const long e = a >> 1;
  if (a >= nac || !mask[e]) return;              // pairs agree: the exchanges stay paired
  const uint32_t step = io.step + (io.step_base ? *io.step_base : 0u);
  Kin9 k;
  Peer p;
  Geo g;
  lane_autoreset(io, r, O, a, e, (int)(a & 1), step, k, p, g);
}

// rl_env.py:583-592 state9_flat: (nac, 9) float64 rows N/E/D m, roll/pitch/yaw deg, u/v/w m/s
__global__ __launch_bounds__(kObsBlock) void state9_kernel(const double* __restrict__ st, long ld,
                                                            int nac, Origin O,
                                                            double* __restrict__ out) {
  const long a = (long)blockIdx.x * kObsBlock + threadIdx.x;
  if (a >= nac) return;
  double s9[9];
  state9(st + a, ld, O, s9);
#pragma unroll
  for (int i = 0; i < 9; ++i) out[a * 9 + i] = s9[i];
}

// ------------------------------------------------------------------------------ host side
static Origin make_origin() {
  // official BaseLat/BaseLon (cuda_fdm/obs_reward.py:376-384), same expressions as the checker
  const double la = 37.240778 * kD2R, lo = 131.869556 * kD2R;
  Origin O;
  O.slat = sin(la); O.clat = cos(la); O.slon = sin(lo); O.clon = cos(lo);
  const double N = kWgsA / sqrt(1.0 - kWgsE2 * O.slat * O.slat);
  O.ox = (N + 0.0) * O.clat * O.clon;
  O.oy = (N + 0.0) * O.clat * O.slon;
  O.oz = (N * (1.0 - kWgsE2) + 0.0) * O.slat;
  O.b = kWgsA * sqrt(1.0 - kWgsE2);
  O.ep2 = (kWgsA * kWgsA - O.b * O.b) / (O.b * O.b);
  return O;
}

static const Origin& origin() {
  static const Origin O = make_origin();
  return O;
}

static int check_recon(const F16Recon* r, bool need_accel) {
  if (!r || r->nenv < 0) return F16_EINVAL;
  if (r->nenv == 0) return 0;
  if ((long)r->nenv * 2 > 0x7fffffffL || r->ld < 2L * r->nenv) return F16_EINVAL;
  if (!r->hp || !r->fuel || !r->t_sec || !r->prev_att || !r->prev_valid || !r->pqr || !r->dealt ||
      !r->taken || !r->hp_loss || !r->act_hist || !r->prev_x || !r->prev_x_valid ||
      !r->prev_alt_log)
    return F16_EINVAL;
  if ((r->accel == nullptr) != (r->prev_vel_ned == nullptr)) return F16_EINVAL;
  if (need_accel && !r->accel) return F16_EINVAL;
  return 0;
}

// Observation matrices are written 16 bytes (184-D) or 8 bytes (214-D) per lane and step.
static bool rows_aligned(const float* p, int obs_dim) {
  return ((uintptr_t)p & (obs_dim % 4 == 0 ? 15u : 7u)) == 0;
}

// Whether a row launch over nenv engagements keeps every workgroup resident at once with the
// full-row tile (limited by LDS per CU); otherwise the vector-block tile is used, which lets
// four wavefronts share a CU.  `groups`: 64-row tiles per workgroup.
static bool full_tile_resident(int nenv, int obs_dim, int groups = 1) {
  static int cus = 0, lds = 0;
  if (cus == 0) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    (void)hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev);
    if (cus <= 0) cus = 256;
    if (lds <= 0) lds = 160 * 1024;
  }
  const long rows = (long)kRowBlock * groups;
  const long blocks = (2L * nenv + rows - 1) / rows;
  const long tile = rows * (obs_dim | 1) * (long)sizeof(float);
  return blocks <= (long)(lds / tile) * cus;
}

static int check_cfg(const F16RewardCfg* c) {
  if (!c || c->mode < 0 || c->mode > 3) return F16_EINVAL;
  return 0;
}

static dim3 grid_for(int nenv) {
  return dim3((unsigned)((2L * nenv + kObsBlock - 1) / kObsBlock));
}

static dim3 grid_rows(int nenv) {
  return dim3((unsigned)((2L * nenv + kRowBlock - 1) / kRowBlock));
}

static dim3 grid_groups(int nenv) {
  constexpr long rows = (long)kRowBlock * kPostGroups;
  return dim3((unsigned)((2L * nenv + rows - 1) / rows));
}

}  // namespace f16obs

using namespace f16obs;

extern "C" int f16_obr_advance(const double* states, long ld, const double* actions,
                               const F16Recon* rec, const F16RewardCfg* cfg, double* reward,
                               unsigned char* term, unsigned char* trunc, void* stream) {
  int rc = check_recon(rec, false);
  if (rc) return rc;
  if ((rc = check_cfg(cfg))) return rc;
  if (rec->nenv == 0) return 0;
  if (!states || !actions || !reward || !term || !trunc || ld < 2L * rec->nenv) return F16_EINVAL;
  hipLaunchKernelGGL(advance_kernel, grid_for(rec->nenv), dim3(kObsBlock), 0,
                     (hipStream_t)stream, states, ld, actions, *rec, *cfg, origin(), reward,
                     term, trunc);
  return f16_last_error();
}

extern "C" int f16_obr_init_reward(const double* states, long ld, const unsigned char* env_mask,
                                   const F16Recon* rec, void* stream) {
  int rc = check_recon(rec, false);
  if (rc) return rc;
  if (rec->nenv == 0) return 0;
  if (!states || ld < 2L * rec->nenv) return F16_EINVAL;
  hipLaunchKernelGGL(init_reward_kernel, grid_for(rec->nenv), dim3(kObsBlock), 0,
                     (hipStream_t)stream, states, ld, env_mask, *rec, origin());
  return f16_last_error();
}

extern "C" int f16_obr_build_obs(const double* states, long ld, const unsigned char* env_mask,
                                 const F16Recon* rec, int obs_dim, float* obs, void* stream) {
  if (obs_dim != 184 && obs_dim != 214) return F16_EINVAL;
  int rc = check_recon(rec, obs_dim == 214);
  if (rc) return rc;
  if (rec->nenv == 0) return 0;
  if (!states || !obs || ld < 2L * rec->nenv) return F16_EINVAL;
  if (!rows_aligned(obs, obs_dim)) return F16_EINVAL;
  const bool full = full_tile_resident(rec->nenv, obs_dim);
  hipStream_t s = (hipStream_t)stream;
#define F16_BUILD_OBS(D, FULL)                                                                  \
  hipLaunchKernelGGL((build_obs_kernel<D, FULL>), grid_rows(rec->nenv), dim3(kRowBlock), 0, s,   \
                     states, ld, env_mask, *rec, origin(), obs)
  if (obs_dim == 184) {
    if (full) F16_BUILD_OBS(184, true); else F16_BUILD_OBS(184, false);
  } else {
    if (full) F16_BUILD_OBS(214, true); else F16_BUILD_OBS(214, false);
  }
#undef F16_BUILD_OBS
  return f16_last_error();
}

// Arguments of a post-physics step: 0 when valid, 1 when there is nothing to do (nenv == 0),
// else the error code.  *full: whether the launch uses the full-row tile.
static int post_step_args(const F16EnvStepIO* io, const F16Recon* rec, const F16RewardCfg* cfg,
                          bool split, bool* full) {
  if (!io) return F16_EINVAL;
  if (io->obs_dim != 184 && io->obs_dim != 214) return F16_EINVAL;
  int rc = check_recon(rec, io->obs_dim == 214);
  if (rc) return rc;
  if ((rc = check_cfg(cfg))) return rc;
  if (rec->nenv == 0) return 1;
  if (!io->states || !io->actions || !io->obs || !io->ic_pool || io->pool_size < 1 ||
      io->pool_size > 0xffffffffL || io->ld < 2L * rec->nenv || rec->ld != io->ld)
    return F16_EINVAL;
  if (io->opp_assign && (!io->opp_cdf || io->n_opp < 1)) return F16_EINVAL;
  if (!rows_aligned(io->obs, io->obs_dim) ||
      (io->terminal_obs && !rows_aligned(io->terminal_obs, io->obs_dim)))
    return F16_EINVAL;
  *full = full_tile_resident(rec->nenv, io->obs_dim, split ? kPostGroups : 1);
  if (io->norm_partial && (!split || !*full || !io->norm_count || !io->norm_count_snap))
    return F16_EINVAL;
  return 0;
}

static int post_step_launch(const F16EnvStepIO* io, const F16Recon* rec, const F16RewardCfg* cfg,
                            void* stream, bool split, bool full) {
  hipStream_t s = (hipStream_t)stream;
#define F16_POST_STEP(D, FULL)                                                                  \
  do {                                                                                          \
    if (split && FULL)                                                                          \
      hipLaunchKernelGGL((env_post_step_quad_kernel<D>), grid_groups(rec->nenv),                \
                         dim3(kQuadPostBlock), 0, s, *io, *rec, *cfg, origin());                \
    else if (split)                                                                             \
      hipLaunchKernelGGL((env_post_step_split_kernel<D, false>), grid_groups(rec->nenv),        \
                         dim3(kPostSplitBlock), 0, s, *io, *rec, *cfg, origin());               \
    else                                                                                        \
      hipLaunchKernelGGL((env_post_step_kernel<D, FULL>), grid_rows(rec->nenv), dim3(kRowBlock), \
                         0, s, *io, *rec, *cfg, origin());                                      \
  } while (0)
  if (io->obs_dim == 184) {
    if (full) F16_POST_STEP(184, true); else F16_POST_STEP(184, false);
  } else {
    if (full) F16_POST_STEP(214, true); else F16_POST_STEP(214, false);
  }
#undef F16_POST_STEP
  return f16_last_error();
}

static int post_step(const F16EnvStepIO* io, const F16Recon* rec, const F16RewardCfg* cfg,
                     void* stream, bool split) {
  bool full = false;
  const int rc = post_step_args(io, rec, cfg, split, &full);
  if (rc) return rc < 0 ? rc : 0;
  return post_step_launch(io, rec, cfg, stream, split, full);
}

extern "C" int f16_env_post_step(const F16EnvStepIO* io, const F16Recon* rec,
                                 const F16RewardCfg* cfg, void* stream) {
  return post_step(io, rec, cfg, stream, true);
}

static int env_step(const F16EnvStepIO* io, const F16Recon* rec, const F16RewardCfg* cfg,
                    const double* actions, int substeps, int fcs_rate, unsigned char* state_finite,
                    void* stream, bool quad) {
  if (!io || !state_finite || substeps < 1) return F16_EINVAL;
  if (fcs_rate != 120 && fcs_rate != 60) return F16_ERATE;
  F16EnvStepIO x = *io;
  x.state_finite = state_finite;
  bool full = false;
  int rc = post_step_args(&x, rec, cfg, true, &full);
  if (rc) return rc < 0 ? rc : 0;
  if (2L * rec->nenv > 0x7fffffffL) return F16_EINVAL;
  const int nac = 2 * rec->nenv;
  const double* act = actions ? actions : io->actions;
  double* keep = act != io->actions ? const_cast<double*>(io->actions) : nullptr;
  if (keep) {   // the physics reads `actions` and writes io->actions as separate arrays
    const uintptr_t a0 = (uintptr_t)act, k0 = (uintptr_t)keep;
    const uintptr_t bytes = (uintptr_t)nac * 4 * sizeof(double);
    if (a0 < k0 + bytes && k0 < a0 + bytes) return F16_EINVAL;
  }
  if (!full) {
    rc = keep ? f16_fdm_step_batch_keep(x.states, x.ld, act, keep, nac, substeps, fcs_rate,
                                        nullptr, 0, state_finite, stream)
              : f16_fdm_step_batch_finite(x.states, x.ld, act, nac, substeps, fcs_rate, nullptr,
                                          0, state_finite, stream);
    if (rc) return rc;
    return post_step_launch(&x, rec, cfg, stream, true, false);
  }
  hipStream_t s = (hipStream_t)stream;
#define F16_ENV_STEP(R, D)                                                                      \
  do {                                                                                          \
    if (quad)                                                                                   \
      hipLaunchKernelGGL((env_step_quad_kernel<R, D>), grid_groups(rec->nenv),                  \
                         dim3(kQuadPostBlock), 0, s, act, substeps, keep, state_finite, x, *rec,\
                         *cfg, origin());                                                       \
    else                                                                                        \
      hipLaunchKernelGGL((env_step_fused_kernel<R, D>), grid_groups(rec->nenv),                 \
                         dim3(kPostSplitBlock), 0, s, act, substeps, keep, state_finite, x,     \
                         *rec, *cfg, origin());                                                 \
  } while (0)
  if (fcs_rate == 120) {
    if (x.obs_dim == 184) F16_ENV_STEP(120, 184); else F16_ENV_STEP(120, 214);
  } else {
    if (x.obs_dim == 184) F16_ENV_STEP(60, 184); else F16_ENV_STEP(60, 214);
  }
#undef F16_ENV_STEP
  return f16_last_error();
}

extern "C" int f16_env_step(const F16EnvStepIO* io, const F16Recon* rec, const F16RewardCfg* cfg,
                            const double* actions, int substeps, int fcs_rate,
                            unsigned char* state_finite, void* stream) {
  return env_step(io, rec, cfg, actions, substeps, fcs_rate, state_finite, stream, true);
}

extern "C" int f16_env_step_tworole(const F16EnvStepIO* io, const F16Recon* rec,
                                    const F16RewardCfg* cfg, const double* actions, int substeps,
                                    int fcs_rate, unsigned char* state_finite, void* stream) {
  return env_step(io, rec, cfg, actions, substeps, fcs_rate, state_finite, stream, false);
}

extern "C" int f16_env_post_step_norm_fusable(int nenv, int obs_dim) {
  if (nenv < 1 || (obs_dim != 184 && obs_dim != 214)) return 0;
  return full_tile_resident(nenv, obs_dim, kPostGroups) ? 1 : 0;
}

extern "C" int f16_env_post_step_onewave(const F16EnvStepIO* io, const F16Recon* rec,
                                         const F16RewardCfg* cfg, void* stream) {
  return post_step(io, rec, cfg, stream, false);
}

extern "C" int f16_env_reseed(const F16EnvStepIO* io, const F16Recon* rec,
                              const unsigned char* mask, void* stream) {
  if (!io || !mask) return F16_EINVAL;
  int rc = check_recon(rec, io->obs_dim == 214);
  if (rc) return rc;
  if (rec->nenv == 0) return 0;
  if (!io->states || !io->ic_pool || io->pool_size < 1 || io->pool_size > 0xffffffffL ||
      io->ld < 2L * rec->nenv || rec->ld != io->ld)
    return F16_EINVAL;
  if (io->opp_assign && (!io->opp_cdf || io->n_opp < 1)) return F16_EINVAL;
  hipLaunchKernelGGL(reseed_kernel, grid_rows(rec->nenv), dim3(kRowBlock), 0, (hipStream_t)stream,
                     *io, *rec, mask, origin());
  return f16_last_error();
}

extern "C" int f16_state9(const double* states, long ld, int nac, double* s9, void* stream) {
  if (nac < 0 || ld < nac) return F16_EINVAL;
  if (nac == 0) return 0;
  if (!states || !s9) return F16_EINVAL;
  hipLaunchKernelGGL(state9_kernel, dim3((unsigned)((nac + kObsBlock - 1) / kObsBlock)),
                     dim3(kObsBlock), 0, (hipStream_t)stream, states, ld, nac, origin(), s9);
  return f16_last_error();
}

// ---- build_future_labels (R/cuda_fdm/future_aux.py:29-55): one lane per engagement walks the
// rollout; episode ids are the running count of episode starts, a horizon is valid when no
// start falls in (t, t + h].
namespace f16obs {
constexpr int kAuxOppH = 5, kAuxSelfH = 10;
constexpr double kAuxPosScaleM = 100.0;

__global__ __launch_bounds__(256) void future_labels_kernel(const double* __restrict__ f,
                                                            const float* __restrict__ starts,
                                                            int T, int nenv, double dt,
                                                            float* __restrict__ labels,
                                                            unsigned char* __restrict__ mask) {
  const long e = (long)blockIdx.x * 256 + threadIdx.x;
  if (e >= nenv) return;
  long eid_t = 0;                                  // episode id at t (starts[0..t] counted)
  for (int t = 0; t < T; ++t) {
    eid_t += (long)starts[(long)t * nenv + e];     // torch: episode_starts.to(int64).cumsum(0)
    const double* ft = f + ((long)t * nenv + e) * kAuxDim;
    for (int slot = 0; slot < 2; ++slot) {
      const int h = slot == 0 ? kAuxOppH : kAuxSelfH;
      const int pos = slot == 0 ? 6 : 0, vel = slot == 0 ? 9 : 3;
      float out[3] = {0.0f, 0.0f, 0.0f};
      unsigned char ok = 0;
      if (t + h < T) {
        long eid_h = eid_t;
        for (int s2 = t + 1; s2 <= t + h; ++s2) eid_h += (long)starts[(long)s2 * nenv + e];
        if (eid_h == eid_t) {
          const double* fh = f + ((long)(t + h) * nenv + e) * kAuxDim;
          double res[3];
          for (int i = 0; i < 3; ++i)
            res[i] = (fh[pos + i] - ft[pos + i]) - ft[vel + i] * ((double)h * dt);
          for (int i = 0; i < 3; ++i) {
            const double* R = ft + 12 + 3 * i;
            out[i] = (float)((R[0] * res[0] + R[1] * res[1] + R[2] * res[2]) / kAuxPosScaleM);
          }
          ok = 1;
        }
      }
      float* L = labels + ((long)t * nenv + e) * 6 + 3 * slot;
      for (int i = 0; i < 3; ++i) L[i] = out[i];
      mask[((long)t * nenv + e) * 2 + slot] = ok;
    }
  }
}
}  // namespace f16obs

extern "C" int f16_future_labels(const double* features, const float* starts, int T, int nenv,
                                 double dt, float* labels, unsigned char* mask, void* stream) {
  if (T < 0 || nenv < 0 || !(dt > 0.0)) return F16_EINVAL;
  if (T == 0 || nenv == 0) return 0;
  if (!features || !starts || !labels || !mask) return F16_EINVAL;
  hipLaunchKernelGGL(f16obs::future_labels_kernel, dim3((nenv + 255) / 256), dim3(256), 0,
                     (hipStream_t)stream, features, starts, T, nenv, dt, labels, mask);
  return f16_last_error();
}
