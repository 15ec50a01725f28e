/* f16_state.h -- layout of the per-aircraft integrator state and of the 17-value FDM output.
 *
 * The state is the reference's FdmState (cuda_fdm/gen/fdm.cuh:519-528), 101 doubles in the
 * order of cuda_fdm/ic.py:92-114.  On the device it is stored structure-of-arrays: field k of
 * aircraft a lives at states[k * ld + a], so a wavefront's 64 lanes touch 512 contiguous bytes
 * per field.  The Python view exposes it as the (nac, 101) row-major tensor the reference
 * hands around (a transposed view of the same memory).
 */
#ifndef F16_STATE_H
#define F16_STATE_H

#define F16S_POS 0          /* ECI position, ft (3) */
#define F16S_VEL 3          /* ECI velocity, ft/s (3) */
#define F16S_Q 6            /* attitude quaternion ECI->body (4) */
#define F16S_PQRI 10        /* inertial body rates vPQRi, rad/s (3) */
#define F16S_EPA 13         /* Earth position angle, rad */
#define F16S_FUEL 14        /* total fuel, lb */
#define F16S_UVWIDOT 15     /* ECI acceleration for the velocity integrator (3) */
#define F16S_PQRIDOT 18     /* body angular acceleration (3) */
#define F16S_QDOT 21        /* quaternion derivative (4) */
#define F16S_DQ 25          /* history of QDOT, newest first (3 x 4) */
#define F16S_DPQRI 37       /* history of PQRIDOT (3 x 3) */
#define F16S_DIVEL 46       /* history of VEL (3 x 3) */
#define F16S_DUVW 55        /* history of UVWIDOT (3 x 3) */
#define F16S_PBA 64         /* previous-frame body acceleration (3) */
#define F16S_PPQRIDOT 67    /* previous-frame angular acceleration (3) */
#define F16S_PPQRI 70       /* previous-frame vPQRi (3) */
#define F16S_PAUX 73        /* previous-frame alpha, mach, vc_kts, vg_fps, n_py, n_pz, p, q, r */
#define F16S_ENG 82         /* N1, N2, N2norm, FuelFlow_pph */
#define F16S_KIN 86         /* FCS kinematic outputs: tef, aileron, elevator, rudder, gear, lef */
#define F16S_PID 92         /* PIDs roll, g-load, yaw x (input_prev, input_prev2, i_out_total) */
#define F16S_N 101

/* FDM output row (cuda_fdm/gpu_env.py:19-22): eci_pos, eci_vel, euler, vUVW, alpha, beta,
 * mach, Vt, alt_asl */
#define F16O_N 17

/* IC row consumed by the seeding kernel:
 * lat_deg, lon_deg, alt_ft, vt_fps, phi_deg, theta_deg, psi_deg, alpha_deg, beta_deg, fuel_lbs */
#define F16IC_N 10

#endif /* F16_STATE_H */
