/*
 * policy_oracle.c -- CPU checker of the policy step's categorical draw.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ to check the HIP policy kernel.
 *
 * The reference draws each of the 4 action channels from torch.distributions.Categorical over
 * 21 logits (research/competition_36500/runtime/claude_code/model.py:195-233,
 * cuda_fdm/ppo_gpu.py:266-276) with torch's generator; this build's draw is specified instead as
 * an inverse-CDF lookup at a Philox4x32-10 uniform (same distribution, its own stream):
 *   m = max_k l_k (fmaxf, k ascending);  e_k = exp(l_k - m) (IEEE-only exp below);  s = sum_k e_k
 *   (k ascending)
 *   x0 = Philox4x32-10(counter = (row, step, channel, salt), key = (seed_lo, seed_hi))[0]
 *   u = (x0 >> 8) 2^-24;  idx = first k with e_0 + ... + e_k > u s (else 20)
 *   logp = sum over channels of (l_idx - m) - log(s)
 * Philox4x32-10 is restated from Salmon et al., SC 2011 (Random123), and pinned by its published
 * known-answer vectors in tests/test_policy.py.
 */
#include <math.h>
#include <stdint.h>

void orc_philox4x32_10(uint32_t ctr[4], uint32_t k0, uint32_t k1)
{
    for (int round = 0; round < 10; round++) {
        uint64_t a = (uint64_t)0xD2511F53u * ctr[0];
        uint64_t b = (uint64_t)0xCD9E8D57u * ctr[2];
        uint32_t x0 = (uint32_t)(b >> 32) ^ ctr[1] ^ k0;
        uint32_t x1 = (uint32_t)b;
        uint32_t x2 = (uint32_t)(a >> 32) ^ ctr[3] ^ k1;
        uint32_t x3 = (uint32_t)a;
        ctr[0] = x0; ctr[1] = x1; ctr[2] = x2; ctr[3] = x3;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
}

/* e^x, x <= 0: Cody-Waite reduction with a 16-bit head of ln 2 and Taylor degree 7, each step
   one fused multiply-add (fmaf is exactly rounded, so the GPU's v_fma_f32 sequence matches) */
static float exp_nonpos(float x)
{
    if (!(x >= -87.0f)) return 0.0f;
    float n = rintf(x * 1.44269504f);
    float r = fmaf(-n, 1.42860677e-6f, fmaf(-n, 0.693145751953125f, x));
    float p = fmaf(1.0f / 5040.0f, r, 1.0f / 720.0f);
    p = fmaf(p, r, 1.0f / 120.0f);
    p = fmaf(p, r, 1.0f / 24.0f);
    p = fmaf(p, r, 1.0f / 6.0f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)n);
}

float orc_exp_nonpos(float x) { return exp_nonpos(x); }

/* logits: (n, 84) float32 rows; rows[i] = physical row used in the counter */
void orc_policy_sample(const float *logits, const long *rows, long n, uint64_t seed, uint32_t step,
                       uint32_t salt, int deterministic, long long *idx_out, float *logp_out)
{
    for (long i = 0; i < n; i++) {
        float lp_ch[4];
        for (int ch = 0; ch < 4; ch++) {
            const float *l = logits + i * 84 + ch * 21;
            float m = l[0];
            int amax = 0;
            for (int k = 1; k < 21; k++) m = fmaxf(m, l[k]);
            for (int k = 20; k >= 0; k--)           /* the first bin at the maximum (0 if none) */
                if (l[k] == m) amax = k;
            float e[21], s = 0.0f;
            for (int k = 0; k < 21; k++) { e[k] = exp_nonpos(l[k] - m); s += e[k]; }
            int idx = amax;
            if (!deterministic) {
                uint32_t c[4] = {(uint32_t)rows[i], step, (uint32_t)ch, salt};
                orc_philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
                float u = (float)(c[0] >> 8) * 0x1p-24f;
                float target = u * s, cum = 0.0f;
                idx = 20;
                for (int k = 0; k < 21; k++) {
                    cum += e[k];
                    if (cum > target) { idx = k; break; }
                }
            }
            idx_out[i * 4 + ch] = idx;
            lp_ch[ch] = (l[idx] - m) - logf(s);
        }
        logp_out[i] = (lp_ch[0] + lp_ch[1]) + (lp_ch[2] + lp_ch[3]);
    }
}
