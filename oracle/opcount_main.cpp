// opcount_main.cpp -- the C restatement (f16_oracle.c) built with the counting `double` of
// opcount.hpp: liborc_opcount.so exports opc_fdm_count(), which steps aircraft states exactly
// as orc_fdm_step_batch does and returns the operation tallies of those substeps.
// TEST INFRASTRUCTURE ONLY (tests/golden/make_flops_golden.py writes the FLOP fixture with it).
#include "opcount.hpp"
thread_local OpCounts g_ops;
#undef _OPENMP
#include "f16_oracle.c"
#undef double

extern "C" void opc_fdm_count(double* states, const double* actions, long nac, int ndec,
                              int substeps, int fcs_rate, unsigned long long* counts7) {
  orc_init();
  const OpDouble dt(1.0 / (double)fcs_rate);    // the FCS period, a constant of the model
  g_ops = OpCounts{};
  for (int d = 0; d < ndec; ++d)
    for (long i = 0; i < nac; ++i) {
      OpDouble* st = reinterpret_cast<OpDouble*>(states + 101 * i);
      const OpDouble* ac = reinterpret_cast<const OpDouble*>(actions + ((long)d * nac + i) * 4);
      for (int s = 0; s < substeps; ++s) fdm_step(st, ac[0], ac[1], ac[2], ac[3], dt, nullptr);
    }
  const unsigned long long* c = &g_ops.add;
  for (int k = 0; k < 7; ++k) counts7[k] = c[k];
}
