// Host build of the skeleton's own fp64 math, for accuracy tests against mpmath.
#include "prelude.h"
#include "nt_skeleton.h"

static void load_tables() {
  blockDim.x = 1;
  threadIdx.x = 0;
  nt_tables_load();
}

extern "C" {
void emu_neg2log(const nt_u32* c, double* out, long n) {
  load_tables();
  for (long i = 0; i < n; ++i) out[i] = nt_neg2log_u32(c[i]);
}
void emu_log(const double* a, double* out, int* bad, long n) {
  load_tables();
  for (long i = 0; i < n; ++i) {
    bool b = false;
    out[i] = nt_log_fast(a[i], b);
    bad[i] = b ? 1 : 0;
  }
}
void emu_sincos(const nt_u32* c, double* s, double* co, long n) {
  load_tables();
  for (long i = 0; i < n; ++i) nt_sincos_2pi_u32(c[i], s[i], co[i]);
}
void emu_exp(const double* x, double* out, long n) {
  load_tables();
  for (long i = 0; i < n; ++i) out[i] = nt_exp(x[i]);
}
void emu_sqrt(const double* a, double* out, long n) {
  for (long i = 0; i < n; ++i) out[i] = nt_sqrt_pos(a[i]);
}
void emu_sqrt_q(const double* a, double* out, double* q, int* bad, long n) {
  for (long i = 0; i < n; ++i) {
    bool b = false;
    out[i] = nt_sqrt_q(a[i], q[i], b);
    bad[i] = b ? 1 : 0;
  }
}
void emu_recip(const double* b, double* out, int* bad, long n) {
  for (long i = 0; i < n; ++i) {
    bool f = false;
    out[i] = nt_recip(b[i], f);
    bad[i] = f ? 1 : 0;
  }
}
void emu_normal_pair(const nt_u32* lo, const nt_u32* hi, const nt_u32* ctr, double* zc, double* zs, long n) {
  load_tables();
  for (long i = 0; i < n; ++i) nt_normal_pair(lo[i], hi[i], ctr[i], zc[i], zs[i]);
}
}
