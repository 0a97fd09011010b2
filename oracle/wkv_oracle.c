/*
 * TEST INFRASTRUCTURE ONLY: CPU oracle for the WKV-7 recurrence, forward and
 * backward.  It restates the reference's JAX scan (src/rwkv7m/model/wkv.py:
 * 60-67 over rwkv_core.py:54-86) and its reverse equations
 * (kernels/wkv_pallas_gpu.py:221-257) as plain C loops.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Exported symbols:
 *   oracle_wkv7_forward_f64 / oracle_wkv7_backward_f64  - the parity oracle
 *   oracle_wkv7_forward_f32 / oracle_wkv7_backward_f32  - the reference's
 *       fp32 arithmetic (timed as the CPU baseline, OpenMP over (b, h))
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define REAL double
#define EXP exp
#define SUFFIX f64
#include "wkv_oracle_body.h"
#undef REAL
#undef EXP
#undef SUFFIX

#define REAL float
#define EXP expf
#define SUFFIX f32
#include "wkv_oracle_body.h"
#undef REAL
#undef EXP
#undef SUFFIX
