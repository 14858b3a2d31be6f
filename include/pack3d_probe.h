/* Measurement scaffolding of the MI355X PACK3D backend: the issue-rate
 * probe behind `bench.py --probe-rates`.  Built into its own library,
 * pack3d_amd/libpack3d_probe.so, from pack3d_amd/probe/issue_rates.hip; the
 * product library libpack3d_hip.so does not export it.  No counterpart in
 * the reference (amilworks/Pack3D has no native code). */
#ifndef PACK3D_PROBE_H
#define PACK3D_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Issue-rate probe: blocks x 4 waves each run iters iterations of kind
 * (0: 16 v_exp_f32 chains, 1: 16 v_fma_f32 chains, 2: 4 bf16 32x32x16
 * MFMAs, 3: 0 and 2 together, independent, 4: the pipelined summary-sweep
 * tile pattern of head_dim 48, two tiles and column blocks) and write their
 * shader-clock cycles and 100 MHz wall-clock ticks to cycles[2 * wave],
 * cycles[2 * wave + 1] (blocks * 8 values).  Measures the issue rates and
 * co-issue the summary pathway is bound by.  Returns 0, or 1 with
 * p3d_last_error() set for bad arguments, 2 for a failed launch. */
int p3d_probe_issue_rates(int32_t kind, int64_t iters, int32_t blocks, long long* cycles, void* stream);

/* The message of the last failure of this library's calls on this thread. */
const char* p3d_last_error(void);

#ifdef __cplusplus
}
#endif

#endif
