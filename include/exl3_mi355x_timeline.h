/*
 * exl3_mi355x_timeline.h -- tracing entry points of the instrumented library build
 * (libexl3_mi355x_timeline.so: exl3_gemv.hip compiled with -DEXL3_TIMELINE; build_ext.py
 * --timeline).  The product library (libexl3_mi355x.so) exports none of these.  No counterpart
 * in the reference.  Callers: bench.py --timeline.
 *
 * Every GEMV workgroup's thread 0 stores the 100 MHz s_memrealtime counter (10 ns a tick) at each
 * phase boundary into a device array [max_wgs][phases] of uint64, slot [blockIdx.x][phase]:
 *   0 entry, 1 prologue loads issued, 2 loop start (input rotated), 3 loop end, 4 partial sums
 *   stored (complete), 5 completion counters counted, 6 partials summed (reducing workgroups only),
 *   7 end; slot 8 holds the workgroup's placement: HW_ID (bits 8-11 CU, 12 SH, 13-15 SE) in the
 *   low word, XCC_ID in the high word.
 * A launch overwrites the slots of its workgroups; a phase a workgroup does not reach keeps the
 * previous value, so clear before the launch of interest.  These calls synchronize the device.
 */
#ifndef EXL3_MI355X_TIMELINE_H
#define EXL3_MI355X_TIMELINE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

int exl3_timeline_shape(int* max_wgs, int* phases);
int exl3_timeline_clear(void);
int exl3_timeline_read(void* host, size_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* EXL3_MI355X_TIMELINE_H */
