/*
 * probe.h -- measurement probes of libkf_probe.so, used by bench.py to
 * put the floors of the small decode step beside its measured time.  Not part
 * of the attention ABI and no counterpart in the reference (whose bench,
 * tests/bench_flash_attn.cu:108-123, times only the kernel itself).
 *
 * Both return 0 on success, 1 for an invalid argument (nothing launched) and
 * 2 for a failed launch.
 */
#ifndef KF_PROBE_H
#define KF_PROBE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Read bytes_each bytes of `a` and of `b` (device, 16-byte aligned,
 * bytes_each a positive multiple of 16) once, with 16-byte loads all issued
 * before their first use; `sink` (device, one unsigned) is written only if
 * the data XORs to a fixed magic value.  The floor of a kernel that must read
 * both buffers once. */
int kf_probe_read(const void* a, const void* b, size_t bytes_each, unsigned* sink, void* stream);

/* Launch an empty kernel (one wave) on `stream`. */
int kf_probe_empty(void* stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* KF_PROBE_H */
