/*
 * Test-only entry point of libnt_rocm.so. Not part of the ABI in
 * include/nablatensor_rocm.h: no caller of the engine needs it, and it
 * changes nothing unless called.
 */
#ifndef NT_TESTING_H
#define NT_TESTING_H

#ifdef __cplusplus
extern "C" {
#endif

/* Appends `text` to every program the calling thread compiles with hipRTC
 * from now on (null or "" stops it). A test appends source that cannot
 * compile to check that nt_exec_create and nt_compile_check return
 * NT_E_COMPILE with hipRTC's log in nt_last_error, as the reference reports a
 * hipRTC failure with its log (HipRuntime.java:351-354). The appended text is
 * part of the code-object cache key, so such a compile never hits the cache. */
void nt_testing_append_source(const char *text);

#ifdef __cplusplus
}
#endif
#endif
