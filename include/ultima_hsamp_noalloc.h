/* The allocation-free sampler entry point, exported by libultima_hsamp_noalloc.so
 * (which links libultima_hsamp.so). It lives in a library of its own because
 * its device array is held, on every GPU the library runs on, by each process
 * that loads it: processes that never call it do not load it. */
#ifndef ULTIMA_HSAMP_NOALLOC_H
#define ULTIMA_HSAMP_NOALLOC_H

#include "ultima_hsamp.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Bytes of the fixed device array ultima_hsamp_run_noalloc() takes its scratch
 * from (each GPU the library runs on holds one until the process ends), and of
 * the part of it at its front that holds the per-row plans. */
#define ULTIMA_HSAMP_NOALLOC_SCRATCH_BYTES (96u << 20)
#define ULTIMA_HSAMP_NOALLOC_PLAN_BYTES (2u << 20)

/* No counterpart in the reference: ultima_hsamp_run() for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No handle: it runs on the current device
 * and calls no allocating routine. The kernels' scratch comes from a fixed
 * device array of ULTIMA_HSAMP_NOALLOC_SCRATCH_BYTES per GPU; a batch whose
 * scratch does not fit (about rows x vocab x 8 bytes, e.g. 64 x 151936 fp32
 * rows fit) returns ULTIMA_HSAMP_ERR_CAPACITY.
 * The per-row knobs are copied from host memory into the array's plan region
 * with hipMemcpyAsync unless it already holds the same ones. Under stream
 * capture nothing is copied: the same knobs must have been used by an
 * uncaptured call first (the last one, or one a graph was captured with),
 * else ULTIMA_HSAMP_ERR_UNSUPPORTED. Knobs a graph was captured with stay in
 * place until the process ends, so later calls with other knobs do not change
 * what the graph's replays read; when the plan region
 * (ULTIMA_HSAMP_NOALLOC_PLAN_BYTES) is full of them, a call with new knobs
 * returns ULTIMA_HSAMP_ERR_CAPACITY.
 * Every call on a GPU shares that GPU's array, which keeps the last call's
 * contents: calls that overlap on one GPU (two streams or threads, or a
 * graph's replay beside another call) race; issue them on one stream.
 * Results are those of ultima_hsamp_run() for the same batch. */
int ultima_hsamp_run_noalloc(const ultima_hsamp_batch* batch, void* hip_stream);

#ifdef __cplusplus
}
#endif
#endif
