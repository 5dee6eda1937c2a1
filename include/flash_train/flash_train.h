/*
 * flash-train for MI355X -- convenience C API.
 *
 * Drop-in for the reference's include/flash_train/flash_train.h:46-48.
 */
#ifndef FTRAIN_FLASH_TRAIN_H_
#define FTRAIN_FLASH_TRAIN_H_

#include <flash_train/common.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * d = alpha * (a @ b) + beta * c with the recommended Primitive (index 0).
 *
 * Equivalent to building the Gemm Pattern, creating Ops and Args, creating a
 * Plan and executing its Primitive 0 (reference src/api/gemm_api.cpp:54-83);
 * the Ops is built once per process and Plan creation is a selection-cache
 * hit after the first call for a given problem description.  a, b, c, d are
 * rank-two device views (c may have null memory, which drops the beta term);
 * alpha and beta are host fp32 scalars.  Asynchronous on `stream`.  On
 * failure the thread's last message is the failing step's message.
 * Under stream capture a problem not yet seen on this thread and stream runs
 * the first Primitive that needs no more than `workspace_bytes` (nothing is
 * allocated during the capture); FTRAIN_STATUS_UNSUPPORTED when none does.
 * A graph that captured a call keeps its Plan alive until the graph and its
 * executable graphs are destroyed.
 */
FTRAIN_API FTrainStatus ftrainGemm(FTrainStorageView a, FTrainStorageView b, FTrainStorageView c, FTrainStorageView d,
                                   FTrainStorageView alpha, FTrainStorageView beta, FTrainNumericType compute_type,
                                   void* workspace, uint64_t workspace_bytes, FTrainStream stream);

/*
 * ftrainGemm without device allocation.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory -- code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.
 *
 * Same operands, result and errors as ftrainGemm, minus the workspace: a
 * split-k Primitive keeps its partial tiles in the library's fixed device
 * scratch array (64 MiB per GPU, held from library load until the process
 * ends) and no call allocates or frees device memory.  The Primitive run is
 * the first in the Plan's rank order whose partial tiles fit the array
 * (Primitive 0 whenever it fits); UNSUPPORTED when none fits.  Every call on
 * one GPU shares that GPU's array: calls that may overlap on one GPU (other
 * streams, other threads) race and must be serialised by the caller.
 * Nothing in the array needs to start at zero.
 */
FTRAIN_API FTrainStatus ftrainGemmNoAlloc(FTrainStorageView a, FTrainStorageView b, FTrainStorageView c,
                                          FTrainStorageView d, FTrainStorageView alpha, FTrainStorageView beta,
                                          FTrainNumericType compute_type, FTrainStream stream);

#ifdef __cplusplus
}
#endif

#endif
