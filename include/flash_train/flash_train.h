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
 */
FTRAIN_API FTrainStatus ftrainGemm(FTrainStorageView a, FTrainStorageView b, FTrainStorageView c, FTrainStorageView d,
                                   FTrainStorageView alpha, FTrainStorageView beta, FTrainNumericType compute_type,
                                   void* workspace, uint64_t workspace_bytes, FTrainStream stream);

#ifdef __cplusplus
}
#endif

#endif
