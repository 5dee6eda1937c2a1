/*
 * flash-train for MI355X -- staged C API (Pattern -> Ops -> Args -> Plan).
 *
 * Drop-in for the reference's include/flash_train/common.h: the same type
 * names, enum values, struct layouts and function signatures, so code and
 * bindings written against the reference compile and link unchanged.  Each
 * declaration cites the reference line it replaces.
 *
 * Error convention (reference common.h:152-175, src/include/flash_train/api.hpp:37-62):
 * every non-query call returns an FTrainStatus and records it, with a
 * diagnostic message, as the calling thread's last result.  Output pointers
 * are left untouched on failure.
 */
#ifndef FTRAIN_COMMON_H_
#define FTRAIN_COMMON_H_

#include <stdbool.h>
#include <stdint.h>

#include <flash_train/control.h>
#include <flash_train/version.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* reference common.h:21-24 */
typedef hipStream_t FTrainStream;
typedef int32_t FTrainDeviceId;

/* reference common.h:28-36 */
typedef uint8_t FTrainStatus;
enum {
    FTRAIN_STATUS_SUCCESS          = 0,
    FTRAIN_STATUS_INVALID_ARGUMENT = 1,
    FTRAIN_STATUS_OUT_OF_MEMORY    = 2,
    FTRAIN_STATUS_OVERFLOW         = 3,
    FTRAIN_STATUS_UNSUPPORTED      = 4,
    FTRAIN_STATUS_INTERNAL_ERROR   = 50,
};

/* reference common.h:38-65 (values are part of the ABI) */
typedef uint8_t FTrainNumericType;
enum {
    FTRAIN_NUMERIC_TYPE_INVALID    = 0,
    FTRAIN_NUMERIC_TYPE_FP64       = 1,
    FTRAIN_NUMERIC_TYPE_INT64      = 2,
    FTRAIN_NUMERIC_TYPE_UINT64     = 3,
    FTRAIN_NUMERIC_TYPE_FP32       = 4,
    FTRAIN_NUMERIC_TYPE_INT32      = 5,
    FTRAIN_NUMERIC_TYPE_UINT32     = 6,
    FTRAIN_NUMERIC_TYPE_FP16       = 7,
    FTRAIN_NUMERIC_TYPE_BF16       = 8,
    FTRAIN_NUMERIC_TYPE_INT16      = 9,
    FTRAIN_NUMERIC_TYPE_UINT16     = 10,
    FTRAIN_NUMERIC_TYPE_FP8_E4M3FN = 11,
    FTRAIN_NUMERIC_TYPE_FP8_E5M2   = 12,
    FTRAIN_NUMERIC_TYPE_UFP8_E8M0  = 13,
    FTRAIN_NUMERIC_TYPE_UFP8_E5M3  = 14,
    FTRAIN_NUMERIC_TYPE_UFP8_E6M2  = 15,
    FTRAIN_NUMERIC_TYPE_INT8       = 16,
    FTRAIN_NUMERIC_TYPE_UINT8      = 17,
    FTRAIN_NUMERIC_TYPE_FP4_E2M1   = 18,
    FTRAIN_NUMERIC_TYPE_FP4_S1P2   = 19,
    FTRAIN_NUMERIC_TYPE_INT4       = 20,
    FTRAIN_NUMERIC_TYPE_UINT4      = 21,
    FTRAIN_NUMERIC_TYPE_UFP1_E1M0  = 22,
    FTRAIN_NUMERIC_TYPE_UINT1      = 23,
    FTRAIN_NUMERIC_TYPE_COUNT,
};

/* reference common.h:67-74 */
typedef uint8_t FTrainIndexType;
enum {
    FTRAIN_INDEX_TYPE_INVALID                  = 0,
    FTRAIN_INDEX_TYPE_CONTINUOUS               = 1,
    FTRAIN_INDEX_TYPE_NVIDIA_SF_128X4_SWIZZLED = 2,
    FTRAIN_INDEX_TYPE_GROUPED_CONTINUOUS       = 3,
    FTRAIN_INDEX_TYPE_COUNT,
};

/*
 * One tensor's storage: address plus shape and layout metadata
 * (reference common.h:87-118).  num_dims == 0 is a scalar and needs a
 * non-null address; a larger rank may carry a null address.  Exactly one of
 * `strides` (element units) and a predefined `index_type` describes the
 * layout.  Setters copy dims/strides; the memory is never owned.
 */
typedef struct {
    void* memory;
    const int64_t* dims;
    const int64_t* strides;
    uint8_t num_dims;
    FTrainNumericType numeric_type;
    FTrainIndexType index_type;
    bool is_host_memory;
} FTrainStorageView;

/* Opaque role identifiers (reference common.h:131-137). */
// clang-format off
typedef struct { uint64_t opaque; } FTrainTensorId;
typedef struct { uint64_t opaque; } FTrainTensorListId;
typedef struct { uint64_t opaque; } FTrainGroupedTensorId;
typedef struct { uint64_t opaque; } FTrainGemmOpId;
typedef struct { uint64_t opaque; } FTrainGroupedABCDGemmOpId;
typedef struct { uint64_t opaque; } FTrainGroupedBCDGemmOpId;
typedef struct { uint64_t opaque; } FTrainGroupedABGemmOpId;
// clang-format on

/* Opaque handles (reference common.h:145-148). */
typedef struct FTrainPatternStruct* FTrainPattern;
typedef struct FTrainOpsStruct* FTrainOps;
typedef struct FTrainArgsStruct* FTrainArgs;
typedef struct FTrainPlanStruct* FTrainPlan;

/* ---- thread-local diagnostics (reference common.h:162,175) ---- */

/* Last status recorded on this thread; SUCCESS before any call. */
FTRAIN_API FTrainStatus ftrainGetLastStatus(void);

/* Last message recorded on this thread ("" after a success), at most 2047
 * characters (reference error.hpp:17,52).  Owned by the
 * library; valid until this thread's next non-query call. */
FTRAIN_API const char* ftrainGetLastMessage(void);

/* ---- Pattern construction (reference common.h:186-306) ---- */

FTRAIN_API FTrainStatus ftrainPatternCreate(FTrainPattern* pattern);
FTRAIN_API FTrainStatus ftrainPatternDestroy(FTrainPattern pattern);
FTRAIN_API FTrainStatus ftrainPatternAddTensor(FTrainPattern pattern, FTrainTensorId* tensor);
FTRAIN_API FTrainStatus ftrainPatternAddTensorList(FTrainPattern pattern, FTrainTensorListId* tensor_list);
FTRAIN_API FTrainStatus ftrainPatternAddGroupedTensor(FTrainPattern pattern, FTrainGroupedTensorId* grouped_tensor);

/* Gemm: d = alpha * (a @ b) + beta * c.  Ports are only recorded here; the
 * structure is validated when ftrainOpsCreate() builds the Pattern. */
FTRAIN_API FTrainStatus ftrainPatternAddGemm(FTrainPattern pattern, FTrainGemmOpId* op, FTrainTensorId a,
                                             FTrainTensorId b, FTrainTensorId c, FTrainTensorId d, FTrainTensorId alpha,
                                             FTrainTensorId beta);

/* Grouped GEMM topologies (reference common.h, grouped op builders).  The
 * reference registers no engine for them, so its ftrainOpsCreate() returns
 * UNSUPPORTED (src/engine.cpp:25-27); this library registers an engine for
 * each, so ftrainOpsCreate() returns an Ops and Plans run grouped kernels. */
FTRAIN_API FTrainStatus ftrainPatternAddGroupedABCDGemm(FTrainPattern pattern, FTrainGroupedABCDGemmOpId* op,
                                                        FTrainGroupedTensorId a, FTrainGroupedTensorId b,
                                                        FTrainGroupedTensorId c, FTrainGroupedTensorId d,
                                                        FTrainTensorId alpha, FTrainTensorId beta);
FTRAIN_API FTrainStatus ftrainPatternAddGroupedBCDGemm(FTrainPattern pattern, FTrainGroupedBCDGemmOpId* op,
                                                       FTrainTensorListId a, FTrainGroupedTensorId b,
                                                       FTrainGroupedTensorId c, FTrainGroupedTensorId d,
                                                       FTrainTensorId alpha, FTrainTensorId beta);
FTRAIN_API FTrainStatus ftrainPatternAddGroupedABGemm(FTrainPattern pattern, FTrainGroupedABGemmOpId* op,
                                                      FTrainGroupedTensorId a, FTrainGroupedTensorId b,
                                                      FTrainTensorListId c, FTrainTensorListId d, FTrainTensorId alpha,
                                                      FTrainTensorId beta);

/* ---- Ops matching (reference common.h:308-331) ---- */

/* Matches the Pattern against every supported Pattern, ignoring insertion
 * order; UNSUPPORTED when nothing matches.  The Ops outlives the Pattern. */
FTRAIN_API FTrainStatus ftrainOpsCreate(FTrainOps* ops, FTrainPattern pattern);
FTRAIN_API FTrainStatus ftrainOpsDestroy(FTrainOps ops);

/* ---- Args binding (reference common.h:333-474) ---- */

FTRAIN_API FTrainStatus ftrainArgsCreate(FTrainArgs* args, FTrainOps ops);
FTRAIN_API FTrainStatus ftrainArgsDestroy(FTrainArgs args);
FTRAIN_API FTrainStatus ftrainArgsSetTensor(FTrainArgs args, FTrainTensorId tensor, FTrainStorageView storage_view);
FTRAIN_API FTrainStatus ftrainArgsSetTensorList(FTrainArgs args, FTrainTensorListId tensor_list,
                                                const FTrainStorageView storage_views[], uint32_t num_storage_views);
FTRAIN_API FTrainStatus ftrainArgsSetGroupedTensor(FTrainArgs args, FTrainGroupedTensorId grouped_tensor,
                                                   uint32_t num_groups, FTrainStorageView data,
                                                   const FTrainStorageView* offsets,
                                                   const FTrainStorageView dim_sizes[],
                                                   const FTrainStorageView strides[]);
FTRAIN_API FTrainStatus ftrainArgsSetGemm(FTrainArgs args, FTrainGemmOpId op, FTrainNumericType compute_type);
FTRAIN_API FTrainStatus ftrainArgsSetGroupedABCDGemm(FTrainArgs args, FTrainGroupedABCDGemmOpId op,
                                                     FTrainNumericType compute_type);
FTRAIN_API FTrainStatus ftrainArgsSetGroupedBCDGemm(FTrainArgs args, FTrainGroupedBCDGemmOpId op,
                                                    FTrainNumericType compute_type);
FTRAIN_API FTrainStatus ftrainArgsSetGroupedABGemm(FTrainArgs args, FTrainGroupedABGemmOpId op,
                                                   FTrainNumericType compute_type);

/* ---- Plan selection and execution (reference common.h:476-589) ---- */

/* Selects (through the per-engine selection cache) and configures every
 * applicable Primitive for the Args on the calling thread's current device,
 * best first.  INVALID_ARGUMENT: incomplete or inconsistent Args;
 * OVERFLOW: a byte count does not fit uint64; UNSUPPORTED: nothing applies
 * (the message names each Primitive's reason).  The Plan binds the Args'
 * addresses and host-scalar values; it outlives the Ops and Args. */
FTRAIN_API FTrainStatus ftrainPlanCreate(FTrainPlan* plan, FTrainArgs args);
FTRAIN_API FTrainStatus ftrainPlanDestroy(FTrainPlan plan);
FTRAIN_API FTrainStatus ftrainPlanGetNumPrimitives(FTrainPlan plan, uint64_t* num_primitives);
/* The returned name is owned by the Plan. */
FTRAIN_API FTrainStatus ftrainPlanGetPrimitiveName(FTrainPlan plan, uint64_t primitive_index, const char** name);
FTRAIN_API FTrainStatus ftrainPlanGetPrimitiveRequiredWorkspaceBytes(FTrainPlan plan, uint64_t primitive_index,
                                                                     uint64_t* workspace_bytes);
/* Enqueues one Primitive on `stream` without synchronizing.  INVALID_ARGUMENT
 * when the index is out of range, the calling thread's device is not the
 * Plan's, or the workspace is too small / null while required.  Concurrent
 * executions of one Plan need external synchronization. */
FTRAIN_API FTrainStatus ftrainPlanExecutePrimitive(FTrainPlan plan, uint64_t primitive_index, void* workspace,
                                                   uint64_t workspace_bytes, FTrainStream stream);

#ifdef __cplusplus
}
#endif

#endif
