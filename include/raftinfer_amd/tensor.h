/* Data-type codes shared with the reference (cpp/include/raftinfer/tensor.h:10-15);
 * values are identical so policies and dtypes pass through unchanged. */
#pragma once

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum RaftInferDataType {
  RAFTINFER_DTYPE_F32 = 1,
  RAFTINFER_DTYPE_F16 = 2,
  RAFTINFER_DTYPE_BF16 = 3,
  RAFTINFER_DTYPE_Q4_K = 100
} RaftInferDataType;

#ifdef __cplusplus
}
#endif
