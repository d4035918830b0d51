// Dense varlen attention at head dims 32 and 64 (bf16 MFMA): placeholder
// entry points until the kernels land; calls report ESA_ERR_HEAD_DIM.
#include "esa_attn_dense.h"
#include "esa_common.h"
#include "../../include/esa_hip.h"

size_t wide_attn_workspace_size(int, int, int, int, bool) { return 0; }
int wide_attn_fwd(const DenseAttnCall&, void*, size_t, hipStream_t) { return ESA_ERR_HEAD_DIM; }
int wide_attn_bwd(const DenseAttnCall&, void*, size_t, hipStream_t) { return ESA_ERR_HEAD_DIM; }
