// Internal interface between the edge kernels and the node-mode plan: the
// CSR build behind esa_csr_build (the stable radix sort of edge ids by key and
// the indptr of the sorted keys), with an optional device flag `skip`: when it
// is non-null and *skip != 0 at launch time, every launch of the build returns
// at once and writes nothing (the caller has produced the CSR another way).
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

int csr_build_impl(const int* keys, int64_t num_edges, int num_nodes, int* indptr, int* perm, void* workspace,
                   size_t workspace_bytes, hipStream_t st, const int* skip);
