// dsa_indexer.hip -- lightning-indexer score + top-k select (placeholder that
// reports DSA_EUNSUPPORTED until the kernels land).
#include "../../include/dsa_abi.h"
#include "dsa_internal.h"

extern "C" int dsa_indexer_topk(const dsa_indexer_args *, void *) { return DSA_EUNSUPPORTED; }
extern "C" size_t dsa_indexer_workspace_bytes(int64_t, int64_t, int64_t, int64_t) { return 0; }
