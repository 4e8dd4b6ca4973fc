// MFMA paged decode kernel (vLLM page layout, P.V on matrix cores).
#include "ssq_common.h"

int ssq_decode_mfma_supported(const ssq_decode_args* a) { (void)a; return 0; }
size_t ssq_decode_mfma_workspace(const ssq_decode_args* a) { (void)a; return 0; }
int ssq_decode_mfma(const ssq_decode_args* a, void* workspace, size_t ws_bytes, hipStream_t st) {
    (void)a; (void)workspace; (void)ws_bytes; (void)st;
    return ssq_fail(SSQ_ERR_UNSUPPORTED, "MFMA decode kernel not built");
}
