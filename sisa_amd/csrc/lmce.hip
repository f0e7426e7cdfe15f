// Chunked linear + cross-entropy (placeholder until the fused kernels land).
#include "host.h"

extern "C" int sisa_lmce_fwd(const sisa_lmce_fwd_args* a, void* stream) {
    (void)a;
    (void)stream;
    sisa::set_error("sisa_lmce_fwd: not implemented");
    return SISA_ERR_UNSUPPORTED;
}

extern "C" int sisa_lmce_bwd(const sisa_lmce_bwd_args* a, void* stream) {
    (void)a;
    (void)stream;
    sisa::set_error("sisa_lmce_bwd: not implemented");
    return SISA_ERR_UNSUPPORTED;
}
