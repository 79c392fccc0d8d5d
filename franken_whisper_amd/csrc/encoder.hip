// encoder.hip — encoder forward API (filled in with the encoder kernels).
#include "fw_internal.h"
#include "fw_kernels.h"

extern "C" fwhip_status fwhip_encoder_load(fwhip_ctx *, const fwhip_encoder_weights *, int32_t, fwhip_encoder **out) {
    if (out) *out = nullptr;
    return fw_fail(FWHIP_ERR_UNSUPPORTED, "encoder not built");
}
extern "C" void fwhip_encoder_free(fwhip_encoder *) {}
extern "C" fwhip_status fwhip_encoder_forward(fwhip_encoder *, const float *, int64_t, const int64_t *, int32_t,
                                              int32_t, float *, fwhip_exec_record *) {
    return fw_fail(FWHIP_ERR_UNSUPPORTED, "encoder not built");
}
extern "C" fwhip_status fwhip_encoder_forward_time_major(fwhip_encoder *, const float *, int32_t, int32_t, float *,
                                                         fwhip_exec_record *) {
    return fw_fail(FWHIP_ERR_UNSUPPORTED, "encoder not built");
}
