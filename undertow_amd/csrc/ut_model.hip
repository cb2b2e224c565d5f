// ut_model.hip -- DeepSeek model / session / MTP loop on device (in progress).
#include "ut_internal.h"

using namespace ut;

struct ut_model { ut_ctx *ctx; };
struct ut_session { ut_model *m; };

extern "C" {
int32_t ut_model_create(ut_ctx *ctx, const ut_model_config *, ut_model **out) { if (out) *out = nullptr; set_error(ctx, "not implemented"); return UT_ERR_STATE; }
int32_t ut_model_set_tensor(ut_model *, const char *, int32_t, const void *, int64_t, const float *, int64_t, int64_t) { return UT_ERR_STATE; }
int32_t ut_model_finalize(ut_model *) { return UT_ERR_STATE; }
int32_t ut_model_synthesize(ut_model *, uint64_t, float, int32_t, int32_t) { return UT_ERR_STATE; }
int64_t ut_model_device_bytes(const ut_model *) { return 0; }
void ut_model_free(ut_model *) {}
int32_t ut_session_create(ut_model *, int32_t, ut_session **out) { if (out) *out = nullptr; return UT_ERR_STATE; }
void ut_session_free(ut_session *) {}
int32_t ut_session_prefill(ut_session *, const int32_t *, int64_t, float *, int32_t *) { return UT_ERR_STATE; }
int32_t ut_session_truncate(ut_session *, int64_t) { return UT_ERR_STATE; }
int64_t ut_session_position(const ut_session *) { return UT_ERR_STATE; }
int64_t ut_generate_greedy(ut_model *, const int32_t *, int64_t, int64_t, int32_t *) { return UT_ERR_STATE; }
int64_t ut_generate_mtp(ut_model *, const int32_t *, int64_t, int64_t, int32_t, int32_t *, int64_t *, int64_t *) { return UT_ERR_STATE; }
}
