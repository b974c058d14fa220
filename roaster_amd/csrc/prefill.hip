/*
 * prefill.hip -- MoE prefill (placeholder until the MFMA path lands).
 */
#include "internal.h"

extern "C" int roaster_moe_prefill(RoasterTable *t, int layer, const float *X, int T, float *Y,
                                   const RoasterPrefillOpts *o)
{
    (void)t; (void)layer; (void)X; (void)T; (void)Y; (void)o;
    return rt_fail(ROASTER_EINVAL, "roaster_moe_prefill: not built yet");
}
