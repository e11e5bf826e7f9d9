// Entry points of include/mako_attn.h whose kernels are not in this build yet: they refuse every call.
#include <hip/hip_runtime.h>

#include "device.hpp"

using namespace mako;

extern "C" size_t mako_cube_select_workspace(uint32_t, uint32_t) { return 0; }
extern "C" int mako_cube_select(uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, mako_dtype,
                                const void*, const void*, const uint32_t*, uint16_t*, uint16_t*, void*, size_t, void*)
{
    return fail(MAKO_EUNSUPPORTED, "cube_select: not in this build");
}
extern "C" int mako_attn_sparse(const mako_sparse_args*, mako_dtype, mako_dtype, const void*, const void*,
                                const void*, void*, const uint16_t*, const uint16_t*, const uint8_t*, const int32_t*,
                                float*, void*)
{
    return fail(MAKO_EUNSUPPORTED, "attention_sparse: not in this build");
}
