// host_internal.h — functions of moe_host.cpp that the library's other host
// files (the checkpoint loader) call. Not part of the public ABI.
#pragma once
#include <stdint.h>

#include <string>

#include "../../include/windlass_moe.h"

namespace wl {

const wl_moe_config& ctx_config(const wl_ctx* c);
uint32_t ctx_shared_inter(const wl_ctx* c);  // moe_inter x n_shared
// Records msg as the context's last error and returns s.
wl_status ctx_fail(wl_ctx* c, wl_status s, const std::string& msg);
// Binds a layer as wl_set_layer (bf16_shared: [gate | up | down] bf16) or
// wl_set_layer_mxfp4 (mxfp4_parts: the six tensors) do, the context taking
// over the device allocations router_w, bias and ln (ln may be null): they
// are freed when the layer is bound again, when the context is destroyed, or
// at once if the call fails.
wl_status ctx_set_layer_owned(wl_ctx* c, uint32_t layer, uint16_t* router_w, float* bias, uint16_t* ln,
                              const uint16_t* bf16_shared, const uint8_t* const* mxfp4_parts);

}  // namespace wl
