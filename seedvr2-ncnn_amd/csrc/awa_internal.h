// Entry points shared between the C ABI translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "awa_plan.h"
#include "seedvr2_awa.h"

namespace awa
{

// Sets the calling thread's awa_last_error() text.
void set_error(const std::string& message);

// Caller-provided device memory for the per-window text rows.
struct Scratch
{
    void* ptr;
    size_t bytes;
};

// awa_forward (norm null) or awa_forward_qknorm, with an optional event
// recorded between the attention kernel and the text-mean kernel (for
// per-kernel timing). scratch null: the text rows go to the plan's
// workspace (allocated on first use, with the work list). scratch set: they
// go there, and nothing is allocated; the plan must already hold the work
// list for the head count.
int forward_fused(const awa_plan* plan, const awa_blob* video_qkv, const awa_blob* text_qkv, const awa_qk_norm* norm,
                  const awa_blob* video_out, const awa_blob* text_out, int compute, hipStream_t stream,
                  hipEvent_t after_attention, const Scratch* scratch = nullptr);

// Resolves the current device's address of awa_forward_noalloc's static
// scratch array (once per device); AWA_ERR_DEVICE with the reason set if the
// runtime cannot.
int noalloc_setup();

} // namespace awa
