// The C ABI's opaque handles (include/tgx.h) over the runtime's objects.
#pragma once
#include "checkpoint.hpp"
#include "patch.hpp"
#include "runtime.hpp"

struct tgx_context {
    tgx::Context* ctx;
};
struct tgx_decoder {
    tgx::Decoder* dec;
    bool borrowed = false;  // an LM side's decoder: destroyed with it, not alone
};
struct tgx_sampler {
    tgx::Sampler* s;
};
struct tgx_lm_side {
    tgx::LmSide* s;
    tgx_decoder base, residual;
};
struct tgx_encoder {
    tgx::Encoder* e;
};
struct tgx_patch_step {
    tgx::PatchStep* p;
};
struct tgx_checkpoint {
    tgx::Checkpoint* ck;
};
