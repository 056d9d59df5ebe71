// fused.h -- the fused decode path: one token of QwenModel::forward as ~7
// fused kernels per layer (include/cactus_hip.h, "fused decode step"),
// captured once into a HIP graph and replayed per token.  The step state
// (token, position, cache length, step) lives on the device, so consecutive
// steps need no host round trip.
#pragma once
#include "engine.h"

namespace cactus {

class FusedDecoder {
public:
    explicit FusedDecoder(QwenModel& m);
    ~FusedDecoder();
    // one greedy step from `token`; returns the next token
    uint32_t step(uint32_t token);
    // n chained greedy steps starting from `token`; tokens written to out
    void run(uint32_t token, size_t n, uint32_t* out);
    // fp16 logits [vocab] of the last step run
    const DevBuf& logits() const { return logits_; }
    // the captured step no longer matches the model's settings
    void invalidate();

private:
    void enqueue();            // all launches of one step on the model stream
    void set_state(uint32_t token);
    void ensure_graph();
    // RoPE positions and token slots for a run; a captured graph that would
    // read past them is dropped and captured again
    void reserve(size_t positions, size_t steps);

    QwenModel& m_;
    DevBuf state_, h_, q_raw_, k_raw_, v_raw_, q_rot_, k_rot_, attn_, mlp_, tokens_, lm_scratch_, logits_, attn_ws_;
    DevBuf lm_tiles_;   // the tied embedding laid out for the streamed LM head
    size_t max_steps_ = 0;
    size_t rope_pos_ = 0;      // positions the RoPE tables hold
    void* graph_ = nullptr;
    bool warmed_ = false;
};

uint32_t fused_decode(QwenModel& m, FusedDecoder& f, uint32_t token);

}  // namespace cactus
