/*
 * starlight_engine.h — the step loop that drives a device through compiled
 * CommandBuffers: a C restatement of sl-core's `Engine::build/step`
 * (docs ARCH-0007 §3.2; the crate itself is not in the reference tree).
 *
 * It is the caller of the Device contract, not part of it: build() allocates
 * the scratchpad, KV state, inputs and outputs through the sl_hip_* entry
 * points and resolves every command's ValueIds to BufferRefs once; step()
 * uploads token ids and positions, dispatches the commands in order, calls
 * synchronize and downloads the logits, allocating nothing
 * (ARCH-0007 §3.2 "step 不得分配").
 */
#ifndef STARLIGHT_ENGINE_H
#define STARLIGHT_ENGINE_H

#include "starlight_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* sl_ir::Effect (ARCH-0004 §4). */
typedef enum sl_effect { SL_EFFECT_NONE = 0, SL_EFFECT_READ_STATE = 1, SL_EFFECT_WRITE_STATE = 2 } sl_effect;

/* sl_ir::Command (ARCH-0004 §6): ValueIds of the ports in signature order
 * (scalar ports included); `state` is the effect's State ValueId. */
typedef struct sl_command {
    sl_op op;
    uint32_t n_inputs;
    uint32_t n_outputs;
    uint32_t inputs[SL_MAX_INPUTS];
    uint32_t outputs[SL_MAX_OUTPUTS];
    uint32_t effect; /* sl_effect */
    uint32_t state;
} sl_command;

/* sl_ir::Slot (ARCH-0004 §7), bytes. */
typedef struct sl_slot {
    uint32_t value;
    uint32_t reserved;
    uint64_t offset;
    uint64_t bytes;
} sl_slot;

/* sl_ir::CommandBuffer (ARCH-0004 §6-7). */
typedef struct sl_command_buffer {
    uint32_t ir_version;
    uint32_t reserved;
    const sl_value *values;
    size_t n_values;
    const sl_command *commands;
    size_t n_commands;
    uint64_t scratchpad_bytes;
    const sl_slot *slots;
    size_t n_slots;
} sl_command_buffer;

/* sl_core::CompiledProgram (ARCH-0007 §3.2). A negative optional id means
 * "absent". Weights are (ValueId, BufferId) pairs uploaded beforehand; they
 * include the scale Param of every group-quantized Param (a separate f32
 * [n, k / group] Param, "<role>.__scales", ARCH-0006:147), paired with it in
 * quant_params[i] -> quant_scales[i] (ValueIds). */
typedef struct sl_compiled_program {
    sl_command_buffer ir;
    const uint32_t *weight_values;
    const uint32_t *weight_buffers;
    size_t n_weights;
    uint32_t token_ids;
    int32_t positions;
    uint32_t seq_len;
    int32_t past_len;
    uint32_t logits;
    const uint32_t *quant_params;
    const uint32_t *quant_scales;
    size_t n_quant;
} sl_compiled_program;

typedef enum sl_step_mode { SL_STEP_PREFILL = 0, SL_STEP_DECODE = 1 } sl_step_mode;

typedef struct sl_engine sl_engine;

/* Engine::build (ARCH-0007 §3.2 build responsibilities 1-4). The two
 * programs share State values with the same ValueId (the KV cache). Every
 * group-quantized Param is bound to its scale Param's buffer here
 * (sl_hip_bind_quantized); a quantized Param without a bound scale Param of
 * shape [n, k / group] fails the build with Execution. */
sl_status sl_engine_build(sl_hip_device *device, const sl_compiled_program *prefill,
                          const sl_compiled_program *decode, uint32_t max_batch, uint32_t max_context,
                          sl_engine **out);

/* Engine::step (ARCH-0007 §3.2 step responsibilities 1-5). `logits` receives
 * the program's Output value (n_logits elements). */
sl_status sl_engine_step(sl_engine *engine, uint32_t mode, const uint32_t *token_ids, size_t n_token_ids,
                         const uint32_t *positions, size_t n_positions, uint32_t seq_len, uint32_t past_len,
                         float *logits, size_t n_logits);

/* Greedy decode loop for benchmarks and tests (not part of sl-core, which
 * has no sampler, ARCH-0008 G-13): after a prefill of `prompt` (batch 1),
 * runs `steps` decode steps feeding back the first maximum logit, writes the
 * steps + 1 generated ids to `tokens_out` (the prefill's first, then one per
 * decode step) and, if `logits_out` is non-null, every step's logits
 * (steps + 1 rows of vocab floats, the prefill row first). */
sl_status sl_engine_generate(sl_engine *engine, const uint32_t *prompt, size_t prompt_len, uint32_t steps,
                             uint32_t *tokens_out, float *logits_out, size_t vocab);

/* Greedy batch-1 decode without a prefill: feeds `token` at position
 * `past_len`, then each step's first maximum logit, for `steps` steps;
 * tokens_out receives the `steps` generated ids. */
sl_status sl_engine_decode(sl_engine *engine, uint32_t token, uint32_t past_len, uint32_t steps,
                           uint32_t *tokens_out);

/* Greedy decode of a batch compiled into the decode program (batch rows of
 * one token each, all at position `past_len + step`, as Engine::step takes
 * one past_len for the batch): `tokens` holds the batch's first tokens;
 * tokens_out receives steps x batch ids, step-major. Each step is
 * sl_engine_step followed by each row's first maximum logit. */
sl_status sl_engine_decode_batch(sl_engine *engine, const uint32_t *tokens, uint32_t past_len, uint32_t steps,
                                 uint32_t *tokens_out);

/* Greedy decode of a batch whose rows sit at their own lengths, for a
 * decode program whose KV State is bound to a paged cache
 * (sl_hip_bind_paged_state; no reference counterpart, gaps G-17 / G-18,
 * ARCH-0008:123-124): in step s row b takes its token at position
 * positions[b] + s; before each step those positions are written to the
 * u32 buffer `lengths` (the binding's seq_lens, one word per row), and the
 * step's past_len scalar is 0 (a paged State does not read it). The block
 * tables must already cover positions[b] + steps of every row. tokens_out
 * receives steps x batch ids, step-major. */
sl_status sl_engine_decode_rows(sl_engine *engine, const uint32_t *tokens, const uint32_t *positions,
                                uint32_t lengths, uint32_t steps, uint32_t *tokens_out);

/* The BufferId the engine allocated for a State value (e.g. to inspect or
 * reset the KV cache), or UINT32_MAX. */
uint32_t sl_engine_state_buffer(const sl_engine *engine, uint32_t value);

void sl_engine_destroy(sl_engine *engine);

/* The greedy choice the loops above make over one row of logits: the first
 * index of the largest value (strict >, so ties keep the first; a NaN is
 * never taken past index 0), as one sequential scan gives it. Host code
 * only (no device call). */
uint32_t sl_engine_first_argmax(const float *logits, size_t n);

#ifdef __cplusplus
}
#endif

#endif /* STARLIGHT_ENGINE_H */
