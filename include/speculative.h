/*
 * speculative.h -- speculative decoding (reference include/speculative.h:8-15).
 *
 * Same five entry points.  The generate loop drafts k tokens with the draft
 * model, verifies all k+1 positions of the target in ONE batched forward on
 * the GPU and applies the acceptance rule on the GPU.  Uniform draws come from
 * a seeded counter-based stream (vx_speculative_set_seed in veltrix_gpu.h)
 * instead of libc rand().  max_draft_tokens is 1..15 (a verify batch holds at
 * most 16 rows); vx_speculative_create returns NULL outside that range or for
 * a NULL model (the reference accepts any count).
 */
#ifndef VX_SPECULATIVE_H
#define VX_SPECULATIVE_H

#include "veltrix.h"

typedef struct vx_speculative_state vx_speculative_state;

vx_speculative_state *vx_speculative_create(vx_model *draft, vx_model *target, int max_draft_tokens);
void vx_speculative_destroy(vx_speculative_state *state);
void vx_speculative_set_temp(vx_speculative_state *state, float temp, float top_p);

int vx_speculative_generate(vx_speculative_state *state, int *prompt, int prompt_len,
                            int *output, int max_tokens);
int vx_speculative_generate_stream(vx_speculative_state *state, int token,
                                   int *output, int max_tokens);

#endif
