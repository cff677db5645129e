/*
 * dmx_ckpt.h — checkpoint readers of the MI355X HTDemucs backend (host code,
 * no GPU needed). They turn a checkpoint file into the named f32 tensors and
 * the config that dmx_runner_create takes, the job of the reference's
 * `load_weights` (crates/demucs-core/src/demucs/weights.rs:30-88).
 *
 * Conventions as in dmx.h: `int` results are DMX_OK or a DMX_ERR_* code with a
 * message in dmx_last_error(). A checkpoint owns its tensors; pointers into it
 * stay valid until dmx_checkpoint_free.
 */
#ifndef DMX_CKPT_H
#define DMX_CKPT_H

#include "dmx.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct dmx_checkpoint dmx_checkpoint;

/* load_weights (weights.rs:56-88): ".th" / ".pth" / ".pt" are torch.save zips
 * (Checkpoint::load, crates/demucs-core/src/ckpt/mod.rs:43-47), anything else is
 * safetensors (SafeTensors::load, crates/demucs-core/src/safetensors.rs:27-32).
 * Errors: DMX_ERR_IO (the file), DMX_ERR_CHECKPOINT (its contents),
 * DMX_ERR_CONFIG (safetensors kwargs that are not a valid config). */
int dmx_checkpoint_load(const char *path, dmx_checkpoint **out);

/* load_weights_from_bytes (weights.rs:30-50): torch_zip != 0 for a torch.save
 * archive, 0 for safetensors. */
int dmx_checkpoint_from_bytes(const void *bytes, size_t len, int torch_zip, dmx_checkpoint **out);

void dmx_checkpoint_free(dmx_checkpoint *ckpt);

/* The tensors, sorted by name, as dmx_tensor entries (f32, row-major, at most
 * 4 dimensions) that dmx_runner_create accepts as they are. */
size_t dmx_checkpoint_count(const dmx_checkpoint *ckpt);
const dmx_tensor *dmx_checkpoint_tensors(const dmx_checkpoint *ckpt);

/* safetensors `__metadata__` (string values only; none for torch zips):
 * the value for `key` or NULL, and the keys in sorted order. */
const char *dmx_checkpoint_metadata(const dmx_checkpoint *ckpt, const char *key);
size_t dmx_checkpoint_metadata_count(const dmx_checkpoint *ckpt);
const char *dmx_checkpoint_metadata_key(const dmx_checkpoint *ckpt, size_t index);

/* The model config: from the safetensors "kwargs" entry when there is one,
 * HtdemucsConfig::default otherwise (weights.rs:40-44, 76-79). */
int dmx_checkpoint_config(const dmx_checkpoint *ckpt, dmx_config *out);

/* HtdemucsConfig::from_kwargs_json (crates/demucs-core/src/demucs/config.rs:150-215):
 * known keys override the defaults, unknown keys are ignored, `segment` is a
 * number or {"numerator", "denominator"}. DMX_ERR_CONFIG when the text is not
 * a JSON object of that form. */
int dmx_config_from_kwargs(const char *json, dmx_config *out);

#ifdef __cplusplus
}
#endif

#endif /* DMX_CKPT_H */
