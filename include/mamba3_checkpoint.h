/* Weight ingestion for the gfx950 Mamba-3 path: the reference's JSON
 * checkpoints and state dicts, read and written on the host.
 *
 *   entry point               replaces                              reference
 *   m3_checkpoint_load        Checkpoint::load                      src/train/checkpoint.rs:61-65
 *   m3_state_dict_load        StateDict::load                       src/nn/module.rs:325-329
 *   m3_state_dict_save        StateDict::save / Checkpoint::save    src/nn/module.rs:318-322,
 *                                                                   src/train/checkpoint.rs:54-58
 *   m3_state_dict_len / _entry / _find / _free, m3_checkpoint_step / _metadata
 *                             the fields of StateDict, TensorData   src/nn/module.rs:297-314
 *                             and Checkpoint                        src/train/checkpoint.rs:16-25
 *
 * The format is serde_json's encoding of those structs:
 *   Checkpoint: {"step": u64, "state": {"entries": {...}}, "metadata": <any JSON>}
 *   StateDict:  {"entries": {path: {"shape": [usize...], "data": [f32...]}, ...}}
 * with entries in key order (a BTreeMap).  Numbers are read as the nearest
 * double and then rounded to f32, as serde_json does; `null` in `data` (how
 * serde_json writes a non-finite f32) fails to load, as there.  The `data`
 * arrays are parsed by several host threads.  Nothing here touches the GPU.
 */
#ifndef MAMBA3_CHECKPOINT_H
#define MAMBA3_CHECKPOINT_H

#include <stddef.h>
#include <stdint.h>

#include "mamba3_ssm.h"

#ifdef __cplusplus
extern "C" {
#endif

/* A loaded state dict (and, for a checkpoint, its step and metadata). */
typedef struct m3_state_dict m3_state_dict;

/* Parse a checkpoint file ("step" and "state" required, "metadata" optional)
 * or a bare state dict file ("entries" required).  Unknown fields are
 * skipped; a repeated key keeps its last value.  M3_ERR_IO when the file
 * cannot be read, M3_ERR_JSON for malformed JSON or a missing field. */
m3_status m3_checkpoint_load(const char *path, m3_state_dict **out);
m3_status m3_state_dict_load(const char *path, m3_state_dict **out);
void m3_state_dict_free(m3_state_dict *sd);

/* Entries in key order.  `shape` and `data` stay valid until
 * m3_state_dict_free; `numel` is the length of `data` as read (it is not
 * checked against the shape here, as the reference checks it on restore). */
size_t m3_state_dict_len(const m3_state_dict *sd);
m3_status m3_state_dict_entry(const m3_state_dict *sd, size_t index, const char **name,
                              size_t *ndim, const size_t **shape, const float **data,
                              size_t *numel);
/* Index of `name`, or -1. */
int64_t m3_state_dict_find(const m3_state_dict *sd, const char *name);

/* The checkpoint's step (0 for a bare state dict) and its metadata as JSON
 * text ("null" when absent). */
uint64_t m3_checkpoint_step(const m3_state_dict *sd);
const char *m3_checkpoint_metadata(const m3_state_dict *sd);

/* Write n entries as a state dict (`as_checkpoint` = 0) or as a checkpoint
 * with `step` and `metadata_json` (valid JSON text, or NULL for null).
 * Entries are sorted by name; a repeated name is M3_ERR_ARGUMENT.  f32 values
 * are written in their shortest round-trip form, non-finite ones as null. */
m3_status m3_state_dict_save(const char *path, int32_t as_checkpoint, uint64_t step,
                             const char *metadata_json, size_t n, const char *const *names,
                             const size_t *ndims, const size_t *const *shapes,
                             const float *const *data, const size_t *numels);

#ifdef __cplusplus
}
#endif

#endif /* MAMBA3_CHECKPOINT_H */
