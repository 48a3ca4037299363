// slots.h -- library-internal: slotted batches (runtime.cpp), the device side of the request
// server (server.cpp). Functions return an MGX_* status and leave the message for
// mgx_last_error on the calling thread.
#pragma once
#include "mgx.h"

struct mgx_slots;

#define MGX_HIDDEN __attribute__((visibility("hidden")))

// n slots of cpr streams (2: guided requests allowed), requests of up to max_gen steps and
// max_ctx conditioning tokens; keep_steps keeps every step's mixed logits.
MGX_HIDDEN int mgx_internal_slots_create(mgx_model* m, int n, int cpr, int max_gen, int max_ctx, int keep_steps,
                                         mgx_slots** out);
MGX_HIDDEN int mgx_internal_slot_check(const mgx_slots* sl, const mgx_batch_request* q, int n_ctx, int prompt_len);
MGX_HIDDEN int mgx_internal_slot_open(mgx_slots* sl, int r, const mgx_batch_request* q, int n_ctx, int prompt_len);
MGX_HIDDEN int mgx_internal_slots_run(mgx_slots* sl, int steps);
MGX_HIDDEN int mgx_internal_slots_sync(mgx_slots* sl);
MGX_HIDDEN int mgx_internal_slot_read(mgx_slots* sl, int r, int32_t* codes_out, float* first_out, float* steps_out);
// host view: live, the next position, the loop start and end
MGX_HIDDEN void mgx_internal_slot_state(const mgx_slots* sl, int r, int* live, int* pos, int* start, int* S);
MGX_HIDDEN uint64_t mgx_internal_slot_cache_bytes(const mgx_slots* sl);
MGX_HIDDEN void mgx_internal_slots_destroy(mgx_slots* sl);
MGX_HIDDEN int mgx_internal_set_error(int code, const char* msg);
