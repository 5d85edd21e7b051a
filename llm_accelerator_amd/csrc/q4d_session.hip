// Host-side decode session: serial prompt prefill, greedy token feedback, stop
// reasons and the context cap, one model invocation per step.  Same state machine
// and event stream as the reference's board session loop
// (FPGA_Project/software/qmap_prompt_demo/qot_session.c:101-276): a runner performs
// one full-model token invocation; the default runners here are the GPU decode step
// (q4d_run_one_token) and the fixed-point GPU step (q4d_fixed_run_one_token).
#include <string.h>

#include "q4d_internal.h"

namespace {

void clear_event(q4d_session_event_t* ev) {
  memset(ev, 0, sizeof(*ev));
  ev->kind = Q4D_SESSION_EVENT_NONE;
  ev->stop_reason = Q4D_SESSION_STOP_NONE;
  ev->error_code = Q4D_OK;
}

// Event fields shared by every terminal report (DONE after STOPPING, DONE at the cap).
void report_done(q4d_session_t* s, q4d_session_event_t* ev) {
  ev->kind = Q4D_SESSION_EVENT_DONE;
  ev->stop_reason = s->stop_reason;
  ev->prompt_tokens_consumed = s->prompt_index;
  ev->generated_index = s->generated_count;
  ev->result = s->last_result;
}

int fail(q4d_session_t* s, q4d_session_event_t* ev, int code) {
  s->last_error = code;
  s->stop_reason = Q4D_SESSION_STOP_HW_ERROR;
  s->state = Q4D_SESSION_STATE_ERROR;
  ev->kind = Q4D_SESSION_EVENT_ERROR;
  ev->stop_reason = s->stop_reason;
  ev->error_code = code;
  ev->result = s->last_result;
  return code;
}

// Why generation ends after the token just produced, checked in this order:
// end-of-text, end-of-turn, the new-token budget, the context cap.
int32_t stop_after(const q4d_session_t* s, uint32_t token) {
  const q4d_session_options_t& o = s->options;
  if (o.stop_on_eos && token == o.eos_token_id) return Q4D_SESSION_STOP_EOS;
  if (o.stop_on_im_end && token == o.im_end_token_id) return Q4D_SESSION_STOP_IM_END;
  if (s->generated_count >= o.max_new_tokens) return Q4D_SESSION_STOP_MAX_NEW;
  if (s->next_position >= s->max_context) return Q4D_SESSION_STOP_CONTEXT;
  return Q4D_SESSION_STOP_NONE;
}

// Host <-> device staging of one runner call: token and position in, next token and
// score out, through the caller's device buffer (no allocation here).
struct StepIo {
  int32_t token, position, next, pad;
};

}  // namespace

extern "C" {

void q4d_session_default_options(q4d_session_options_t* o) {
  if (!o) return;
  memset(o, 0, sizeof(*o));
  o->max_new_tokens = 1;
  o->eos_token_id = Q4D_SESSION_DEFAULT_EOS_TOKEN_ID;
  o->im_end_token_id = Q4D_SESSION_DEFAULT_IM_END_TOKEN_ID;
  o->stop_on_eos = 1;
  o->stop_on_im_end = 1;
}

int q4d_session_init(q4d_session_t* s, uint32_t start_position, uint32_t max_context, uint32_t vocab_size,
                     q4d_session_runner_fn runner, void* runner_context) {
  if (!s || !runner) return Q4D_ERR_NULL;
  if (max_context == 0 || start_position >= max_context) return Q4D_ERR_CONTEXT;
  if (vocab_size == 0) return Q4D_ERR_SHAPE;
  memset(s, 0, sizeof(*s));
  s->start_position = start_position;
  s->max_context = max_context;
  s->vocab_size = vocab_size;
  s->runner = runner;
  s->runner_context = runner_context;
  s->last_error = Q4D_OK;
  s->state = Q4D_SESSION_STATE_IDLE;
  s->stop_reason = Q4D_SESSION_STOP_NONE;
  return Q4D_OK;
}

int q4d_session_begin(q4d_session_t* s, const uint32_t* prompt, uint32_t prompt_count,
                      const q4d_session_options_t* options) {
  if (!s || !prompt) return Q4D_ERR_NULL;
  if (s->state == Q4D_SESSION_STATE_UNINITIALIZED || !s->runner) return Q4D_SESSION_ERR_STATE;
  if (prompt_count == 0) return Q4D_ERR_CAPACITY;
  q4d_session_options_t o;
  q4d_session_default_options(&o);
  if (options) o = *options;
  if (o.max_new_tokens == 0) return Q4D_ERR_CAPACITY;
  if ((o.stop_on_eos && o.eos_token_id >= s->vocab_size) || (o.stop_on_im_end && o.im_end_token_id >= s->vocab_size))
    return Q4D_ERR_BAD_TOKEN;
  for (uint32_t i = 0; i < prompt_count; ++i)
    if (prompt[i] >= s->vocab_size) return Q4D_ERR_BAD_TOKEN;
  if ((uint64_t)s->start_position + prompt_count > (uint64_t)s->max_context) return Q4D_ERR_CONTEXT;
  s->prompt = prompt;
  s->prompt_count = prompt_count;
  s->prompt_index = 0;
  s->next_position = s->start_position;
  s->pending_token = 0;
  s->generated_count = 0;
  s->options = o;
  memset(&s->last_result, 0, sizeof(s->last_result));
  s->last_error = Q4D_OK;
  s->stop_reason = Q4D_SESSION_STOP_NONE;
  s->state = Q4D_SESSION_STATE_PREFILL;
  return Q4D_OK;
}

int q4d_session_step(q4d_session_t* s, q4d_session_event_t* ev) {
  if (!s || !ev) return Q4D_ERR_NULL;
  clear_event(ev);
  switch (s->state) {
    case Q4D_SESSION_STATE_STOPPING:  // the stop was decided with the last token: report it
      s->state = Q4D_SESSION_STATE_DONE;
      report_done(s, ev);
      return Q4D_OK;
    case Q4D_SESSION_STATE_PREFILL:
    case Q4D_SESSION_STATE_DECODE:
      break;
    default:
      return Q4D_SESSION_ERR_STATE;
  }
  const bool prefill = s->state == Q4D_SESSION_STATE_PREFILL;
  if (!prefill && s->next_position >= s->max_context) {
    s->stop_reason = Q4D_SESSION_STOP_CONTEXT;
    s->state = Q4D_SESSION_STATE_DONE;
    report_done(s, ev);
    return Q4D_OK;
  }
  const uint32_t token = prefill ? s->prompt[s->prompt_index] : s->pending_token;
  const uint32_t position = s->next_position;
  memset(&s->last_result, 0, sizeof(s->last_result));
  const int rc = s->runner(s->runner_context, token, position, &s->last_result);
  if (rc != Q4D_OK || s->last_result.token_id >= s->vocab_size) {
    ev->input_token_id = token;
    ev->input_position = position;
    return fail(s, ev, rc != Q4D_OK ? rc : Q4D_ERR_BAD_TOKEN);
  }
  ++s->next_position;
  ev->input_token_id = token;
  ev->input_position = position;
  ev->result = s->last_result;
  if (prefill) {
    ++s->prompt_index;
    if (s->prompt_index < s->prompt_count) {  // prompt not consumed yet: its prediction is dropped
      ev->kind = Q4D_SESSION_EVENT_PREFILL;
      ev->prompt_tokens_consumed = s->prompt_index;
      return Q4D_OK;
    }
  }
  // a generated token: fed back as the next input unless a stop condition holds
  s->pending_token = s->last_result.token_id;
  ++s->generated_count;
  ev->kind = Q4D_SESSION_EVENT_TOKEN;
  ev->prompt_tokens_consumed = s->prompt_index;
  ev->generated_index = s->generated_count - 1;
  const int32_t why = stop_after(s, s->last_result.token_id);
  if (why != Q4D_SESSION_STOP_NONE) {
    s->stop_reason = why;
    s->state = Q4D_SESSION_STATE_STOPPING;
    ev->stop_reason = why;
  } else {
    s->state = Q4D_SESSION_STATE_DECODE;
  }
  return Q4D_OK;
}

void q4d_session_reset(q4d_session_t* s) {
  if (!s || s->state == Q4D_SESSION_STATE_UNINITIALIZED) return;
  s->prompt = nullptr;
  s->prompt_count = 0;
  s->prompt_index = 0;
  s->next_position = s->start_position;
  s->pending_token = 0;
  s->generated_count = 0;
  memset(&s->last_result, 0, sizeof(s->last_result));
  s->last_error = Q4D_OK;
  s->state = Q4D_SESSION_STATE_IDLE;
  s->stop_reason = Q4D_SESSION_STOP_NONE;
}

int q4d_session_is_terminal(const q4d_session_t* s) {
  return !s || s->state == Q4D_SESSION_STATE_DONE || s->state == Q4D_SESSION_STATE_ERROR;
}

const char* q4d_session_state_name(int32_t state) {
  static const char* const names[] = {"UNINITIALIZED", "IDLE", "PREFILL", "DECODE", "STOPPING", "DONE", "ERROR"};
  return state >= 0 && state < 7 ? names[state] : "UNKNOWN";
}

const char* q4d_session_stop_reason_name(int32_t reason) {
  static const char* const names[] = {"NONE", "EOS", "IM_END", "MAX_NEW", "CONTEXT", "HW_ERROR"};
  return reason >= 0 && reason < 6 ? names[reason] : "UNKNOWN";
}

// One decode step on the GPU: stage (token, position), run q4d_run_one_token, read back
// the argmax and its logit.  Synchronises the runner's stream (one host event per token,
// as the board loop polls per token).
int q4d_session_gpu_runner(void* context, uint32_t token, uint32_t position, q4d_token_result_t* result) {
  const q4d_gpu_runner_t* r = static_cast<const q4d_gpu_runner_t*>(context);
  if (!r || !r->model || !r->kv || !r->io || !result) return Q4D_ERR_NULL;
  hipStream_t st = reinterpret_cast<hipStream_t>(r->stream);
  StepIo io{(int32_t)token, (int32_t)position, 0, 0};
  int32_t* d = r->io;  // device int32[8]: token, position, next token, pad, score (fp32 bits), ...
  if (hipMemcpyAsync(d, &io, 2 * sizeof(int32_t), hipMemcpyHostToDevice, st) != hipSuccess) return Q4D_ERR_LAUNCH;
  int rc = q4d_run_one_token(r->model, d, d + 1, r->kv, d + 2, reinterpret_cast<float*>(d + 4), nullptr, r->ws,
                             r->ws_bytes, r->stream);
  if (rc) return rc;
  int32_t out[4];
  if (hipMemcpyAsync(out, d + 2, sizeof(out), hipMemcpyDeviceToHost, st) != hipSuccess) return Q4D_ERR_LAUNCH;
  if (hipStreamSynchronize(st) != hipSuccess) return Q4D_ERR_LAUNCH;
  int32_t status = 0;
  if ((rc = q4d_read_status(r->ws, r->ws_bytes, r->model, 1, &status, r->stream))) return rc;
  result->status = (uint32_t)status;
  if (status) return Q4D_ERR_STATUS;
  result->token_id = (uint32_t)out[0];
  memcpy(&result->score, &out[2], sizeof(float));
  result->score_q26 = 0;
  return Q4D_OK;
}

// One fixed-point decode step on the GPU (q4d_fixed_run_one_token): the argmax and its
// Q26 score, as the board's qot_run_token returns them.
int q4d_session_fixed_runner(void* context, uint32_t token, uint32_t position, q4d_token_result_t* result) {
  const q4d_fixed_runner_t* r = static_cast<const q4d_fixed_runner_t*>(context);
  if (!r || !r->model || !r->kv || !r->io || !result) return Q4D_ERR_NULL;
  hipStream_t st = reinterpret_cast<hipStream_t>(r->stream);
  StepIo io{(int32_t)token, (int32_t)position, 0, 0};
  int32_t* d = r->io;  // device int32[8]: token, position, next token, pad, score (int64 at d + 4)
  if (hipMemcpyAsync(d, &io, 2 * sizeof(int32_t), hipMemcpyHostToDevice, st) != hipSuccess) return Q4D_ERR_LAUNCH;
  int rc = q4d_fixed_run_one_token(r->model, d, d + 1, r->kv, d + 2, reinterpret_cast<int64_t*>(d + 4), nullptr,
                                   nullptr, r->ws, r->ws_bytes, r->stream);
  if (rc) return rc;
  int32_t out[4];
  if (hipMemcpyAsync(out, d + 2, sizeof(out), hipMemcpyDeviceToHost, st) != hipSuccess) return Q4D_ERR_LAUNCH;
  int32_t counts[1] = {0};
  if ((rc = q4d_fixed_read_counts(r->ws, r->ws_bytes, counts, 1, r->stream))) return rc;  // synchronises
  result->status = (uint32_t)counts[0];
  if (counts[0]) return Q4D_ERR_STATUS;
  result->token_id = (uint32_t)out[0];
  int64_t sc;
  memcpy(&sc, &out[2], sizeof(sc));
  result->score_q26 = sc;
  result->score = 0.f;
  return Q4D_OK;
}

}  // extern "C"
