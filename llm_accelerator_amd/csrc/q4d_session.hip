// Host-side decode session: serial prompt prefill, greedy token feedback, stop
// reasons and the context cap, one model invocation per step, with the event stream
// of the reference's board session loop (FPGA_Project/software/qmap_prompt_demo/
// qot_session.h and qot_session.c:101-276).  The runner performs one full-model token
// invocation; the runners at the end of this file are the GPU decode step
// (q4d_run_one_token) and the fixed-point GPU step (q4d_fixed_run_one_token).
//
// Model: the session is a cursor over one input stream.  The stream is the prompt
// followed by the model's own outputs; input i runs at position start_position + i.
// The contract, as rules:
//   R1  the outputs for all prompt inputs but the last are discarded (PREFILL events);
//       every later output is a generated token (TOKEN event) and the next input;
//   R2  after a generated token, the first rule of kStopRules that holds ends the
//       stream: the session parks in STOPPING and its next step reports DONE;
//   R3  a feedback step that finds the stream at the context cap reports DONE with
//       stop reason CONTEXT and runs nothing;
//   R4  a runner error, or an output outside the vocabulary, ends the session in
//       ERROR (stop reason HW_ERROR, the error code in the event).
// q4d_session_begin validates in the order of kBeginChecks (the first failing check
// gives the return code), then rewinds the cursor onto the prompt; q4d_session_reset
// rewinds it to IDLE without one.
#include <string.h>

#include "q4d_internal.h"

namespace {

using Session = q4d_session_t;
using Event = q4d_session_event_t;
using Options = q4d_session_options_t;

// R2, in priority order: when several hold, the first one is the reported reason.
struct StopRule {
  int32_t reason;
  bool (*holds)(const Session& s, uint32_t token);
};
const StopRule kStopRules[] = {
    {Q4D_SESSION_STOP_EOS,
     [](const Session& s, uint32_t t) { return s.options.stop_on_eos != 0 && t == s.options.eos_token_id; }},
    {Q4D_SESSION_STOP_IM_END,
     [](const Session& s, uint32_t t) { return s.options.stop_on_im_end != 0 && t == s.options.im_end_token_id; }},
    {Q4D_SESSION_STOP_MAX_NEW, [](const Session& s, uint32_t) { return s.generated_count >= s.options.max_new_tokens; }},
    {Q4D_SESSION_STOP_CONTEXT, [](const Session& s, uint32_t) { return s.next_position >= s.max_context; }},
};

int32_t first_stop_rule(const Session& s, uint32_t token) {
  for (const StopRule& r : kStopRules)
    if (r.holds(s, token)) return r.reason;
  return Q4D_SESSION_STOP_NONE;
}

// Preconditions of q4d_session_begin, in priority order.
struct BeginArgs {
  const Session& s;
  const uint32_t* prompt;
  uint32_t count;
  const Options& o;
};
bool out_of_vocab(const BeginArgs& a, uint32_t id) { return id >= a.s.vocab_size; }
struct BeginCheck {
  int code;
  bool (*fails)(const BeginArgs& a);
};
const BeginCheck kBeginChecks[] = {
    {Q4D_SESSION_ERR_STATE,
     [](const BeginArgs& a) { return a.s.state == Q4D_SESSION_STATE_UNINITIALIZED || a.s.runner == nullptr; }},
    {Q4D_ERR_CAPACITY, [](const BeginArgs& a) { return a.count == 0; }},
    {Q4D_ERR_CAPACITY, [](const BeginArgs& a) { return a.o.max_new_tokens == 0; }},
    {Q4D_ERR_BAD_TOKEN,
     [](const BeginArgs& a) {
       return (a.o.stop_on_eos != 0 && out_of_vocab(a, a.o.eos_token_id)) ||
              (a.o.stop_on_im_end != 0 && out_of_vocab(a, a.o.im_end_token_id));
     }},
    {Q4D_ERR_BAD_TOKEN,
     [](const BeginArgs& a) {
       for (uint32_t i = 0; i < a.count; ++i)
         if (out_of_vocab(a, a.prompt[i])) return true;
       return false;
     }},
    {Q4D_ERR_CONTEXT, [](const BeginArgs& a) { return uint64_t(a.s.start_position) + a.count > a.s.max_context; }},
};

// Puts the cursor at the start of a stream (begin: the prompt; reset: none).
void rewind(Session& s, const uint32_t* prompt, uint32_t count, int32_t state) {
  s.prompt = prompt;
  s.prompt_count = count;
  s.prompt_index = 0;
  s.generated_count = 0;
  s.pending_token = 0;
  s.next_position = s.start_position;
  s.last_result = q4d_token_result_t{};
  s.last_error = Q4D_OK;
  s.stop_reason = Q4D_SESSION_STOP_NONE;
  s.state = state;
}

// The event a step reports.  Which counters an event carries depends on its kind:
// DONE the final counts; PREFILL / TOKEN the input and the counts so far; ERROR only
// the input that failed.
Event make_event(const Session& s, int32_t kind, uint32_t token, uint32_t position) {
  Event e{};  // kind NONE, stop reason NONE, error code OK
  e.kind = kind;
  e.result = s.last_result;
  switch (kind) {
    case Q4D_SESSION_EVENT_DONE:
      e.stop_reason = s.stop_reason;
      e.prompt_tokens_consumed = s.prompt_index;
      e.generated_index = s.generated_count;
      break;
    case Q4D_SESSION_EVENT_ERROR:
      e.input_token_id = token;
      e.input_position = position;
      e.stop_reason = s.stop_reason;
      e.error_code = s.last_error;
      break;
    case Q4D_SESSION_EVENT_TOKEN:
      e.generated_index = s.generated_count - 1;
      [[fallthrough]];
    default:  // PREFILL
      e.input_token_id = token;
      e.input_position = position;
      e.prompt_tokens_consumed = s.prompt_index;
      break;
  }
  return e;
}

// What a step does before any model work, from the state alone.
enum class Action { kReject, kReportStop, kReportCap, kRunModel };
Action plan(const Session& s) {
  switch (s.state) {
    case Q4D_SESSION_STATE_STOPPING: return Action::kReportStop;
    case Q4D_SESSION_STATE_PREFILL: return Action::kRunModel;
    case Q4D_SESSION_STATE_DECODE: return s.next_position >= s.max_context ? Action::kReportCap : Action::kRunModel;
    default: return Action::kReject;
  }
}

// R3 and the report that follows R2: the stream ends with `reason`.
int finish(Session& s, Event* ev, int32_t reason) {
  s.stop_reason = reason;
  s.state = Q4D_SESSION_STATE_DONE;
  *ev = make_event(s, Q4D_SESSION_EVENT_DONE, 0, 0);
  return Q4D_OK;
}

// One model invocation on input (token, position), then R1 / R2 / R4.
int run_model(Session& s, Event* ev) {
  const bool prompt_input = s.state == Q4D_SESSION_STATE_PREFILL;
  const uint32_t token = prompt_input ? s.prompt[s.prompt_index] : s.pending_token;
  const uint32_t position = s.next_position;
  s.last_result = q4d_token_result_t{};
  int rc = s.runner(s.runner_context, token, position, &s.last_result);
  if (rc == Q4D_OK && s.last_result.token_id >= s.vocab_size) rc = Q4D_ERR_BAD_TOKEN;
  if (rc != Q4D_OK) {  // R4
    s.last_error = rc;
    s.stop_reason = Q4D_SESSION_STOP_HW_ERROR;
    s.state = Q4D_SESSION_STATE_ERROR;
    *ev = make_event(s, Q4D_SESSION_EVENT_ERROR, token, position);
    return rc;
  }
  s.next_position += 1;
  if (prompt_input) s.prompt_index += 1;
  if (prompt_input && s.prompt_index < s.prompt_count) {  // R1: a prompt prediction, dropped
    *ev = make_event(s, Q4D_SESSION_EVENT_PREFILL, token, position);
    return Q4D_OK;
  }
  s.generated_count += 1;  // R1: a generated token, the next input
  s.pending_token = s.last_result.token_id;
  *ev = make_event(s, Q4D_SESSION_EVENT_TOKEN, token, position);
  const int32_t reason = first_stop_rule(s, s.pending_token);  // R2
  ev->stop_reason = reason;
  if (reason != Q4D_SESSION_STOP_NONE) s.stop_reason = reason;
  s.state = reason != Q4D_SESSION_STOP_NONE ? Q4D_SESSION_STATE_STOPPING : Q4D_SESSION_STATE_DECODE;
  return Q4D_OK;
}

const char* lookup_name(int32_t value, const char* const* names, int32_t count) {
  return value >= 0 && value < count ? names[value] : "UNKNOWN";
}

// Host <-> device staging of one runner call: token and position in, next token and
// score out, through the caller's device buffer (no allocation here).
struct StepIo {
  int32_t token, position, next, pad;
};

}  // namespace

extern "C" {

void q4d_session_default_options(q4d_session_options_t* o) {
  if (o) *o = Options{/*max_new_tokens=*/1, Q4D_SESSION_DEFAULT_EOS_TOKEN_ID, Q4D_SESSION_DEFAULT_IM_END_TOKEN_ID,
                      /*stop_on_eos=*/1, /*stop_on_im_end=*/1};
}

int q4d_session_init(q4d_session_t* s, uint32_t start_position, uint32_t max_context, uint32_t vocab_size,
                     q4d_session_runner_fn runner, void* runner_context) {
  if (!s || !runner) return Q4D_ERR_NULL;
  if (max_context == 0 || start_position >= max_context) return Q4D_ERR_CONTEXT;
  if (vocab_size == 0) return Q4D_ERR_SHAPE;
  *s = Session{};
  s->start_position = start_position;
  s->max_context = max_context;
  s->vocab_size = vocab_size;
  s->runner = runner;
  s->runner_context = runner_context;
  s->state = Q4D_SESSION_STATE_IDLE;  // no stream yet: counters, error and stop reason stay zero
  return Q4D_OK;
}

int q4d_session_begin(q4d_session_t* s, const uint32_t* prompt, uint32_t prompt_count,
                      const q4d_session_options_t* options) {
  if (!s || !prompt) return Q4D_ERR_NULL;
  Options o;
  q4d_session_default_options(&o);
  if (options) o = *options;
  const BeginArgs args{*s, prompt, prompt_count, o};
  for (const BeginCheck& c : kBeginChecks)
    if (c.fails(args)) return c.code;
  s->options = o;
  rewind(*s, prompt, prompt_count, Q4D_SESSION_STATE_PREFILL);
  return Q4D_OK;
}

int q4d_session_step(q4d_session_t* s, q4d_session_event_t* ev) {
  if (!s || !ev) return Q4D_ERR_NULL;
  *ev = Event{};
  switch (plan(*s)) {
    case Action::kReportStop: return finish(*s, ev, s->stop_reason);
    case Action::kReportCap: return finish(*s, ev, Q4D_SESSION_STOP_CONTEXT);
    case Action::kRunModel: return run_model(*s, ev);
    case Action::kReject: break;
  }
  return Q4D_SESSION_ERR_STATE;
}

void q4d_session_reset(q4d_session_t* s) {
  if (s && s->state != Q4D_SESSION_STATE_UNINITIALIZED) rewind(*s, nullptr, 0, Q4D_SESSION_STATE_IDLE);
}

int q4d_session_is_terminal(const q4d_session_t* s) {
  return s == nullptr || s->state == Q4D_SESSION_STATE_DONE || s->state == Q4D_SESSION_STATE_ERROR;
}

const char* q4d_session_state_name(int32_t state) {
  static const char* const kNames[] = {"UNINITIALIZED", "IDLE", "PREFILL", "DECODE", "STOPPING", "DONE", "ERROR"};
  return lookup_name(state, kNames, 7);
}

const char* q4d_session_stop_reason_name(int32_t reason) {
  static const char* const kNames[] = {"NONE", "EOS", "IM_END", "MAX_NEW", "CONTEXT", "HW_ERROR"};
  return lookup_name(reason, kNames, 6);
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
