/*
 * moert_policy.h -- the expert residency policy: the page table
 * (exp_slot / slot_exp / slot_state), the routing scores, the cost-aware
 * promotion decision and its telemetry.  Host code only, no HIP.
 *
 * Replaces moert/include/moert/policy.h (the declarations below keep its
 * names, argument meaning and struct layouts, so a host linked against the
 * reference's moert policy links against this one unchanged).  Every
 * decision is the reference's: the use-rate EMA and its forecast
 * f = H * min(1, rate * (1 - decay)), the pairing of the best non-residents
 * with free slots while f_in > r and then with the worst residents while
 * f_in - f_out > r, the pairs applied by descending net saving up to
 * cost_per_token per visible token (policy.cpp:250-340).
 *
 * Slot states: FREE 0, FILLING 1 (asynchronous promotion in flight: the
 * slot is occupied by its new expert, which the partition still serves
 * cold), READY 2 (the only hot state; policy.h:46-52).
 */
#ifndef MOERT_POLICY_HIP_H
#define MOERT_POLICY_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct moert_policy moert_policy;

/* policy.h:31-37 */
enum moert_refresh_reason {
    MOERT_REFRESH_PROMPT_END = 0,
    MOERT_REFRESH_VISIBLE_INTERVAL = 1,   /* capped at cost_per_token promotions */
    MOERT_REFRESH_TURN_END = 2,
    MOERT_REFRESH_BOUNDARY = 4,
};

/* policy.h:46 */
enum moert_slot_state { MOERT_SLOT_FREE = 0, MOERT_SLOT_FILLING = 1, MOERT_SLOT_READY = 2 };

/* policy.h:49-74 (layout is ABI) */
typedef struct moert_policy_config {
    int32_t n_layers, n_expert, k;
    float   seed_prior, session_decay, recent_decay;
    float   blend_a, blend_b, blend_c;
    const int32_t * k_per_layer;      /* n_layers capacities in [1, n_expert], or NULL */
    int32_t cost_horizon;             /* H */
    float   cost_reuse;               /* r */
    float   cost_rate_decay;
    int32_t cost_per_token;
} moert_policy_config;

/* policy.h:76-78: H 16, r 2, decay 0.5^(1/32), 4 per token; geometry zeroed. */
void moert_policy_config_defaults(moert_policy_config * cfg);

/* policy.h:82-104.  stream_expert returns 1 (bytes in place: READY), 2
 * (accepted asynchronously: FILLING) or 0 (failed). */
typedef struct moert_policy_callbacks {
    int32_t (*stream_expert)(void * user, int32_t il, int32_t e, int32_t slot);
    void (*publish_layer)(void * user, int32_t il);
    void (*fetch_external)(void * user);
    void * user;
} moert_policy_callbacks;

/* policy.h:107-118 */
typedef struct moert_policy_stats {
    int64_t promotions, demotions, tokens, visible_tokens;
    int64_t hot_routes, cold_routes;
    int64_t refresh_count, refresh_promotions, refresh_demotions;
    double  refresh_pause_ms_total, refresh_pause_ms_max;
    int64_t last_refresh_tok, last_refresh_promos;
    double  last_refresh_pause_ms;
    double  occupancy;
    int64_t fills_async, fills_completed, fills_stale, fills_aborted;
} moert_policy_stats;

moert_policy * moert_policy_create(const moert_policy_config * cfg, const moert_policy_callbacks * cbs);
void moert_policy_free(moert_policy * p);
void moert_policy_set_external_observation(moert_policy * p, int32_t on);
void moert_policy_observe(moert_policy * p, int32_t il, const int32_t * ids, int32_t n_used, int64_t n_tok);
void moert_policy_on_prompt_token(moert_policy * p, int64_t n_tokens);
void moert_policy_on_token_end(moert_policy * p);
void moert_policy_refresh(moert_policy * p, int32_t reason);
int32_t moert_policy_resize_k(moert_policy * p, int32_t k_new);
int32_t moert_policy_set_active_k(moert_policy * p, int32_t k);
int32_t moert_policy_can_seed(const moert_policy * p, int32_t il, int32_t e);
int32_t moert_policy_commit_seed(moert_policy * p, int32_t il, int32_t e, int32_t slot);
int32_t moert_policy_complete_fill(moert_policy * p, int32_t il, int32_t slot, int32_t e);
int32_t moert_policy_abort_fill(moert_policy * p, int32_t il, int32_t slot, int32_t e);
int32_t moert_policy_boundary_layer(moert_policy * p, int32_t il, const int32_t * counts, int64_t n_tok,
                                    float weight, float r);
void moert_policy_add_external_counts(moert_policy * p, int32_t il, const int32_t * counts, int64_t hot,
                                      int64_t cold);
void moert_policy_reset_stats(moert_policy * p);
int32_t moert_policy_layer_k(const moert_policy * p, int32_t il);
void moert_policy_set_external_forecast(moert_policy * p, const float * f, float r, int32_t cap);
double moert_policy_hit_rate(moert_policy * p);
void moert_policy_get_stats(moert_policy * p, moert_policy_stats * out);

/* policy.h:196-204 */
typedef struct moert_policy_window {
    int32_t tokens;
    double  span_ms;
    double  tok_per_s, ms_per_tok;
    double  hit_rate;
    int64_t hot_routes, cold_routes;
} moert_policy_window;
void moert_policy_get_window(moert_policy * p, int32_t n_tokens, moert_policy_window * out);

/* policy.h:214-218: the page table and the device-mirror sources; valid until
 * free (slot arrays until resize_k). */
const int32_t * moert_policy_exp_slot_view(const moert_policy * p, int32_t il);
const int32_t * moert_policy_slot_exp_view(const moert_policy * p, int32_t il);
const int32_t * moert_policy_slot_state_view(const moert_policy * p, int32_t il);
const int32_t * moert_policy_hotmap_view(const moert_policy * p, int32_t il);
const float *   moert_policy_resid_view(const moert_policy * p, int32_t il);

#ifdef __cplusplus
}
#endif
#endif
