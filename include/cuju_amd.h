/*
 * The C ABI of the MI355X batched football step engine (libcuju_amd.so). Each entry point is the
 * one the reference's Python binding calls for the same operation, with the same arguments and
 * error convention, so a ctypes binding written for the reference binds this library unchanged.
 *
 * Calls are synchronous unless noted. A failure returns -1 or null, and cuju_last_error() gives
 * the message (per thread). A `stream` is a HIP stream (hipStream_t), or null for the default
 * stream. Device pointers are HIP device memory of the current device.
 */
#ifndef CUJU_AMD_H
#define CUJU_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CUJU_CONFIGURATION_VERSION 2

/* The batch configuration, version 2: src/environment_api.h:49-95 of the reference. */
struct cuju_configuration {
    int version; /* CUJU_CONFIGURATION_VERSION */
    const char *const *assets; /* [asset_count] paths of .cjb bundles */
    int asset_count;
    const int *assignment; /* [environment_count] bundle indices, or null for bundle 0 */
    const char *animations; /* path of animations.bin */
    int environment_count;
    unsigned long long seed; /* env i plays GRF after random.seed(seed * 2**32 + first_index + i) */
    int action_set; /* 0 default, 1 v2, 2 full */
    int observation; /* bit mask: 1 simple115, 2 simple115v2, 4 SMM (extracted), 8 raw */
    int checkpoints; /* nonzero adds the checkpoint reward */
    int numpy_legacy; /* nonzero adds it as numpy before 2.0 does */
    int auto_reset; /* nonzero resets every environment whose episode ended within the step */
    int threads; /* host threads of the debugging backend; ignored by the GPU */
    int ticks_per_step; /* GRF physics_steps_per_frame, 10 there */
    int smm_width, smm_height; /* GRF channel_dimensions */
    int stack; /* 4 stacks observations as GRF's `stacked`, else 1 */
    const long long *fixed_seeds; /* [environment_count] GRF game_engine_random_seed, -1 draws; null draws all */
    const int *agent_counts; /* [asset_count][2] left/right agents, -1 keeps the bundle's; null keeps all */
    int episode_number; /* GRF episode_number */
    unsigned long long first_index; /* seed-rule index of environment 0 */
    /* device memory from the caller: null when it has none; released once the device is idle.
       Both null take hipMalloc and hipFree (src/environment_api.h:81-86) */
    void *(*allocate)(size_t bytes, void *context);
    void (*release)(void *pointer, void *context);
    void *allocator_context;
    int pin_threads; /* CPU-only options of the reference, ignored */
    int numa;
    int page_aligned;
};

/* src/environment_api.h:41 */
const char *cuju_last_error(void);
/* src/environment_api.h:44; "cuda", the torch device type of a HIP device on ROCm */
const char *cuju_backend(void);
/* src/environment_api.h:98 */
void *cuju_environment_create(const struct cuju_configuration *settings);
/* src/environment_api.h:161 */
int cuju_memory_estimate(const struct cuju_configuration *settings, unsigned long long *bytes);
/* src/environment_api.h:172 */
int cuju_local_memory_bytes(unsigned long long *bytes);
/* src/environment_api.h:186 */
unsigned long long cuju_environment_memory_bytes(void *environment);
/* src/environment_api.h:191 */
void cuju_environment_destroy(void *environment);
/* src/environment_api.h:195 */
int cuju_environment_count(void *environment);
/* src/environment_api.h:200 */
int cuju_environment_threads(void *environment);
/* No counterpart in the reference: the launch geometry the library chose for the batch, the
   environments in each wavefront, and in `lanes` the lanes that run each environment. */
int cuju_environment_geometry(void *environment, int *lanes);
/* src/environment_api.h:206 */
int cuju_environment_agents(void *environment, int *left, int *right);
/* src/environment_api.h:218 */
int cuju_environment_players(void *environment, int *left, int *right);
/* src/environment_api.h:229 */
int cuju_environment_set_difficulty(void *environment, const float *difficulty);
/* src/environment_api.h:240 */
void cuju_environment_difficulty(void *environment, float *difficulty);
/* src/environment_api.h:250 */
int cuju_environment_reset(void *environment, const unsigned int *seeds, const int *reverse, void *stream);
/* src/environment_api.h:269 */
int cuju_environment_reset_masked(void *environment, const unsigned char *mask, int mask_on_device, const int64_t *seeds,
                                  const int *reverse, void *stream, int synchronize);
/* src/environment_api.h:287 */
int cuju_environment_reset_done(void *environment, void *stream);
/* src/environment_api.h:302; -2 for a host action outside [-n, n) */
int cuju_environment_step(void *environment, const int *actions, int on_device, void *stream, int synchronize);
/* src/environment_api.h:323 */
int cuju_environment_step_async(void *environment, const int *actions, int on_device, void *stream);
/* No counterpart in the reference: cuju_environment_step for callers that cannot allocate (code
   under HIP graph capture, serving loops that forbid device allocation). The step runs on
   `stream` with device actions int32 [environments][agents], unchecked, and returns without
   waiting; its working memory is a static array of the library on each GPU instead of the
   batch's, so the call allocates and frees nothing. It takes batches of at most 64 environments
   (-1 with cuju_last_error() beyond). Every such call on a GPU shares that GPU's array: calls that
   overlap on one GPU race, so a caller serializes them (one stream, or events). */
int cuju_environment_step_no_alloc(void *environment, const int *actions, void *stream);
/* src/environment_api.h:341 */
int cuju_environment_step_wait(void *environment);
/* src/environment_api.h:353 */
int cuju_environment_synchronize(void *environment, void *stream);
/* src/environment_api.h:367 */
const char *cuju_environment_get_state(void *environment, int index, unsigned long long *size, int *episode);
/* src/environment_api.h:392; `bytes` are engine bytes of get_state, `episode` as get_state writes it */
int cuju_environment_set_state(void *environment, int index, const char *bytes, unsigned long long size, const int *episode);
/* src/environment_api.h:410; simple115 only: [agents][115 * stack] float32, oldest frame first */
int cuju_environment_set_stack(void *environment, int index, const char *name, const void *frames, unsigned long long size);
/* src/environment_api.h:449; raw array `field` from 0: its name, type (0 float32, 1 int32, 2 bool,
   3 uint8), the two dimensions after the agent axis (0 if absent) and its byte offset into raw and
   final_raw; null past the last array or without the raw representation */
const char *cuju_environment_raw_field(void *environment, int field, int *type, int *dimensions, unsigned long long *offset);
/* src/environment_api.h:430; simple115, final_simple115, smm, final_smm (uint8
   [E][A][smm_height][smm_width][4 * stack]), raw, final_raw, reward, done, score_reward */
void *cuju_environment_buffer(void *environment, const char *name);
/* src/environment_api.h:470; the current episode of environment `index`, synchronously: 17 values
   (seed, reverse, resets so far, episode_number, bundle, step of the last observation or -1,
   fixed seed or -1, deterministic, ticks per step, left and right agents, left and right players,
   the designated player of each team now and at the last episode end) and, unless null, the
   played left/right difficulty then the scenario's */
int cuju_environment_episode(void *environment, int index, long long *values, float *difficulty);
/* src/environment_api.h:519; the scenario name that bundle `bundle` records, or null past the last */
const char *cuju_environment_scenario(void *environment, int bundle);

/* The scenario builder (src/scenario_api.h:19-51). `cuju_scenario_build_bundle` refuses a
   description of another version. */
#define CUJU_SCENARIO_VERSION 1

/* One `AddPlayer` call of a GRF scenario file (src/scenario_api.h:22-28): the start position in
   environment coordinates, an `e_PlayerRole` from 0 (goalkeeper) to 9, and two flags. */
struct cuju_scenario_player {
    double x, y;
    int role;
    int lazy;
    int controllable;
};

/* What a scenario file builds for one parity of the episode number, in the fields of GRF's
   `ScenarioConfig` (src/scenario_api.h:30-47). An empty team is refused: the caller adds GRF's
   lazy goalkeeper first. */
struct cuju_scenario_description {
    int version;
    double ball_x, ball_y;
    const struct cuju_scenario_player *left_team;
    int left_size;
    const struct cuju_scenario_player *right_team;
    int right_size;
    int use_magnet, offsides, real_time;
    double left_team_difficulty, right_team_difficulty;
    int deterministic, end_episode_on_score, end_episode_on_possession_change, end_episode_on_out_of_play;
    int game_duration, second_half;
    int control_all_players;
    unsigned int game_engine_random_seed;
};

/* src/scenario_api.h:52; writes the agentless bundle of a scenario (its even and odd episodes) to
   `out`, with the animation tables at `animations`; 0, or -1 with cuju_last_error() */
int cuju_scenario_build_bundle(const struct cuju_scenario_description *even, const struct cuju_scenario_description *odd,
                               const char *name, const char *animations, const char *out);

/* No counterpart in the reference: a check of the device's math routines for tests. It evaluates
   the routines the step calls (glibc 2.39's algorithms, tables read from LDS as in the step) on
   `count` inputs: the consecutive float bit patterns from `first` (kind 0), the float arrays `x`
   and `y` (kind 1) or the double arrays `x` and `y` (kind 2), into `out`. Pointers are device
   memory; the work is enqueued on `stream`. `which`: float 0 sinf, 1 cosf, 2 powf(x, y),
   3 atan2f(x, y), 4 atanf, 5 acosf, 6 asinf, 7 and 8 the sine and cosine of sincosf; double 0 sin,
   1 cos, 2 pow(x, y), 3 acos, 4 and 5 the sine and cosine of sincos. 0, or -1 for arguments out of
   range or a failed launch. */
int cuju_debug_libm_device(int kind, int which, unsigned int first, long long count, const void *x, const void *y, void *out,
                           void *stream);

#ifdef __cplusplus
}
#endif

#endif
