/*
 * k4_router.c -- a C99 caller of include/ter_hip.h (CPU only).
 *
 * Implements the ter_k4_call routing a HIP-enabled libter_k4 adds
 * (src/k4/ter_k4.cpp:47-59): the native table first, and the Sim for every
 * name the native table does not hold.  The Sim is a stub that records its
 * calls, so the program checks, without a GPU, that
 *   - the reference's 3-argument "tk_matmul_b_9t" call (r1 = X, r2 = W,
 *     r3 = Y: src/kernels/tk_matmul_b_9t.tasm:1-3) reaches the Sim unchanged;
 *   - the native matmul slot answers its own name, with its own codes for too
 *     few (TER_HIP_ERR_FEWARGS) and too many (TER_HIP_ERR_NARGS) arguments;
 *   - an installed native function receives the caller's arguments.
 * Built by tests/test_abi.py with gcc -std=c99 -Wall -Wextra -Werror -pedantic.
 * Prints "ok" and exits 0, or names the failed check and exits 1.
 */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "ter_hip.h"

static int sim_calls;
static char sim_name[32];
static int64_t sim_args[7];
static size_t sim_n;

/* Stand-in for Sim::call_kernel behind KernelTable::find (src/sim/call_kernel.cpp:55-78). */
static int sim_call(const char* name, const int64_t* args, size_t n_args) {
    size_t i;
    ++sim_calls;
    strncpy(sim_name, name, sizeof sim_name - 1);
    sim_name[sizeof sim_name - 1] = '\0';
    for (i = 0; i < n_args && i < 7; ++i) sim_args[i] = args[i];
    sim_n = n_args;
    return strcmp(name, "tk_matmul_b_9t") == 0 ? 0 : TER_HIP_ERR_NOTFOUND;
}

/* ter_k4_call with the native table routed first. */
static int k4_call(ter_hip_handle_t* hip, const char* name, const int64_t* args, size_t n_args) {
    int rc;
    if (!name) return TER_HIP_ERR_NULL;
    if (n_args > 7) return TER_HIP_ERR_NARGS;
    if (hip) {
        rc = ter_hip_call(hip, name, args, n_args);
        if (rc != TER_HIP_ERR_NOTFOUND) return rc;
    }
    return sim_call(name, args, n_args);
}

static int native_seen;
static int64_t native_first;

static int my_native(ter_hip_handle_t* h, const int64_t* args, size_t n_args) {
    (void)h;
    ++native_seen;
    native_first = n_args > 0 ? args[0] : -1;
    return 7;
}

#define CHECK(c)                                                        \
    do {                                                                \
        if (!(c)) {                                                     \
            fprintf(stderr, "k4_router: check failed: %s (line %d)\n", #c, __LINE__); \
            return 1;                                                   \
        }                                                               \
    } while (0)

int main(void) {
    const int64_t xwy[3] = {4096, 8192, 12288}; /* Sim addresses of X, W, Y */
    const int64_t six[6] = {0, 0, 0, 0, 0, 1};
    const int64_t eight[8] = {0, 1, 2, 3, 4, 5, 6, 7};
    ter_hip_op_counts_t counts;
    ter_hip_handle_t* h = ter_hip_create(-1);
    CHECK(h != NULL);

    /* the reference's own call falls through to the Sim, arguments intact */
    CHECK(k4_call(h, "tk_matmul_b_9t", xwy, 3) == 0);
    CHECK(sim_calls == 1 && strcmp(sim_name, "tk_matmul_b_9t") == 0 && sim_n == 3);
    CHECK(sim_args[0] == 4096 && sim_args[1] == 8192 && sim_args[2] == 12288);

    /* the native matmul slot: too few, too many, and a null weight handle */
    CHECK(k4_call(h, TER_HIP_SLOT_MATMUL, six, 5) == TER_HIP_ERR_FEWARGS);
    CHECK(k4_call(h, TER_HIP_SLOT_MATMUL, eight, 8) == TER_HIP_ERR_NARGS);
    CHECK(ter_hip_call(h, TER_HIP_SLOT_MATMUL, eight, 8) == TER_HIP_ERR_NARGS);
    CHECK(k4_call(h, TER_HIP_SLOT_MATMUL, six, 6) == TER_HIP_ERR_NULL);
    CHECK(sim_calls == 1);

    /* unknown names reach the Sim, which reports them unknown itself */
    CHECK(k4_call(h, "tk_rmsnorm", xwy, 2) == TER_HIP_ERR_NOTFOUND);
    CHECK(sim_calls == 2);

    /* an installed native function shadows the Sim for its name */
    CHECK(ter_hip_install_native(h, "tk_custom", my_native) == TER_HIP_OK);
    CHECK(k4_call(h, "tk_custom", xwy, 3) == 7);
    CHECK(native_seen == 1 && native_first == 4096 && sim_calls == 2);

    /* failed calls count nothing */
    ter_hip_op_counts(h, &counts);
    CHECK(counts.tvmac == 0 && counts.total_ops == 0);

    /* the weight handle's layout as the ctypes mirror declares it */
    CHECK(sizeof(ter_hip_wpk_t) == 48);
    CHECK(ter_hip_wpk_bytes(256, 16) == 1024 + 16 * 8);

    ter_hip_destroy(h);
    printf("ok\n");
    return 0;
}
