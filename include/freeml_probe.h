/* freeml_probe.h -- measurement library (lib/libfreeml_probe.so), kept out of the product
 * library libfreeml_hip.so: it launches a kernel that measures the machine, not the model.
 * Links against libfreeml_hip.so (device selection, stream, error text: fmlh_last_error). */
#ifndef FREEML_PROBE_H
#define FREEML_PROBE_H

#include "freeml_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Measurement hook: the latency of one hand-off through the exchange words the persistent decode
 * kernels pass values between workgroups with.  One cooperative launch of one workgroup per CU;
 * group_a (na workgroup ids) and, if nb > 0, group_b take part.  nb == 0: every round, each
 * workgroup of A publishes its share of `words` words and gathers all of them (one hop per
 * round).  nb > 0: A publishes `words` words, each workgroup of B gathers them and publishes
 * `words` words back, each workgroup of A gathers those (two hops per round).  scope 0: device
 * scope (agent-scope atomics, any placement); 1..12: the other store / load forms measured
 * (probe.hip lists them; the XCD-local ones are not coherent between CUs on MI355X, so a wait
 * on them can give up).  *ns_per_hop: mean over
 * `rounds` timed rounds after 8 untimed ones (device wall clock).  xcc_out (NULL or one int32
 * per CU): the XCD each workgroup ran on.  A wait that gives up (bounded) returns FMLH_E_STATE.
 * No counterpart in the reference, which has no device code of this kind. */
int fmlh_probe_exchange(int scope, const int32_t* group_a, uint32_t na, const int32_t* group_b,
                        uint32_t nb, uint32_t words, uint32_t rounds, int32_t* xcc_out,
                        double* ns_per_hop);

#ifdef __cplusplus
}
#endif

#endif /* FREEML_PROBE_H */
