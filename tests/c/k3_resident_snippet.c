/* SPDX-License-Identifier: Apache-2.0 */
/*
 * The "Resident weights" example of the integration guide, compiled against include/k3.h
 * (tests/test_c_caller.py builds it with -Werror), so that the guide's calls keep the
 * exported signatures: register the router and each expert's byte run once, then make the
 * unchanged k3_moe call (reference include/k3/k3.h:418-419).
 */
#include "k3.h"

#include <stddef.h>

void k3amd_resident_example(float *out, const float *x, const K3MoeW *w, const K3Cfg *c, int T,
                            int *idx, float *wt, float *scratch, const K3ExpertQ *bank,
                            size_t run_bytes)
{
    k3_dev_register(w->gate, (size_t)c->n_experts * c->hidden * sizeof(float));
    for (int e = 0; e < c->n_experts; e++) {          /* each expert's run of bytes */
        k3_dev_register(bank[e].p1, run_bytes);
    }
    k3_moe(out, x, w, c, T, idx, wt, scratch);        /* unchanged call */
}
