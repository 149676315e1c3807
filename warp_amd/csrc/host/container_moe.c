/* SPDX-License-Identifier: Apache-2.0 */
/*
 * container_moe.c — a device MoE layer built from a container layer.
 *
 * The tensors and settings moe_layer reads for layer L
 * (src/model.c:5488-5497, 5932-5936) are found by name in the trunk, the
 * shapes REQUIRE_MATRIX insists on are checked (src/model.c:1700-1712),
 * and the layer gets only its own nine codebooks (its bank's
 * codebook_base onward) rather than the whole table.
 */
#include "waste_hip.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static int matrix(waste_hip_container *c, const char *prefix, int layer, const char *what, int rows, int cols,
                  waste_hip_tensor *t)
{
    char name[512];
    snprintf(name, sizeof name, "%smodel.layers.%d.block_sparse_moe.%s", prefix, layer, what);
    int nd = 0, sh[4];
    const int rc = waste_hip_container_tensor(c, name, t, &nd, sh);
    if (rc) return rc;
    if (nd != 2 || sh[0] != rows || sh[1] != cols) return WASTE_HIP_EFORMAT;
    return 0;
}

int waste_hip_container_moe(waste_hip_container *c, int layer, int max_tokens, int prefill_min_tokens, int flags,
                            waste_hip_moe **out)
{
    if (!out) return WASTE_HIP_EINVAL;
    *out = NULL;
    waste_hip_container_cfg g;
    int n_exp = 0, cb = 0;
    size_t rec_bytes = 0;
    if (!c || waste_hip_container_config(c, &g) ||
        waste_hip_container_bank(c, layer, &n_exp, &cb, &rec_bytes) || max_tokens < 1)
        return WASTE_HIP_EINVAL;
    /* the layer decodes VQ3R (three stages of 256 eight-wide entries),
     * VQ2R (two) and VQ4P (index_bits 6: four stages of 64) */
    const int p6 = g.index_bits == 6, r2 = !p6 && g.stages == 2;
    if (g.vec_dim != 8 || g.latent_dim ||
        (p6 ? g.stages != 4 || g.entries != 64
            : (g.stages != 3 && g.stages != 2) || g.entries != 256 || g.index_bits != 8))
        return WASTE_HIP_EINVAL;
    const int E = g.n_experts, H = g.hidden, I = g.moe_inter;
    const int SI = I * (g.n_shared ? g.n_shared : 1);
    waste_hip_tensor router, bias, sg, su, sd;
    int rc;
    if ((rc = matrix(c, g.prefix, layer, "gate.weight", E, H, &router))) return rc;
    if ((rc = matrix(c, g.prefix, layer, "shared_experts.gate_proj.weight", SI, H, &sg))) return rc;
    if ((rc = matrix(c, g.prefix, layer, "shared_experts.up_proj.weight", SI, H, &su))) return rc;
    if ((rc = matrix(c, g.prefix, layer, "shared_experts.down_proj.weight", H, SI, &sd))) return rc;
    const float *b = NULL;
    {
        char name[512];
        snprintf(name, sizeof name, "%smodel.layers.%d.block_sparse_moe.gate.e_score_correction_bias", g.prefix,
                 layer);
        int nd = 0, sh[4];
        rc = waste_hip_container_tensor(c, name, &bias, &nd, sh);
        if (rc == 0) {
            /* the engine reads it as E floats (src/model.c:5497) */
            if (bias.fmt != WQ_F32 || (size_t)bias.rows * (size_t)bias.cols != (size_t)E) return WASTE_HIP_EFORMAT;
            b = (const float *)bias.q;
        } else if (rc != WASTE_HIP_EFORMAT) {
            return rc;
        }
    }

    waste_hip_moe_cfg mc;
    memset(&mc, 0, sizeof mc);
    mc.hidden = H;
    mc.n_experts = E;
    mc.top_k = g.top_k;
    mc.moe_inter = I;
    mc.n_shared = g.n_shared ? g.n_shared : 1;
    mc.score_func = g.score_func;
    mc.renorm = g.renorm;
    mc.routed_scale = g.routed_scale;
    mc.n_group = (flags & WASTE_HIP_CT_GROUP_LIMIT) ? g.n_group : 1;
    mc.topk_group = (flags & WASTE_HIP_CT_GROUP_LIMIT) ? g.topk_group : 1;
    mc.layer = layer;
    mc.max_tokens = max_tokens;
    mc.verify_records = 0;             /* the container's reads check the checksum */
    mc.prefill_min_tokens = prefill_min_tokens;
    mc.index_bits = p6 ? 6 : 8;
    mc.stages = g.stages;
    mc.p6_order = p6 || r2 ? waste_hip_vq_p6_order() : 0;   /* the engine's arithmetic on this host */
    waste_hip_moe *m = NULL;
    if ((rc = waste_hip_moe_create(&mc, &m))) return rc;
    int n_books = 0;
    const uint16_t *books = waste_hip_container_codebooks(c, &n_books);
    const size_t per = (size_t)g.entries * g.vec_dim;
    if ((rc = waste_hip_moe_set_router(m, &router, b)) || (rc = waste_hip_moe_set_shared(m, &sg, &su, &sd)) ||
        (rc = waste_hip_moe_set_codebooks_at(m, books + (size_t)cb * per, cb, 3 * g.stages)))
        goto fail;
    if (flags & WASTE_HIP_CT_RECORDS) {
        void *buf = malloc(rec_bytes);
        if (!buf) {
            rc = WASTE_HIP_ENOMEM;
            goto fail;
        }
        for (int e = 0; e < n_exp && !rc; e++) {
            rc = waste_hip_container_read_expert(c, layer, e, buf, rec_bytes);
            if (!rc) rc = waste_hip_moe_set_expert(m, e, buf, rec_bytes);
        }
        free(buf);
        if (rc) goto fail;
    }
    *out = m;
    return 0;
fail:
    waste_hip_moe_destroy(m);
    return rc;
}
