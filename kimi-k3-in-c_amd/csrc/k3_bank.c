/* SPDX-License-Identifier: Apache-2.0 */
/*
 * k3_bank.c -- an expert bank resident in HBM behind the reference's K3ExpertSrc.
 *
 * The reference streams MXFP4 experts from disk into a host-RAM LRU cache and hands the
 * kernels host pointers through K3ExpertSrc.get / getmany / resident (include/k3/k3.h of
 * the reference, :323-355; src/cache/k3_cache.c:24-33 turns a slot into K3ExpertQ
 * pointers). On the MI355X the cache belongs in HBM: 288 GB holds every expert of a
 * 384-expert layer (8.98 GB) many times over, or about 16,000 of Kimi K3's
 * 17,547,264-byte experts. This file is that cache:
 *
 *   - get(layer, e) means "ensure resident in HBM": a hit returns device pointers at once;
 *     a miss asks the upstream source (any K3ExpertSrc handing out host pointers, e.g. the
 *     reference's own disk cache) for the bytes, copies them into a free or least-recently
 *     used slot (tiling them for the expert kernels once, at admission) and returns the
 *     slot's device pointers;
 *   - getmany is the batch form, resident() answers without any transfer;
 *   - k3_devbank_put_run admits an expert from its on-disk byte run (w1.packed w1.scale
 *     w2.packed w2.scale w3.packed w3.scale, src/io/k3_load.h:3-9 of the reference).
 *
 * The host MoE entry points (k3_moe, k3_moe_prefill) recognise a bank's source and run
 * the experts straight from the slots: after warm-up a call moves no weight bytes over
 * PCIe. During such a call every slot it has fetched is pinned, so a later get() of the
 * same call cannot evict an expert the call still has to compute. When a call names more
 * experts than the bank has slots, the call computes what it has fetched before the get()
 * that would need one more slot, then releases its slots (k3_bank_full, k3_bank_call).
 */
#include "k3.h"
#include "k3_bank.h"
#include "k3_dev.h"
#include "k3k.h"

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

struct K3DevBank {
    K3ExpertSrc src;            /* what callers receive; ctx points back here */
    K3ExpertSrc *upstream;      /* host-pointer source for misses, or NULL */
    int n_layers, n_experts, width, inter, layout, nslot;
    size_t off[6], sz[6];       /* tensor offsets / sizes inside a slot: p1 s1 p3 s3 p2 s2 */
    size_t slot_bytes;
    char *arena;                /* device, nslot * slot_bytes */
    void *stage[2];             /* device staging for the tiled layout */
    int *slot_of;               /* [n_layers * n_experts] -> slot, or -1 */
    int *key_of;                /* [nslot] -> key, or -1 */
    uint64_t *used_at, clock;
    uint64_t *pin, epoch;       /* pin[s] == epoch while a MoE call holds the slot */
    int in_call;
    K3DevBankStats st;
};

static int bank_error(const char *fmt, const char *what)
{
    k3h_set_error(fmt, what);
    return -1;
}

/* Sizes of gate/up [inter][width] and down [width][inter] in the bank's layout. */
static void tensor_sizes(int layout, int width, int inter, size_t sz[6])
{
    const int rows[3] = {inter, inter, width}, in[3] = {width, width, inter};
    for (int m = 0; m < 3; m++) {
        size_t r = (size_t)rows[m];
        if (layout == K3_BANK_TILED) r = (r + 63) / 64 * 64;   /* tile groups of 64 rows */
        sz[2 * m] = r * (size_t)in[m] / 2;
        sz[2 * m + 1] = r * (size_t)in[m] / 32;
    }
}

size_t k3_devbank_run_bytes(int width, int inter)
{
    if (width <= 0 || inter <= 0) return 0;
    return (size_t)3 * ((size_t)width * inter / 2 + (size_t)width * inter / 32);
}

static void fill_q(const K3DevBank *b, int slot, K3ExpertQ *q)
{
    const unsigned char *base = (const unsigned char *)b->arena + (size_t)slot * b->slot_bytes;
    q->p1 = base + b->off[0];
    q->s1 = base + b->off[1];
    q->p3 = base + b->off[2];
    q->s3 = base + b->off[3];
    q->p2 = base + b->off[4];
    q->s2 = base + b->off[5];
}

static int key_ok(const K3DevBank *b, int layer, int expert)
{
    return layer >= 0 && layer < b->n_layers && expert >= 0 && expert < b->n_experts;
}

static void touch(K3DevBank *b, int slot)
{
    b->used_at[slot] = ++b->clock;
    if (b->in_call) b->pin[slot] = b->epoch;
}

/* A free slot, else the least recently used one not pinned by the current call. */
static int pick_victim(const K3DevBank *b)
{
    int best = -1;
    uint64_t oldest = UINT64_MAX;
    for (int s = 0; s < b->nslot; s++) {
        if (b->key_of[s] < 0) return s;
        if (b->in_call && b->pin[s] == b->epoch) continue;
        if (b->used_at[s] < oldest) {
            oldest = b->used_at[s];
            best = s;
        }
    }
    return best;
}

/* Copies one expert's six host tensors (p1 s1 p3 s3 p2 s2) into a slot for `key`. */
static int admit(K3DevBank *b, int key, const void *const host[6])
{
    const int slot = pick_victim(b);
    if (slot < 0) {
        b->st.failures++;
        return bank_error("k3_devbank: every slot is pinned by the current call (%s)",
                          "raise the slot count");
    }
    void *stream = k3h_stream();
    if (b->key_of[slot] >= 0) {
        b->slot_of[b->key_of[slot]] = -1;
        b->key_of[slot] = -1;
        b->st.evictions++;
    }
    char *base = b->arena + (size_t)slot * b->slot_bytes;
    const int rows[3] = {b->inter, b->inter, b->width}, in[3] = {b->width, b->width, b->inter};
    for (int m = 0; m < 3; m++) {
        const size_t pk = (size_t)rows[m] * in[m] / 2, sc = (size_t)rows[m] * in[m] / 32;
        if (b->layout == K3_BANK_TILED) {
            if (k3k_h2d(b->stage[0], host[2 * m], pk, stream) ||
                k3k_h2d(b->stage[1], host[2 * m + 1], sc, stream) ||
                k3k_mx_tile((uint8_t *)base + b->off[2 * m], (uint8_t *)base + b->off[2 * m + 1],
                            (const uint8_t *)b->stage[0], (const uint8_t *)b->stage[1], rows[m],
                            in[m], stream))
                return bank_error("k3_devbank: upload: %s", k3k_error());
        } else if (k3k_h2d(base + b->off[2 * m], host[2 * m], pk, stream) ||
                   k3k_h2d(base + b->off[2 * m + 1], host[2 * m + 1], sc, stream)) {
            return bank_error("k3_devbank: upload: %s", k3k_error());
        }
        b->st.bytes_uploaded += pk + sc;
    }
    /* the host bytes may be recycled by the upstream source's next get() */
    if (k3k_sync(stream)) return bank_error("k3_devbank: upload: %s", k3k_error());
    b->key_of[slot] = key;
    b->slot_of[key] = slot;
    b->st.misses++;
    touch(b, slot);
    return slot;
}

static int ensure(K3DevBank *b, int layer, int expert, K3ExpertQ *out)
{
    if (!key_ok(b, layer, expert)) return -1;
    const int key = layer * b->n_experts + expert;
    int slot = b->slot_of[key];
    if (slot >= 0) {
        b->st.hits++;
        touch(b, slot);
    } else {
        if (!b->upstream || !b->upstream->get) return -1;
        K3ExpertQ h;
        memset(&h, 0, sizeof h);
        if (b->upstream->get(b->upstream, layer, expert, &h) != 0) return -1;
        const void *host[6] = {h.p1, h.s1, h.p3, h.s3, h.p2, h.s2};
        for (int k = 0; k < 6; k++)
            if (!host[k]) return -1;
        slot = admit(b, key, host);
        if (slot < 0) return -1;
    }
    if (out) fill_q(b, slot, out);
    return 0;
}

static int src_get(K3ExpertSrc *self, int layer, int expert, K3ExpertQ *out)
{
    K3DevBank *b = (K3DevBank *)self->ctx;
    k3h_lock();
    const int rc = ensure(b, layer, expert, out);
    k3h_unlock();
    return rc;
}

/* Whether admitting `expert` now needs a slot the current call cannot give: it is not
 * pinned by the call and every slot is. */
static int call_full(const K3DevBank *b, int layer, int expert)
{
    if (!b->in_call || !key_ok(b, layer, expert)) return 0;
    const int slot = b->slot_of[layer * b->n_experts + expert];
    if (slot >= 0 && b->pin[slot] == b->epoch) return 0;
    for (int s = 0; s < b->nslot; s++)
        if (b->key_of[s] < 0 || b->pin[s] != b->epoch) return 0;
    return 1;
}

static int src_getmany(K3ExpertSrc *self, int layer, const int *experts, int n)
{
    K3DevBank *b = (K3DevBank *)self->ctx;
    k3h_lock();
    /* the upstream may read its misses concurrently; our admissions then follow in order */
    if (b->upstream && b->upstream->getmany) {
        int *miss = (int *)malloc((size_t)(n > 0 ? n : 1) * sizeof(int));
        int nm = 0;
        for (int i = 0; miss && i < n; i++)
            if (key_ok(b, layer, experts[i]) && b->slot_of[layer * b->n_experts + experts[i]] < 0)
                miss[nm++] = experts[i];
        if (nm) b->upstream->getmany(b->upstream, layer, miss, nm);
        free(miss);
    }
    /* a hint: admissions stop where the call has pinned every slot (its later get()s make
     * room by computing what is fetched first) */
    int got = 0;
    for (int i = 0; i < n; i++)
        if (!call_full(b, layer, experts[i])) got += ensure(b, layer, experts[i], NULL) == 0;
    k3h_unlock();
    return got;
}

static int src_resident(K3ExpertSrc *self, int layer, int expert, K3ExpertQ *out)
{
    K3DevBank *b = (K3DevBank *)self->ctx;
    k3h_lock();
    int r = 0;
    if (key_ok(b, layer, expert)) {
        const int slot = b->slot_of[layer * b->n_experts + expert];
        if (slot >= 0) {
            r = 1;
            if (out) {
                touch(b, slot);
                fill_q(b, slot, out);
            }
        }
    }
    k3h_unlock();
    return r;
}

/* ------------------------------------------------------------------ public API ---- */
K3DevBank *k3_devbank_create(int n_layers, int n_experts, int width, int inter, int slots,
                             int layout, K3ExpertSrc *upstream)
{
    k3h_lock();
    K3DevBank *b = NULL;
    if (n_layers <= 0 || n_experts <= 0 || slots <= 0 || width <= 0 || inter <= 0 ||
        width % 32 || inter % 32) {
        bank_error("k3_devbank_create: %s", "need positive counts and widths that are multiples of 32");
        goto out;
    }
    if (layout != K3_BANK_ROWS && layout != K3_BANK_TILED) {
        bank_error("k3_devbank_create: %s", "unknown layout");
        goto out;
    }
    if (layout == K3_BANK_TILED && (width % 512 || inter % 512)) {
        bank_error("k3_devbank_create: %s", "the tiled layout needs widths that are multiples of 512");
        goto out;
    }
    if ((long long)n_layers * n_experts > 0x7fffffffLL) {
        bank_error("k3_devbank_create: %s", "too many (layer, expert) keys");
        goto out;
    }
    if (k3h_init()) goto out;
    b = (K3DevBank *)calloc(1, sizeof *b);
    if (!b) {
        bank_error("k3_devbank_create: %s", "out of host memory");
        goto out;
    }
    b->upstream = upstream;
    b->n_layers = n_layers;
    b->n_experts = n_experts;
    b->width = width;
    b->inter = inter;
    b->layout = layout;
    b->nslot = slots;
    tensor_sizes(layout, width, inter, b->sz);
    /* slot order p1 s1 p3 s3 p2 s2, each 256-byte aligned */
    size_t o = 0;
    for (int k = 0; k < 6; k++) {
        b->off[k] = o;
        o = (o + b->sz[k] + 255u) & ~(size_t)255u;
    }
    b->slot_bytes = o;
    const size_t nkey = (size_t)n_layers * n_experts;
    b->slot_of = (int *)malloc(nkey * sizeof(int));
    b->key_of = (int *)malloc((size_t)slots * sizeof(int));
    b->used_at = (uint64_t *)calloc((size_t)slots, sizeof(uint64_t));
    b->pin = (uint64_t *)calloc((size_t)slots, sizeof(uint64_t));
    if (!b->slot_of || !b->key_of || !b->used_at || !b->pin) {
        bank_error("k3_devbank_create: %s", "out of host memory");
        goto fail;
    }
    for (size_t k = 0; k < nkey; k++) b->slot_of[k] = -1;
    for (int s = 0; s < slots; s++) b->key_of[s] = -1;
    b->arena = (char *)k3k_malloc((size_t)slots * b->slot_bytes);
    if (!b->arena) {
        bank_error("k3_devbank_create: HBM for the slots: %s", k3k_error());
        goto fail;
    }
    if (layout == K3_BANK_TILED) {
        const size_t big = (size_t)(inter > width ? inter : width) * (inter > width ? width : inter);
        b->stage[0] = k3k_malloc(big / 2);
        b->stage[1] = k3k_malloc(big / 32);
        if (!b->stage[0] || !b->stage[1]) {
            bank_error("k3_devbank_create: staging: %s", k3k_error());
            goto fail;
        }
    }
    b->src.get = src_get;
    b->src.getmany = src_getmany;
    b->src.resident = src_resident;
    b->src.ctx = b;
    b->st.slots = slots;
    b->st.slot_bytes = b->slot_bytes;
    goto out;
fail:
    if (b) {
        k3k_free(b->arena);
        k3k_free(b->stage[0]);
        k3k_free(b->stage[1]);
        free(b->slot_of);
        free(b->key_of);
        free(b->used_at);
        free(b->pin);
        free(b);
    }
    b = NULL;
out:
    k3h_unlock();
    return b;
}

K3ExpertSrc *k3_devbank_source(K3DevBank *b) { return b ? &b->src : NULL; }

int k3_devbank_put_run(K3DevBank *b, int layer, int expert, const void *run, size_t bytes)
{
    if (!b || !run) return bank_error("k3_devbank_put_run: %s", "NULL bank or run");
    k3h_lock();
    int rc = -1;
    const size_t want = k3_devbank_run_bytes(b->width, b->inter);
    if (bytes != want) {
        char m[96];
        snprintf(m, sizeof m, "run of %zu bytes, this bank's experts are %zu", bytes, want);
        bank_error("k3_devbank_put_run: %s", m);
    } else if (!key_ok(b, layer, expert)) {
        bank_error("k3_devbank_put_run: %s", "layer or expert out of range");
    } else {
        /* run order w1.p w1.s w2.p w2.s w3.p w3.s: gate = w1, down = w2, up = w3 */
        const size_t gp = (size_t)b->inter * b->width / 2, gs = gp / 16;
        const unsigned char *r = (const unsigned char *)run;
        const void *host[6] = {r, r + gp, r + 2 * (gp + gs), r + 2 * (gp + gs) + gp, r + gp + gs,
                               r + 2 * gp + gs};
        const int key = layer * b->n_experts + expert;
        if (b->slot_of[key] >= 0) {            /* replace in place */
            const int s = b->slot_of[key];
            b->slot_of[key] = -1;
            b->key_of[s] = -1;
        }
        rc = admit(b, key, host) < 0 ? -1 : 0;
    }
    k3h_unlock();
    return rc;
}

int k3_devbank_stats(const K3DevBank *b, K3DevBankStats *st)
{
    if (!b || !st) return bank_error("k3_devbank_stats: %s", "NULL argument");
    k3h_lock();
    *st = b->st;
    st->resident = 0;
    for (int s = 0; s < b->nslot; s++) st->resident += b->key_of[s] >= 0;
    k3h_unlock();
    return 0;
}

void k3_devbank_destroy(K3DevBank *b)
{
    if (!b) return;
    k3h_lock();
    k3k_sync(k3h_stream());
    k3k_free(b->arena);
    k3k_free(b->stage[0]);
    k3k_free(b->stage[1]);
    free(b->slot_of);
    free(b->key_of);
    free(b->used_at);
    free(b->pin);
    free(b);
    k3h_unlock();
}

/* ------------------------------------------------------ for the host MoE layer ---- */
int k3_bank_layout(const K3ExpertSrc *src, int width, int inter)
{
    if (!src || src->get != src_get) return -1;
    const K3DevBank *b = (const K3DevBank *)src->ctx;
    if (b->width != width || b->inter != inter) return -2;
    return b->layout;
}

int k3_bank_full(const K3ExpertSrc *src, int layer, int expert)
{
    if (!src || src->get != src_get) return 0;
    k3h_lock();
    const int r = call_full((const K3DevBank *)src->ctx, layer, expert);
    k3h_unlock();
    return r;
}

void k3_bank_call(K3ExpertSrc *src, int begin)
{
    if (!src || src->get != src_get) return;
    K3DevBank *b = (K3DevBank *)src->ctx;
    if (begin) b->epoch++;
    b->in_call = begin;
}
