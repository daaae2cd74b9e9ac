/*
 * TEST INFRASTRUCTURE ONLY: CPU oracle for the two-stack probability model,
 * the lane predictor and normal-stream packing. Restates
 *   src/common/cpu_transformer.tpp:99-175, 205-224, 285-419  (composition, caches)
 *   src/common/transformer.cpp:26-245                           (lane schedule, replay)
 *   src/format/entropy.cpp:26-155                               (stream order, FBAZ)
 * with geometry taken from orc_geometry instead of the reference's constants
 * (src/models/config.hpp:11-16 gives 12+3 layers, width 512, 4x128 heads).
 */
#include "oracle_format.h"
#include "oracle_internal.h"

#include <pthread.h>
#include <stdatomic.h>
#include <string.h>

enum
{
    replay_frames = 256
};

typedef struct orc_lane
{
    uint16_t *temporal_keys, *temporal_values; /* [Lt][extent][width] */
    size_t temporal_extent, temporal_position;
    uint16_t *codebook_keys, *codebook_values; /* [Lc][books][width] */
    size_t codebook_position;
    uint16_t *conditioning, *input, *prefix, *embedded;
    uint16_t prefix_tokens[16];
    size_t prefix_count;
    /* workspace */
    uint16_t *normalized, *qkv, *query, *key, *attention, *projected, *mlp, *logits;
} orc_lane;

struct orc_model
{
    orc_geometry g;
    orc_linear* projections;
    size_t projection_count;
    const uint16_t** gain;
    const uint16_t** bias;
    size_t norm_count;
    const uint16_t *positions, *rotations, *embeddings;
    orc_header header;
    orc_lane* lanes;
    size_t lane_count;
};

typedef struct
{
    size_t input, output;
} shape;

static shape projection_shape(const orc_geometry* g, size_t index)
{
    const size_t stacked = 4 * (size_t)(g->temporal_layers + g->codebook_layers);
    if (index == stacked || index == stacked + 1)
    {
        return (shape){g->latent, g->width};
    }
    if (index == stacked + 2)
    {
        return (shape){g->width, g->alphabet};
    }
    switch (index % 4)
    {
    case 0:
        return (shape){g->width, 3 * (size_t)g->width};
    case 1:
        return (shape){g->width, g->width};
    case 2:
        return (shape){g->width, g->ffn};
    default:
        return (shape){g->ffn, g->width};
    }
}

static int apply_linear(const orc_model* m, size_t index, const uint16_t* x, uint16_t* y)
{
    const shape s = projection_shape(&m->g, index);
    const orc_linear* l = &m->projections[index];
    return orc_qlinear(l->values, l->scales, l->bias, s.input, s.output, x, 1, y);
}

int orc_model_create(const orc_model_desc* desc, orc_model** out)
{
    const orc_geometry* g = &desc->geometry;
    if (!g->width || g->width % 256 || g->heads * g->head_width != g->width ||
        g->head_width % 2 || g->ffn % 256 || g->latent % 256 || !g->books || g->books > 16 ||
        !g->alphabet || !g->context || g->context < replay_frames)
    {
        return orc_fail("invalid model geometry");
    }
    orc_model* m = orc_alloc(sizeof *m);
    m->g = *g;
    m->projection_count = 4 * (size_t)(g->temporal_layers + g->codebook_layers) + 3;
    m->norm_count = 2 * (size_t)(g->temporal_layers + g->codebook_layers) + 2;
    m->projections = orc_alloc(m->projection_count * sizeof(orc_linear));
    memcpy(m->projections, desc->projections, m->projection_count * sizeof(orc_linear));
    m->gain = orc_alloc(m->norm_count * sizeof(uint16_t*));
    m->bias = orc_alloc(m->norm_count * sizeof(uint16_t*));
    memcpy(m->gain, desc->norm_gain, m->norm_count * sizeof(uint16_t*));
    memcpy(m->bias, desc->norm_bias, m->norm_count * sizeof(uint16_t*));
    m->positions = desc->positions;
    m->rotations = desc->rotations;
    m->embeddings = desc->embeddings;
    *out = m;
    return 0;
}

static void free_lanes(orc_model* m)
{
    for (size_t i = 0; i < m->lane_count; ++i)
    {
        orc_lane* l = &m->lanes[i];
        void* blocks[] = {l->temporal_keys, l->temporal_values, l->codebook_keys,
                          l->codebook_values, l->conditioning, l->input, l->prefix,
                          l->embedded, l->normalized, l->qkv, l->query, l->key, l->attention,
                          l->projected, l->mlp, l->logits};
        for (size_t b = 0; b < sizeof blocks / sizeof *blocks; ++b)
        {
            free(blocks[b]);
        }
    }
    free(m->lanes);
    m->lanes = NULL;
    m->lane_count = 0;
}

void orc_model_destroy(orc_model* model)
{
    if (!model)
    {
        return;
    }
    free_lanes(model);
    free(model->projections);
    free(model->gain);
    free(model->bias);
    free(model);
}

static size_t min_size(size_t a, size_t b)
{
    return a < b ? a : b;
}

/* src/common/cpu_transformer.tpp:285-329 */
int orc_backend_reset(orc_model* m, const orc_header* h, size_t count)
{
    if (orc_validate_header(h))
    {
        return 1;
    }
    if (!(h->model_channels == m->g.channels && h->codebooks <= m->g.books &&
          count == min_size(h->batch, h->frames) * h->groups))
    {
        return orc_fail("Transformer stream/model mismatch");
    }
    const size_t context = m->g.context;
    const size_t base = h->frames / h->batch, extra = h->frames % h->batch;
    const size_t contexts = (size_t)h->groups * ((h->batch - extra) * min_size(base, context) +
                                                 extra * min_size(base + 1, context));
    const size_t temporal_bytes =
        contexts * (size_t)m->g.temporal_layers * m->g.width * 2 * sizeof(uint16_t);
    const size_t codebook_bytes =
        count * h->codebooks * (size_t)m->g.codebook_layers * m->g.width * 2 * sizeof(uint16_t);
    if (temporal_bytes + codebook_bytes > (size_t)1024 * 1024 * 1024)
    {
        return orc_fail("Transformer caches exceed byte limit; reduce the encoding batch size or "
                        "channel count");
    }
    free_lanes(m);
    m->header = *h;
    m->lane_count = count;
    m->lanes = orc_alloc(count * sizeof(orc_lane));
    const size_t w = m->g.width;
    for (size_t i = 0; i < count; ++i)
    {
        orc_lane* l = &m->lanes[i];
        l->temporal_extent = min_size(base + (i / h->groups < extra), context);
        const size_t tsize = (size_t)m->g.temporal_layers * l->temporal_extent * w;
        const size_t csize = (size_t)m->g.codebook_layers * h->codebooks * w;
        l->temporal_keys = orc_alloc(tsize * 2);
        l->temporal_values = orc_alloc(tsize * 2);
        l->codebook_keys = orc_alloc(csize * 2);
        l->codebook_values = orc_alloc(csize * 2);
        l->conditioning = orc_alloc(w * 2);
        l->input = orc_alloc(w * 2);
        l->prefix = orc_alloc(m->g.latent * 2);
        l->embedded = orc_alloc(m->g.latent * 2);
        l->normalized = orc_alloc(w * 2);
        l->qkv = orc_alloc(3 * w * 2);
        l->query = orc_alloc(w * 2);
        l->key = orc_alloc(w * 2);
        l->attention = orc_alloc(w * 2);
        l->projected = orc_alloc(w * 2);
        l->mlp = orc_alloc((size_t)m->g.ffn * 2);
        l->logits = orc_alloc((size_t)m->g.alphabet * 2);
    }
    return 0;
}

int orc_backend_reset_temporal(orc_model* m, size_t lane)
{
    if (lane >= m->lane_count)
    {
        return orc_fail("invalid lane");
    }
    m->lanes[lane].temporal_position = 0;
    return 0;
}

int orc_backend_reset_codebook(orc_model* m, size_t lane)
{
    if (lane >= m->lane_count)
    {
        return orc_fail("invalid lane");
    }
    m->lanes[lane].prefix_count = 0;
    m->lanes[lane].codebook_position = 0;
    return 0;
}

static void add_in_place(uint16_t* left, const uint16_t* right, size_t n)
{
    for (size_t i = 0; i < n; ++i)
    {
        left[i] = orc_add_bf16(left[i], right[i]);
    }
}

/* src/common/cpu_transformer.tpp:133-175. keys/values hold `extent` rows per layer. */
static int evaluate_stack(const orc_model* m, orc_lane* l, int temporal, uint16_t* input,
                          size_t position, const uint16_t* rotation, int prefill)
{
    const orc_geometry* g = &m->g;
    const size_t w = g->width, hw = g->head_width;
    const size_t layers = temporal ? g->temporal_layers : g->codebook_layers;
    const size_t extent = temporal ? l->temporal_extent : m->header.codebooks;
    uint16_t* keys = temporal ? l->temporal_keys : l->codebook_keys;
    uint16_t* values = temporal ? l->temporal_values : l->codebook_values;
    const size_t projection_base = temporal ? 0 : 4 * (size_t)g->temporal_layers;
    const size_t norm_base = temporal ? 0 : 2 * (size_t)g->temporal_layers + 1;
    if (position >= extent)
    {
        return orc_fail("Transformer cache position mismatch");
    }
    for (size_t i = 0; i < layers; ++i)
    {
        const size_t p = projection_base + 4 * i, n = norm_base + 2 * i;
        uint16_t* layer_keys = keys + i * extent * w;
        uint16_t* layer_values = values + i * extent * w;
        if (orc_layer_norm(input, m->gain[n], m->bias[n], w, l->normalized) ||
            apply_linear(m, p, l->normalized, l->qkv))
        {
            return 1;
        }
        memcpy(l->query, l->qkv, w * 2);
        memcpy(l->key, l->qkv + w, w * 2);
        if (rotation)
        {
            for (size_t head = 0; head < g->heads; ++head)
            {
                orc_rotary(l->query + head * hw, rotation, hw, l->query + head * hw);
                orc_rotary(l->key + head * hw, rotation, hw, l->key + head * hw);
            }
        }
        memcpy(layer_keys + position * w, l->key, w * 2);
        memcpy(layer_values + position * w, l->qkv + 2 * w, w * 2);
        if (orc_attention(l->query, layer_keys, layer_values, position + 1, g->heads, hw,
                          g->attention_scale, prefill, l->attention) ||
            apply_linear(m, p + 1, l->attention, l->projected))
        {
            return 1;
        }
        add_in_place(input, l->projected, w);
        if (orc_layer_norm(input, m->gain[n + 1], m->bias[n + 1], w, l->normalized) ||
            apply_linear(m, p + 2, l->normalized, l->mlp))
        {
            return 1;
        }
        for (size_t j = 0; j < g->ffn; ++j)
        {
            l->mlp[j] = orc_gelu(l->mlp[j]);
        }
        if (apply_linear(m, p + 3, l->mlp, l->projected))
        {
            return 1;
        }
        add_in_place(input, l->projected, w);
    }
    const size_t final_norm = norm_base + 2 * layers;
    return orc_layer_norm(input, m->gain[final_norm], m->bias[final_norm], w, input);
}

/* src/common/cpu_transformer.tpp:205-224 */
static int embed_into(const orc_model* m, const uint16_t* tokens, size_t count, uint16_t* out)
{
    const size_t latent = m->g.latent, alphabet = m->g.alphabet;
    if (!count || count > m->g.books)
    {
        return orc_fail("invalid Transformer feedback shape");
    }
    for (size_t book = 0; book < count; ++book)
    {
        if (tokens[book] >= alphabet)
        {
            return orc_fail("Transformer feedback token exceeds alphabet");
        }
        const uint16_t* e = m->embeddings + (book * alphabet + tokens[book]) * latent;
        if (book == 0)
        {
            memcpy(out, e, latent * 2);
        }
        else
        {
            add_in_place(out, e, latent);
        }
    }
    return 0;
}

/* src/common/cpu_transformer.tpp:351-364 */
int orc_backend_temporal_step(orc_model* m, size_t lane, size_t position,
                              const uint16_t* feedback, size_t count, int replay)
{
    if (lane >= m->lane_count)
    {
        return orc_fail("invalid lane");
    }
    orc_lane* l = &m->lanes[lane];
    if (!(position < m->g.context && count == m->header.codebooks) ||
        position != l->temporal_position)
    {
        return orc_fail("invalid temporal step");
    }
    const size_t projection = 4 * (size_t)(m->g.temporal_layers + m->g.codebook_layers);
    if (embed_into(m, feedback, count, l->embedded) ||
        apply_linear(m, projection, l->embedded, l->conditioning) ||
        evaluate_stack(m, l, 1, l->conditioning, position,
                       m->rotations + position * (size_t)m->g.head_width, replay))
    {
        return 1;
    }
    l->temporal_position = position + 1;
    return 0;
}

/* src/common/cpu_transformer.tpp:378-419 */
int orc_backend_codebook_step(orc_model* m, size_t lane, size_t book, const uint16_t* prefix,
                              size_t count, uint16_t* distribution)
{
    if (lane >= m->lane_count)
    {
        return orc_fail("invalid lane");
    }
    orc_lane* l = &m->lanes[lane];
    const size_t w = m->g.width;
    if (!(book < m->header.codebooks && count == book) || book != l->codebook_position)
    {
        return orc_fail("invalid codebook step");
    }
    if (book == 0)
    {
        memcpy(l->input, l->conditioning, w * 2);
    }
    else
    {
        int incremental = count == l->prefix_count + 1 && l->prefix_count > 0;
        for (size_t i = 0; incremental && i < l->prefix_count; ++i)
        {
            incremental = l->prefix_tokens[i] == prefix[i];
        }
        if (incremental)
        {
            if (prefix[count - 1] >= m->g.alphabet)
            {
                return orc_fail("Transformer feedback token exceeds alphabet");
            }
            add_in_place(l->prefix,
                         m->embeddings +
                             ((book - 1) * (size_t)m->g.alphabet + prefix[count - 1]) * m->g.latent,
                         m->g.latent);
        }
        else if (embed_into(m, prefix, count, l->prefix))
        {
            return 1;
        }
        memcpy(l->prefix_tokens, prefix, count * sizeof(uint16_t));
        l->prefix_count = count;
        const size_t projection = 4 * (size_t)(m->g.temporal_layers + m->g.codebook_layers) + 1;
        if (apply_linear(m, projection, l->prefix, l->input))
        {
            return 1;
        }
    }
    add_in_place(l->input, m->positions + book * w, w);
    if (evaluate_stack(m, l, 0, l->input, book, NULL, 0))
    {
        return 1;
    }
    const size_t output = 4 * (size_t)(m->g.temporal_layers + m->g.codebook_layers) + 2;
    if (apply_linear(m, output, l->input, l->logits) ||
        orc_softmax(l->logits, m->g.alphabet, distribution))
    {
        return 1;
    }
    l->codebook_position = book + 1;
    return 0;
}

/* ---- lane worker pool (src/apple-arm/workers.cpp semantics: fork/join per call) -- */

typedef struct pool pool;
typedef int (*pool_task)(void* context, size_t index);

struct pool
{
    pthread_mutex_t mutex;
    pthread_cond_t start, done;
    pthread_t* threads;
    unsigned workers;
    unsigned generation, finished;
    int stop;
    pool_task task;
    void* context;
    size_t count;
    atomic_size_t next;
    atomic_int status;
};

static void run_items(pool* p)
{
    for (;;)
    {
        const size_t i = atomic_fetch_add(&p->next, 1);
        if (i >= p->count)
        {
            break;
        }
        if (p->task(p->context, i))
        {
            atomic_store(&p->status, 1);
        }
    }
}

static void* worker(void* argument)
{
    pool* p = argument;
    unsigned seen = 0;
    pthread_mutex_lock(&p->mutex);
    for (;;)
    {
        while (p->generation == seen && !p->stop)
        {
            pthread_cond_wait(&p->start, &p->mutex);
        }
        if (p->stop)
        {
            break;
        }
        seen = p->generation;
        pthread_mutex_unlock(&p->mutex);
        run_items(p);
        pthread_mutex_lock(&p->mutex);
        if (++p->finished == p->workers)
        {
            pthread_cond_signal(&p->done);
        }
    }
    pthread_mutex_unlock(&p->mutex);
    return NULL;
}

static pool* pool_create(unsigned threads)
{
    if (threads <= 1)
    {
        return NULL;
    }
    pool* p = orc_alloc(sizeof *p);
    pthread_mutex_init(&p->mutex, NULL);
    pthread_cond_init(&p->start, NULL);
    pthread_cond_init(&p->done, NULL);
    p->workers = threads - 1;
    p->threads = orc_alloc(p->workers * sizeof(pthread_t));
    for (unsigned i = 0; i < p->workers; ++i)
    {
        pthread_create(&p->threads[i], NULL, worker, p);
    }
    return p;
}

static int pool_run(pool* p, size_t count, pool_task task, void* context)
{
    if (!p || count <= 1)
    {
        int status = 0;
        for (size_t i = 0; i < count; ++i)
        {
            status |= task(context, i);
        }
        return status;
    }
    pthread_mutex_lock(&p->mutex);
    p->task = task;
    p->context = context;
    p->count = count;
    atomic_store(&p->next, 0);
    atomic_store(&p->status, 0);
    p->finished = 0;
    ++p->generation;
    pthread_cond_broadcast(&p->start);
    pthread_mutex_unlock(&p->mutex);
    run_items(p);
    pthread_mutex_lock(&p->mutex);
    while (p->finished != p->workers)
    {
        pthread_cond_wait(&p->done, &p->mutex);
    }
    pthread_mutex_unlock(&p->mutex);
    return atomic_load(&p->status);
}

static void pool_destroy(pool* p)
{
    if (!p)
    {
        return;
    }
    pthread_mutex_lock(&p->mutex);
    p->stop = 1;
    pthread_cond_broadcast(&p->start);
    pthread_mutex_unlock(&p->mutex);
    for (unsigned i = 0; i < p->workers; ++i)
    {
        pthread_join(p->threads[i], NULL);
    }
    pthread_mutex_destroy(&p->mutex);
    pthread_cond_destroy(&p->start);
    pthread_cond_destroy(&p->done);
    free(p->threads);
    free(p);
}

/* ---- predictor (src/common/transformer.cpp:26-245) -------------------------- */

typedef struct
{
    size_t frame, group, codebook, lane, step, token_offset;
} position_t;

typedef struct
{
    size_t completed_frames, next_book, context_used;
    uint16_t current[16];
    uint16_t* history; /* ring of replay_frames x books */
    size_t history_start, history_count;
    uint16_t* distribution;
    int prepared;
} predictor_lane;

typedef struct
{
    orc_model* model;
    orc_header header;
    predictor_lane* lanes;
    size_t count;
    size_t* ready;
    pool* workers;
    int pending;
    position_t pending_position;
} predictor;

static size_t lane_length(const orc_header* h, size_t independent)
{
    return h->frames / h->batch + (independent / h->groups < h->frames % h->batch);
}

static void predictor_free(predictor* p)
{
    for (size_t i = 0; i < p->count; ++i)
    {
        free(p->lanes[i].history);
        free(p->lanes[i].distribution);
    }
    free(p->lanes);
    free(p->ready);
    pool_destroy(p->workers);
}

static int predictor_reset(predictor* p, orc_model* m, const orc_header* h, unsigned threads)
{
    memset(p, 0, sizeof *p);
    if (orc_validate_header(h))
    {
        return 1;
    }
    if (h->method != 1)
    {
        return orc_fail("Transformer predictor requires normal framing");
    }
    p->model = m;
    p->header = *h;
    p->count = min_size(h->batch, h->frames) * h->groups;
    if (orc_backend_reset(m, h, p->count))
    {
        return 1;
    }
    p->lanes = orc_alloc((p->count ? p->count : 1) * sizeof(predictor_lane));
    p->ready = orc_alloc((p->count ? p->count : 1) * sizeof(size_t));
    for (size_t i = 0; i < p->count; ++i)
    {
        p->lanes[i].history = orc_alloc((size_t)replay_frames * h->codebooks * 2);
        p->lanes[i].distribution = orc_alloc((size_t)m->g.alphabet * 2);
    }
    p->workers = pool_create(threads);
    return 0;
}

static const uint16_t* history_at(const predictor* p, const predictor_lane* l, size_t i)
{
    return l->history + ((l->history_start + i) % replay_frames) * p->header.codebooks;
}

/* src/common/transformer.cpp:184-220 */
static int prepare(predictor* p, size_t index)
{
    predictor_lane* l = &p->lanes[index];
    orc_model* m = p->model;
    const size_t books = p->header.codebooks;
    if (l->next_book == 0)
    {
        memset(l->current, 0, sizeof l->current);
        if (l->context_used == m->g.context)
        {
            if (l->history_count != replay_frames)
            {
                return orc_fail("incomplete Transformer replay history");
            }
            if (orc_backend_reset_temporal(m, index))
            {
                return 1;
            }
            l->context_used = 0;
            for (size_t i = 0; i < l->history_count; ++i)
            {
                if (orc_backend_temporal_step(m, index, l->context_used++, history_at(p, l, i),
                                              books, 1))
                {
                    return 1;
                }
            }
        }
        else
        {
            const uint16_t* feedback =
                l->history_count ? history_at(p, l, l->history_count - 1) : l->current;
            if (orc_backend_temporal_step(m, index, l->context_used++, feedback, books, 0))
            {
                return 1;
            }
        }
        if (orc_backend_reset_codebook(m, index))
        {
            return 1;
        }
    }
    if (orc_backend_codebook_step(m, index, l->next_book, l->current, l->next_book,
                                  l->distribution))
    {
        return 1;
    }
    l->prepared = 1;
    return 0;
}

static int prepare_task(void* context, size_t i)
{
    predictor* p = context;
    return prepare(p, p->ready[i]);
}

/* src/common/transformer.cpp:120-135 */
static int lane_index(const predictor* p, const position_t* q, size_t* index)
{
    const orc_header* h = &p->header;
    const size_t base = h->frames / h->batch, extra = h->frames % h->batch;
    const size_t length = base + (q->lane < extra);
    const size_t start = q->lane * base + min_size(q->lane, extra);
    if (!(q->lane < min_size(h->batch, h->frames) && q->group < h->groups &&
          q->codebook < h->codebooks) ||
        !(q->step < length && q->frame == start + q->step &&
          q->token_offset == (q->frame * h->groups + q->group) * h->codebooks + q->codebook))
    {
        return orc_fail("inconsistent Transformer entropy position");
    }
    *index = q->lane * h->groups + q->group;
    return 0;
}

/* src/common/transformer.cpp:137-182 */
static int predict(predictor* p, const position_t* q, const uint16_t** distribution)
{
    if (p->pending)
    {
        return orc_fail("Transformer prediction needs its token committed");
    }
    size_t index = 0;
    if (lane_index(p, q, &index))
    {
        return 1;
    }
    predictor_lane* l = &p->lanes[index];
    if (!(q->step == l->completed_frames && q->codebook == l->next_book))
    {
        return orc_fail("out-of-order Transformer prediction");
    }
    if (!l->prepared)
    {
        if (p->workers)
        {
            size_t ready = 0;
            for (size_t i = 0; i < p->count; ++i)
            {
                const predictor_lane* c = &p->lanes[i];
                if (!c->prepared && c->completed_frames == q->step && c->next_book == q->codebook &&
                    q->step < lane_length(&p->header, i))
                {
                    p->ready[ready++] = i;
                }
            }
            if (pool_run(p->workers, ready, prepare_task, p))
            {
                return 1;
            }
        }
        else if (prepare(p, index))
        {
            return 1;
        }
    }
    p->pending = 1;
    p->pending_position = *q;
    *distribution = l->distribution;
    return 0;
}

/* src/common/transformer.cpp:222-244 */
static int commit(predictor* p, const position_t* q, uint16_t token)
{
    if (!p->pending || memcmp(&p->pending_position, q, sizeof *q))
    {
        return orc_fail("Transformer commit does not match prediction");
    }
    if (token >= p->model->g.alphabet)
    {
        return orc_fail("Transformer feedback token exceeds alphabet");
    }
    size_t index = 0;
    if (lane_index(p, q, &index))
    {
        return 1;
    }
    predictor_lane* l = &p->lanes[index];
    l->prepared = 0;
    l->current[q->codebook] = token;
    ++l->next_book;
    if (l->next_book == p->header.codebooks)
    {
        const size_t books = p->header.codebooks;
        if (l->history_count == replay_frames)
        {
            memcpy(l->history + l->history_start * books, l->current, books * 2);
            l->history_start = (l->history_start + 1) % replay_frames;
        }
        else
        {
            memcpy(l->history + ((l->history_start + l->history_count) % replay_frames) * books,
                   l->current, books * 2);
            ++l->history_count;
        }
        l->next_book = 0;
        ++l->completed_frames;
    }
    p->pending = 0;
    return 0;
}

/* ---- stream walks (src/format/entropy.cpp:26-155) --------------------------- */

typedef int (*symbol_visit)(void* context, predictor* p, const position_t* q);

static int visit_positions(predictor* p, symbol_visit visit, void* context, size_t max_symbols)
{
    const orc_header* h = &p->header;
    const size_t per_lane = h->frames / h->batch, extra = h->frames % h->batch;
    const size_t steps = per_lane + (extra != 0);
    const size_t lanes = min_size(h->batch, h->frames);
    size_t visited = 0;
    for (size_t step = 0; step < steps; ++step)
    {
        for (size_t book = 0; book < h->codebooks; ++book)
        {
            for (size_t lane = 0; lane < lanes; ++lane)
            {
                if (step >= per_lane + (lane < extra))
                {
                    continue;
                }
                const size_t frame = lane * per_lane + min_size(lane, extra) + step;
                for (size_t group = 0; group < h->groups; ++group)
                {
                    if (visited++ == max_symbols)
                    {
                        return 0;
                    }
                    const position_t q = {frame, group, book, lane, step,
                                          (frame * h->groups + group) * h->codebooks + book};
                    if (visit(context, p, &q))
                    {
                        return 1;
                    }
                }
            }
        }
    }
    return 0;
}

static void widen(const uint16_t* distribution, size_t n, float* out)
{
    for (size_t i = 0; i < n; ++i)
    {
        out[i] = orc_float(distribution[i]);
    }
}

typedef struct
{
    orc_encoder encoder;
    const uint16_t* tokens;
    uint32_t* bits;       /* per symbol in stream order, or NULL */
    uint64_t* positions;  /* 6 per symbol in stream order, or NULL */
    size_t visited;
    float probabilities[4096];
} pack_context;

static int pack_visit(void* context, predictor* p, const position_t* q)
{
    pack_context* c = context;
    const uint16_t* distribution;
    const size_t alphabet = p->model->g.alphabet;
    if (predict(p, q, &distribution))
    {
        return 1;
    }
    widen(distribution, alphabet, c->probabilities);
    const uint16_t token = c->tokens[q->token_offset];
    const size_t before = orc_encoder_bit_position(&c->encoder);
    if (orc_encode_categorical(&c->encoder, c->probabilities, alphabet, token))
    {
        return 1;
    }
    /* pack_normal's after_symbol(position, bits) (src/format/entropy.cpp:86-100). */
    if (c->bits)
    {
        c->bits[c->visited] = (uint32_t)(orc_encoder_bit_position(&c->encoder) - before);
    }
    if (c->positions)
    {
        uint64_t* r = c->positions + 6 * c->visited;
        r[0] = q->frame;
        r[1] = q->group;
        r[2] = q->codebook;
        r[3] = q->lane;
        r[4] = q->step;
        r[5] = q->token_offset;
    }
    ++c->visited;
    return commit(p, q, token);
}

int orc_pack_normal(orc_model* m, const orc_header* header, const uint16_t* tokens, size_t count,
                    unsigned threads, uint8_t** out, size_t* length)
{
    return orc_pack_normal_observed(m, header, tokens, count, threads, out, length, NULL, NULL);
}

int orc_pack_normal_observed(orc_model* m, const orc_header* header, const uint16_t* tokens,
                             size_t count, unsigned threads, uint8_t** out, size_t* length,
                             uint32_t* bits, uint64_t* positions)
{
    orc_header h = *header;
    h.method = 1;
    if (orc_validate_header(&h))
    {
        return 1;
    }
    if (h.frames > 0xffffffffu)
    {
        return orc_fail("normal frame count exceeds uint32");
    }
    if (count != h.frames * h.groups * h.codebooks)
    {
        return orc_fail("normal token count does not match header");
    }
    for (size_t i = 0; i < count; ++i)
    {
        if (tokens[i] >= 1024)
        {
            return orc_fail("index outside 10-bit alphabet");
        }
    }
    if (m->g.alphabet > 4096)
    {
        return orc_fail("alphabet too large");
    }
    const uint32_t crc = orc_token_crc32(tokens, count);
    pack_context* c = orc_alloc(sizeof *c);
    orc_encoder_init(&c->encoder, (size_t)512 * 1024 * 1024 - 18);
    c->tokens = tokens;
    c->bits = bits;
    c->positions = positions;
    c->visited = 0;
    predictor p;
    int status = predictor_reset(&p, m, &h, threads);
    if (!status)
    {
        status = visit_positions(&p, pack_visit, c, (size_t)-1);
    }
    if (!status)
    {
        status = orc_encoder_finish(&c->encoder);
    }
    if (!status)
    {
        const size_t n = 14 + c->encoder.size + 4;
        uint8_t* b = orc_alloc(n);
        b[0] = 'F';
        b[1] = 'B';
        b[2] = 'A';
        b[3] = 'Z';
        b[4] = 0;
        b[5] = 1;
        b[6] = (uint8_t)(h.groups | ((h.model_channels - 1) << 7));
        b[7] = h.codebooks;
        for (int i = 0; i < 4; ++i)
        {
            b[8 + i] = (uint8_t)(h.frames >> (8 * (3 - i)));
        }
        b[12] = (uint8_t)(h.batch >> 8);
        b[13] = (uint8_t)h.batch;
        memcpy(b + 14, c->encoder.bytes, c->encoder.size);
        for (int i = 0; i < 4; ++i)
        {
            b[14 + c->encoder.size + i] = (uint8_t)(crc >> (8 * (3 - i)));
        }
        *out = b;
        *length = n;
    }
    predictor_free(&p);
    free(c->encoder.bytes);
    free(c);
    return status;
}

typedef struct
{
    orc_decoder decoder;
    uint16_t* tokens;
    float probabilities[4096];
} unpack_context;

static int unpack_visit(void* context, predictor* p, const position_t* q)
{
    unpack_context* c = context;
    const uint16_t* distribution;
    const size_t alphabet = p->model->g.alphabet;
    if (predict(p, q, &distribution))
    {
        return 1;
    }
    widen(distribution, alphabet, c->probabilities);
    size_t symbol;
    if (orc_decode_categorical(&c->decoder, c->probabilities, alphabet, &symbol))
    {
        return 1;
    }
    c->tokens[q->token_offset] = (uint16_t)symbol;
    return commit(p, q, (uint16_t)symbol);
}

int orc_unpack_normal(orc_model* m, const uint8_t* bytes, size_t length, unsigned threads,
                      uint16_t** tokens, size_t* count)
{
    orc_header h;
    size_t offset, payload;
    uint32_t crc;
    if (orc_parse_header(bytes, length, &h, &offset, &payload, &crc))
    {
        return 1;
    }
    if (h.method != 1)
    {
        return orc_fail("unpack_normal requires method 1");
    }
    if (m->g.alphabet > 4096)
    {
        return orc_fail("alphabet too large");
    }
    const size_t n = h.frames * h.groups * h.codebooks;
    unpack_context* c = orc_alloc(sizeof *c);
    c->tokens = orc_alloc(n * 2);
    int status = orc_decoder_init(&c->decoder, bytes + offset, payload);
    predictor p;
    memset(&p, 0, sizeof p);
    if (!status)
    {
        status = predictor_reset(&p, m, &h, threads);
    }
    if (!status)
    {
        status = visit_positions(&p, unpack_visit, c, (size_t)-1);
    }
    if (!status && orc_token_crc32(c->tokens, n) != crc)
    {
        status = orc_fail("invalid token CRC32");
    }
    predictor_free(&p);
    if (status)
    {
        free(c->tokens);
    }
    else
    {
        *tokens = c->tokens;
        *count = n;
    }
    free(c);
    return status;
}

typedef struct
{
    const uint16_t* tokens;
    uint16_t* out;
} distribution_context;

static int distribution_visit(void* context, predictor* p, const position_t* q)
{
    distribution_context* c = context;
    const uint16_t* distribution;
    const size_t alphabet = p->model->g.alphabet;
    if (predict(p, q, &distribution))
    {
        return 1;
    }
    memcpy(c->out + q->token_offset * alphabet, distribution, alphabet * 2);
    return commit(p, q, c->tokens[q->token_offset]);
}

int orc_distributions_prefix(orc_model* m, const orc_header* header, const uint16_t* tokens,
                             size_t count, unsigned threads, size_t max_symbols, uint16_t* out)
{
    orc_header h = *header;
    h.method = 1;
    if (orc_validate_header(&h))
    {
        return 1;
    }
    if (count != h.frames * h.groups * h.codebooks)
    {
        return orc_fail("normal token count does not match header");
    }
    distribution_context c = {tokens, out};
    predictor p;
    int status = predictor_reset(&p, m, &h, threads);
    if (!status)
    {
        status = visit_positions(&p, distribution_visit, &c, max_symbols);
    }
    predictor_free(&p);
    return status;
}

int orc_distributions(orc_model* m, const orc_header* header, const uint16_t* tokens,
                      size_t count, unsigned threads, uint16_t* out)
{
    return orc_distributions_prefix(m, header, tokens, count, threads, (size_t)-1, out);
}
