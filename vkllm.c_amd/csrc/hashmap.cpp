// String -> u64 open-addressing map with linear probing and tombstones, used for context->stats.node_time_cost.
// Same interface as src/core/vkllm_hashmap.h:28-48 (FNV-1a hashing here).
#include <cstdlib>
#include <cstring>

#include "vkllm/vkllm_common.h"
#include "vkllm/vkllm_hashmap.h"

extern "C" uint64_t vkllm_hashmap_hash(const char *key, size_t capacity)
{
    uint64_t h = 1469598103934665603ull;
    for (const unsigned char *p = (const unsigned char *)key; *p; ++p)
        h = (h ^ *p) * 1099511628211ull;
    return capacity ? h % capacity : h;
}

extern "C" vkllm_err_t vkllm_hashmap_new(struct vkllm_hashmap **map, size_t init_capacity)
{
    if (!map)
        return VKLLM_ERR_ARGS;
    auto *m = (vkllm_hashmap *)calloc(1, sizeof(vkllm_hashmap));
    if (!m)
        return VKLLM_ERR_ALLOC;
    m->capacity = init_capacity < 8 ? 8 : init_capacity;
    m->entries = (vkllm_hashmap_entry *)calloc(m->capacity, sizeof(vkllm_hashmap_entry));
    if (!m->entries)
    {
        free(m);
        return VKLLM_ERR_ALLOC;
    }
    *map = m;
    return VKLLM_ERR_OK;
}

extern "C" void vkllm_hashmap_clear(struct vkllm_hashmap *m)
{
    if (!m)
        return;
    for (size_t i = 0; i < m->capacity; ++i)
    {
        free(m->entries[i].key);
        m->entries[i].key = nullptr;
        m->entries[i].occupied = false;
        m->entries[i].value = 0;
    }
    m->size = 0;
    m->tombstones = 0;
}

extern "C" void vkllm_hashmap_free(struct vkllm_hashmap *m)
{
    if (!m)
        return;
    vkllm_hashmap_clear(m);
    free(m->entries);
    free(m);
}

// slot holding `key`, or SIZE_MAX
static size_t find_slot(const vkllm_hashmap *m, const char *key)
{
    size_t i = vkllm_hashmap_hash(key, m->capacity);
    for (size_t n = 0; n < m->capacity; ++n, i = (i + 1) % m->capacity)
    {
        const vkllm_hashmap_entry &e = m->entries[i];
        if (!e.occupied && !e.key)
            return SIZE_MAX; // never used: end of the probe chain
        if (e.occupied && strcmp(e.key, key) == 0)
            return i;
    }
    return SIZE_MAX;
}

extern "C" vkllm_err_t vkllm_hashmap_resize(struct vkllm_hashmap *m, size_t new_capacity)
{
    if (!m || new_capacity < m->size + 1)
        return VKLLM_ERR_ARGS;
    vkllm_hashmap_entry *old = m->entries;
    size_t old_cap = m->capacity;
    m->entries = (vkllm_hashmap_entry *)calloc(new_capacity, sizeof(vkllm_hashmap_entry));
    if (!m->entries)
    {
        m->entries = old;
        return VKLLM_ERR_ALLOC;
    }
    m->capacity = new_capacity;
    m->size = 0;
    m->tombstones = 0;
    for (size_t i = 0; i < old_cap; ++i)
    {
        if (old[i].occupied)
        {
            size_t j = vkllm_hashmap_hash(old[i].key, m->capacity);
            while (m->entries[j].occupied)
                j = (j + 1) % m->capacity;
            m->entries[j] = old[i];
            m->size++;
        }
        else
            free(old[i].key);
    }
    free(old);
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_hashmap_insert(struct vkllm_hashmap *m, const char *key, uint64_t value)
{
    if (!m || !key)
        return VKLLM_ERR_ARGS;
    size_t s = find_slot(m, key);
    if (s != SIZE_MAX)
    {
        m->entries[s].value = value;
        return VKLLM_ERR_OK;
    }
    if ((m->size + m->tombstones + 1) * 4 > m->capacity * 3)
    {
        vkllm_err_t rc = vkllm_hashmap_resize(m, m->capacity * 2);
        if (rc != VKLLM_ERR_OK)
            return rc;
    }
    size_t i = vkllm_hashmap_hash(key, m->capacity);
    while (m->entries[i].occupied)
        i = (i + 1) % m->capacity;
    vkllm_hashmap_entry &e = m->entries[i];
    if (e.key) // reusing a tombstone
    {
        free(e.key);
        m->tombstones--;
    }
    e.key = strdup(key);
    if (!e.key)
        return VKLLM_ERR_ALLOC;
    e.value = value;
    e.occupied = true;
    m->size++;
    return VKLLM_ERR_OK;
}

extern "C" bool vkllm_hashmap_get(const struct vkllm_hashmap *m, const char *key, uint64_t *out_value)
{
    if (!m || !key)
        return false;
    size_t s = find_slot(m, key);
    if (s == SIZE_MAX)
        return false;
    if (out_value)
        *out_value = m->entries[s].value;
    return true;
}

extern "C" bool vkllm_hashmap_contains(const struct vkllm_hashmap *m, const char *key)
{
    return vkllm_hashmap_get(m, key, nullptr);
}

extern "C" vkllm_err_t vkllm_hashmap_remove(struct vkllm_hashmap *m, const char *key)
{
    if (!m || !key)
        return VKLLM_ERR_ARGS;
    size_t s = find_slot(m, key);
    if (s == SIZE_MAX)
        return VKLLM_ERR_ARGS;
    m->entries[s].occupied = false; // key kept as the tombstone marker
    m->size--;
    m->tombstones++;
    return VKLLM_ERR_OK;
}

extern "C" size_t vkllm_hashmap_size(const struct vkllm_hashmap *m)
{
    return m ? m->size : 0;
}

extern "C" bool vkllm_hashmap_empty(const struct vkllm_hashmap *m)
{
    return !m || m->size == 0;
}
