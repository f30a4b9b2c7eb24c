// GGUF v3 reader (header, key/values, tensor infos, aligned data section) over mmap.
#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>

namespace gguf
{

namespace
{
struct Cursor
{
    const uint8_t *p, *end;
    bool ok = true;
    template <typename T> T get()
    {
        T v{};
        if ((size_t)(end - p) < sizeof(T))
        {
            ok = false;
            return v;
        }
        memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    std::string str()
    {
        uint64_t n = get<uint64_t>();
        if (!ok || (uint64_t)(end - p) < n)
        {
            ok = false;
            return {};
        }
        std::string s((const char *)p, (size_t)n);
        p += n;
        return s;
    }
};

size_t scalar_size(uint32_t t)
{
    switch (t)
    {
    case T_UINT8:
    case T_INT8:
    case T_BOOL:
        return 1;
    case T_UINT16:
    case T_INT16:
        return 2;
    case T_UINT32:
    case T_INT32:
    case T_FLOAT32:
        return 4;
    case T_UINT64:
    case T_INT64:
    case T_FLOAT64:
        return 8;
    default:
        return 0;
    }
}

void skip(Cursor &c, uint32_t t)
{
    if (t == T_STRING)
    {
        uint64_t n = c.get<uint64_t>();
        if ((uint64_t)(c.end - c.p) < n)
            c.ok = false;
        else
            c.p += n;
        return;
    }
    if (t == T_ARRAY)
    {
        uint32_t et = c.get<uint32_t>();
        uint64_t n = c.get<uint64_t>();
        size_t es = scalar_size(et);
        if (es)
        {
            if ((uint64_t)(c.end - c.p) / es < n)
                c.ok = false;
            else
                c.p += es * n;
            return;
        }
        for (uint64_t i = 0; i < n && c.ok; ++i)
            skip(c, et);
        return;
    }
    size_t s = scalar_size(t);
    if (!s || (size_t)(c.end - c.p) < s)
        c.ok = false;
    else
        c.p += s;
}
} // namespace

File::~File()
{
    if (base)
        munmap((void *)base, size);
    if (fd >= 0)
        close(fd);
}

bool File::open(const char *path, std::string *err)
{
    fd = ::open(path, O_RDONLY);
    if (fd < 0)
    {
        *err = "cannot open file";
        return false;
    }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24)
    {
        *err = "file too small";
        return false;
    }
    size = (size_t)st.st_size;
    void *m = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (m == MAP_FAILED)
    {
        *err = "mmap failed";
        return false;
    }
    base = (const uint8_t *)m;
    Cursor c{base, base + size};
    if (memcmp(base, "GGUF", 4) != 0)
    {
        *err = "bad magic";
        return false;
    }
    c.p += 4;
    version = c.get<uint32_t>();
    if (version != 3 && version != 2)
    {
        *err = "unsupported GGUF version";
        return false;
    }
    uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
    for (uint64_t i = 0; i < n_kv && c.ok; ++i)
    {
        KV kv;
        kv.key = c.str();
        kv.type = c.get<uint32_t>();
        if (kv.type == T_STRING)
            kv.str = c.str();
        else if (kv.type == T_ARRAY)
        {
            kv.arr_type = c.get<uint32_t>();
            kv.arr_len = c.get<uint64_t>();
            kv.arr_data = c.p;
            size_t es = scalar_size(kv.arr_type);
            if (es)
            {
                if ((uint64_t)(c.end - c.p) / es < kv.arr_len)
                    c.ok = false;
                else
                    c.p += es * kv.arr_len;
            }
            else
                for (uint64_t k = 0; k < kv.arr_len && c.ok; ++k)
                    skip(c, kv.arr_type);
            kv.arr_end = c.p;
        }
        else
        {
            size_t s = scalar_size(kv.type);
            if (!s || (size_t)(c.end - c.p) < s)
            {
                c.ok = false;
                break;
            }
            uint64_t raw = 0;
            memcpy(&raw, c.p, s);
            kv.u64 = raw;
            if (kv.type == T_FLOAT32)
            {
                float f;
                memcpy(&f, c.p, 4);
                kv.f64 = f;
            }
            else if (kv.type == T_FLOAT64)
                memcpy(&kv.f64, c.p, 8);
            c.p += s;
        }
        if (kv.key == "general.alignment" && kv.type == T_UINT32 && kv.u64)
            alignment = (uint32_t)kv.u64;
        kvs.push_back(std::move(kv));
    }
    for (uint64_t i = 0; i < n_tensors && c.ok; ++i)
    {
        TensorInfo t;
        t.name = c.str();
        t.n_dims = c.get<uint32_t>();
        if (t.n_dims > 4)
        {
            c.ok = false;
            break;
        }
        for (uint32_t d = 0; d < t.n_dims; ++d)
            t.ne[d] = c.get<uint64_t>();
        t.type = c.get<uint32_t>();
        t.offset = c.get<uint64_t>();
        tensors.push_back(std::move(t));
    }
    if (!c.ok)
    {
        *err = "truncated or malformed header";
        return false;
    }
    // Every size below is checked by subtraction against what remains of the file, so no sum or product wraps.
    const uint64_t header_end = (uint64_t)(c.p - base);
    if (alignment > size)
    {
        *err = "alignment larger than the file";
        return false;
    }
    const uint64_t data_start = (header_end + alignment - 1) / alignment * alignment;
    if (data_start > size && !tensors.empty())
    {
        *err = "data section starts past end of file";
        return false;
    }
    const uint64_t data_size = tensors.empty() ? 0 : size - data_start;
    for (size_t i = 0; i < tensors.size(); ++i)
    {
        TensorInfo &t = tensors[i];
        if (t.offset > data_size)
        {
            *err = "tensor offset past end of file: " + t.name;
            return false;
        }
        const uint64_t room = data_size - t.offset; // bytes from the tensor's start to the end of the file
        uint64_t n = 1;
        for (int d = 0; d < 4; ++d)
        {
            if (t.ne[d] != 0 && n > UINT64_MAX / t.ne[d])
            {
                *err = "tensor element count overflows: " + t.name;
                return false;
            }
            n *= t.ne[d];
        }
        if (t.type == GGML_F32 || t.type == GGML_F16)
        {
            const uint64_t es = t.type == GGML_F32 ? 4 : 2;
            if (n > room / es)
            {
                *err = "tensor data past end of file: " + t.name;
                return false;
            }
            t.bytes = n * es;
        }
        else
        {
            // other encodings: the span up to the next tensor (or the end of the file)
            uint64_t next = data_size;
            for (const TensorInfo &o : tensors)
                if (o.offset > t.offset && o.offset < next)
                    next = o.offset;
            t.bytes = next - t.offset;
        }
        t.data = base + data_start + t.offset;
    }
    return true;
}

const KV *File::find(const char *key) const
{
    for (const KV &kv : kvs)
        if (kv.key == key)
            return &kv;
    return nullptr;
}

std::vector<std::string> string_array(const KV &kv)
{
    std::vector<std::string> out;
    if (kv.type != T_ARRAY || kv.arr_type != T_STRING)
        return out;
    Cursor c{kv.arr_data, kv.arr_end};
    for (uint64_t i = 0; i < kv.arr_len && c.ok; ++i)
        out.push_back(c.str());
    return out;
}

std::vector<float> f32_array(const KV &kv)
{
    std::vector<float> out;
    if (kv.type == T_ARRAY && kv.arr_type == T_FLOAT32 && (size_t)(kv.arr_end - kv.arr_data) / 4 >= kv.arr_len)
    {
        out.resize(kv.arr_len);
        memcpy(out.data(), kv.arr_data, kv.arr_len * 4);
    }
    return out;
}

std::vector<int32_t> i32_array(const KV &kv)
{
    std::vector<int32_t> out;
    if (kv.type == T_ARRAY && kv.arr_type == T_INT32 && (size_t)(kv.arr_end - kv.arr_data) / 4 >= kv.arr_len)
    {
        out.resize(kv.arr_len);
        memcpy(out.data(), kv.arr_data, kv.arr_len * 4);
    }
    return out;
}

} // namespace gguf
