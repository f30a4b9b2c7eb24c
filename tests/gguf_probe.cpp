// Test driver for the library's GGUF reader (vkllm.c_amd/csrc/gguf.cpp), built on the CPU with AddressSanitizer and
// UndefinedBehaviorSanitizer by tests/test_gguf_reader.py. For each file named on the command line it prints one
// line: "ERR <reason>" when the reader rejects the file, else "OK <n_kv> <n_tensors>" followed by one line per tensor
// "T <name> <ne0> <ne1> <ne2> <ne3> <type> <offset> <bytes> <sum of its bytes>" (the sum touches every byte the
// reader hands out, so a span past the mapping is a sanitizer report, not a silent success), and for every string
// array key "S <key> <count> <total length>".
#include <cstdio>
#include <string>

#include "gguf.h"

int main(int argc, char **argv)
{
    for (int i = 1; i < argc; ++i)
    {
        gguf::File f;
        std::string err;
        if (!f.open(argv[i], &err))
        {
            printf("ERR %s\n", err.c_str());
            continue;
        }
        printf("OK %zu %zu\n", f.kvs.size(), f.tensors.size());
        for (const gguf::TensorInfo &t : f.tensors)
        {
            unsigned long long sum = 0;
            for (uint64_t k = 0; k < t.bytes; ++k)
                sum += t.data[k];
            printf("T %s %llu %llu %llu %llu %u %llu %llu %llu\n", t.name.c_str(), (unsigned long long)t.ne[0],
                   (unsigned long long)t.ne[1], (unsigned long long)t.ne[2], (unsigned long long)t.ne[3], t.type,
                   (unsigned long long)t.offset, (unsigned long long)t.bytes, sum);
        }
        for (const gguf::KV &kv : f.kvs)
            if (kv.type == gguf::T_ARRAY && kv.arr_type == gguf::T_STRING)
            {
                size_t total = 0;
                const std::vector<std::string> s = gguf::string_array(kv);
                for (const std::string &x : s)
                    total += x.size();
                printf("S %s %zu %zu\n", kv.key.c_str(), s.size(), total);
            }
    }
    return 0;
}
