#pragma once
#include <cstddef>
#include <string>

/**
 * Read-only mapping of a whole file (the reference's MMapFile,
 * xstar_cpp/include/mmap_file.h): the constructor maps the file, the destructor
 * unmaps it.  Tensor views built by make_weight_view point into the mapping, so
 * it is neither copyable nor movable.  Throws std::runtime_error when the file
 * cannot be opened or mapped.
 */
class MMapFile
{
public:
    explicit MMapFile(const std::string &path);
    ~MMapFile();
    MMapFile(const MMapFile &) = delete;
    MMapFile &operator=(const MMapFile &) = delete;

    const void *addr() const { return addr_; }
    std::size_t size() const { return size_; }

private:
    const void *addr_ = nullptr;
    std::size_t size_ = 0;
};
