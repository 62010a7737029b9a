// mmap_file.cpp -- whole-file read-only mapping (POSIX mmap).
#include "mmap_file.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <stdexcept>

MMapFile::MMapFile(const std::string &path)
{
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) throw std::runtime_error("cannot open " + path + ": " + std::strerror(errno));
    struct stat st;
    if (::fstat(fd, &st) != 0) {
        const int e = errno;
        ::close(fd);
        throw std::runtime_error("cannot stat " + path + ": " + std::strerror(e));
    }
    size_ = static_cast<std::size_t>(st.st_size);
    if (size_ > 0) {
        void *p = ::mmap(nullptr, size_, PROT_READ, MAP_SHARED, fd, 0);
        if (p == MAP_FAILED) {
            const int e = errno;
            ::close(fd);
            throw std::runtime_error("cannot mmap " + path + ": " + std::strerror(e));
        }
        addr_ = p;
    }
    ::close(fd);   // the mapping keeps its own reference to the file
}

MMapFile::~MMapFile()
{
    if (addr_) ::munmap(const_cast<void *>(addr_), size_);
}
