/* The Python interpreter, linked with AddressSanitizer: the sanitizer's runtime is the first
 * in the process, so its allocator and checks cover the instrumented library that pytest loads
 * through ctypes (IRON_HIP_LIB). */
#define PY_SSIZE_T_CLEAN
#include <Python.h>

int main(int argc, char** argv) { return Py_BytesMain(argc, argv); }
