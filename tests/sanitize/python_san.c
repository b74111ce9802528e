/* The Python interpreter, linked with AddressSanitizer and
 * UndefinedBehaviorSanitizer.  The sanitizer runtimes are linked into this
 * executable, so the instrumented shared libraries that the tests open with
 * ctypes (the HIP library's host code and the CPU oracle, built by this
 * directory's Makefile) find them without any preloading. */
#include <Python.h>

int main(int argc, char** argv) { return Py_BytesMain(argc, argv); }
