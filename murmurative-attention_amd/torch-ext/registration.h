#pragma once

#include <Python.h>

// Python module init for the extension: importing the shared object runs its
// static TORCH_LIBRARY registrars, which is all the module is for.
#define MURM_STR2(x) #x
#define MURM_STR(x) MURM_STR2(x)
#define MURM_CAT2(a, b) a##b
#define MURM_CAT(a, b) MURM_CAT2(a, b)

#define REGISTER_EXTENSION(NAME)                                                  \
  PyMODINIT_FUNC MURM_CAT(PyInit_, NAME)() {                                      \
    static struct PyModuleDef def = {PyModuleDef_HEAD_INIT, MURM_STR(NAME),       \
                                     "murmurative_attention ops (MI355X)", 0,     \
                                     nullptr};                                    \
    return PyModule_Create(&def);                                                 \
  }
