// r97/adjoint_family.h -- which adjoint family an op's backward belongs to: the reference's
// src/adjoint_family.h:20-55 contract. A file claims its ops with R97_REGISTER_ADJOINT_FAMILY; an
// op claimed by two different families is a hard error (std::logic_error), and an op nobody
// claimed reports None.
#pragma once

#include <initializer_list>
#include <string>

namespace r97 {

enum class AdjointFamily {
    None,
    Elementwise,
    Linear,
    Quant,
    Lora,
    Qk,
    Attention,
    GdnPrep,
    GdnKkt,
    GdnScan,
};

const char* adjoint_family_name(AdjointFamily family);
AdjointFamily family_find(const std::string& op);
void family_register(AdjointFamily family, std::initializer_list<const char*> ops);

struct FamilyRegistrar {
    FamilyRegistrar(AdjointFamily family, std::initializer_list<const char*> ops) { family_register(family, ops); }
};

#define R97_FAMILY_NAME2(a, b) a##b
#define R97_FAMILY_NAME(a, b) R97_FAMILY_NAME2(a, b)
#define R97_REGISTER_ADJOINT_FAMILY(family, ...)                                         \
    static ::r97::FamilyRegistrar R97_FAMILY_NAME(r97_reg_family_, __LINE__){ \
        ::r97::AdjointFamily::family, {__VA_ARGS__}}

}  // namespace r97
