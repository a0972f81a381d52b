// backend-hip: the FFM binding of libjmodels_attn (include/jmodels_attn.h) and backend-java's
// AttentionKernel on it. Like backend-native, it needs --enable-native-access at run time and the
// library path in -Dmodels.hip.attention.library (or MODELS_HIP_ATTENTION_LIBRARY).
plugins {
    `java-library`
}

java {
    toolchain {
        languageVersion.set(JavaLanguageVersion.of(25))
    }
}

dependencies {
    api(project(":backend-java"))
    api(project(":models-api"))
}

tasks.withType<Test>().configureEach {
    jvmArgs("--enable-native-access=ALL-UNNAMED")
    systemProperty("models.hip.attention.library",
        System.getProperty("models.hip.attention.library") ?: "")
}
