{
  "targets": [
    {
      "target_name": "tlm_addon",
      "sources": ["tlm_addon.cc"],
      "include_dirs": ["../include"],
      "cflags_cc": ["-std=c++17", "-O2"],
      "libraries": ["-ldl"]
    }
  ]
}
