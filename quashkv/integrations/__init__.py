"""quashkv.integrations -> quashkv_amd.integrations."""
