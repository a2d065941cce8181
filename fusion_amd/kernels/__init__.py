"""Drop-in launchers for `glm52/kernels/{add_rmsnorm,norm_router,moe_gateup,moe_down_merge,
merge_resadd,oproj_resadd,lazy_prenorm}.py`."""
