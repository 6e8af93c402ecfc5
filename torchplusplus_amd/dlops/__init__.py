"""Op API mirroring torchpp.dlops (reference: torchpp/dlops/)."""
